"""Lexical shortlist candidates (host side) and candidate scoring in the oracle.

The shortlist tests follow the reference's own (crates/marian-model/src/
shortlist.rs:261-291): the full vocabulary masks the control ids, a shortlist
must supply EOS, the entry count is bounded; plus the candidate rules of
:150-198 (firstNum, union over the source tokens, the generation mask, padding
to a multiple of 8 with the lowest absent ids from 50).  The oracle's
candidate scoring is pinned against its full-vocabulary scoring restricted to
the candidates and an int64 closed form.
"""

import importlib

import numpy as np
import pytest


@pytest.fixture(scope="module")
def sl(pkg):
    return importlib.import_module(pkg.__name__ + ".shortlist")


def test_full_vocabulary_masks_control_tokens(sl):
    c = sl.LexicalShortlist.from_bytes(None, 64, 64).candidates([0, 63])
    assert 1 not in c and not any(i in c for i in range(7, 39))
    assert 0 in c and 63 in c
    assert np.all(np.diff(c.astype(np.int64)) > 0)


def test_shortlist_must_supply_eos(sl):
    data = sl.LexicalShortlist.to_bytes(0, [0, 1], [2])
    s = sl.LexicalShortlist.from_bytes(data, 1, 64)
    with pytest.raises(sl.ShortlistError, match="EOS"):
        s.candidates([0])


def test_shortlist_entry_count_is_bounded(sl):
    data = bytearray(sl.LexicalShortlist.to_bytes(0, [0, 0], []))
    data[40:48] = (sl.MAX_TARGET_ENTRIES + 1).to_bytes(8, "little")
    with pytest.raises(sl.ShortlistError):
        sl.LexicalShortlist.from_bytes(bytes(data), 1, 64)


def test_candidate_rules(sl):
    # source vocab 4: token 0 -> {5, 60}, token 1 -> {2, 9, 61}, token 3 -> {70}
    data = sl.LexicalShortlist.to_bytes(3, [0, 2, 5, 5, 6], [5, 60, 2, 9, 61, 70])
    s = sl.LexicalShortlist.from_bytes(data, 4, 100)
    c = s.candidates([1, 0])
    # firstNum 3 gives 0, 1, 2 (1 masked); 9 is masked; union {0,2,5,60,61}: 5 ids,
    # padded with the absent ids 50, 51, 52 to 8
    assert c.tolist() == [0, 2, 5, 50, 51, 52, 60, 61]
    assert len(s.candidates([3])) % 8 == 0
    with pytest.raises(sl.ShortlistError):
        s.candidates([4])
    with pytest.raises(sl.ShortlistError):
        sl.LexicalShortlist.from_bytes(data[:-4], 4, 100)
    bad = sl.LexicalShortlist.to_bytes(0, [0, 1, 1, 1, 1], [100])
    with pytest.raises(sl.ShortlistError, match="exceeds"):
        sl.LexicalShortlist.from_bytes(bad, 4, 100)


def test_oracle_candidate_scoring(orc, sl):
    rng = np.random.default_rng(4)
    V, K, M = 700, 128, 3
    emb = rng.integers(-127, 128, size=(V, K)).astype(np.int8)
    emb[301] = emb[300]  # equal rows: the first candidate of the two wins
    mult = rng.uniform(50, 500, size=V).astype(np.float32)
    mult[301] = mult[300]
    bias = (rng.standard_normal(V) * 0.1).astype(np.float32)
    bias[301] = bias[300]
    xq = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    xa = rng.uniform(1, 40, size=M).astype(np.float32)
    lists = [np.sort(rng.choice(V, size=n, replace=False)).astype(np.uint32) for n in (40, 8, 200)]
    lists[1] = np.array([0, 5, 299, 300, 301, 302, 400, 699], np.uint32)
    flat, offs, _ = sl.pack_candidates(lists)
    tok, lg = orc.candidate_argmax(xq, xa, emb, mult, bias, flat, offs)
    for m, c in enumerate(lists):
        acc = xq[m].astype(np.int64) @ emb[c].astype(np.int64).T
        inv = (np.float32(1) / (xa[m] * mult[c])).astype(np.float32)
        want = acc.astype(np.float32) * inv + bias[c]
        assert np.array_equal(lg[offs[m]:offs[m + 1]], want)
        assert tok[m] == c[int(np.argmax(want))]
    # force the tie: row 1's best is the duplicated pair
    xq2 = xq.copy()
    xq2[1] = np.clip(emb[300].astype(np.int64), -127, 127).astype(np.int8)
    bias2 = bias.copy()
    bias2[[300, 301]] = 100.0
    tok2, _ = orc.candidate_argmax(xq2, xa, emb, mult, bias2, flat, offs)
    assert tok2[1] == 300
    with pytest.raises(orc.OracleError):
        orc.candidate_argmax(xq, xa, emb, mult, bias, np.array([V], np.uint32),
                             np.array([0, 1], np.uint32))


def _unmasked(V):
    ids = np.arange(V, dtype=np.uint32)
    return ids[(ids != 1) & ((ids < 7) | (ids > 38))]


def test_oracle_translate_with_the_full_list_equals_masked_vocabulary(pkg, orc, sl):
    """No shortlist (from_bytes(None)) gives every unmasked id ascending:
    scoring that list must reproduce full-vocabulary scoring with the mask,
    in both graphs."""
    g = pkg.Geometry(vocab=400, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    m = pkg.seeded_model(seed=21, geometry=g, std=0.3)
    b = pkg.ragged_batch(seed=2, n=4, vocab=400)
    lim = np.minimum(b.max_output_tokens, 12)
    full = sl.LexicalShortlist.from_bytes(None, 400, 400).candidates([3])
    assert np.array_equal(full, _unmasked(400))
    flat, offs, _ = sl.pack_candidates([full] * 4)
    om = orc.OracleModel(m)
    assert orc.translate_shortlisted(om, b.tokens, b.offsets, lim, b.limits, flat, offs) == \
        orc.translate(om, b.tokens, b.offsets, lim, b.limits)
    syn = importlib.import_module(pkg.__name__ + ".synthetic")
    sg = syn.SsruGeometry(source_vocab=400, target_vocab=400, dim=128, heads=2, ffn_dim=256,
                          encoder_layers=1, decoder_layers=1)
    sm = orc.OracleSsruModel(syn.seeded_ssru_model(seed=22, geometry=sg, std=0.1))
    assert orc.translate_ssru(sm, b.tokens, b.offsets, lim, b.limits, candidates=flat,
                              candidate_offsets=offs) == \
        orc.translate_ssru(sm, b.tokens, b.offsets, lim, b.limits)


def test_oracle_translate_scores_only_the_candidates(pkg, orc, sl):
    """A narrow list: every generated id is on the row's list, and a list that
    is one id long makes the row emit that id at every step."""
    g = pkg.Geometry(vocab=400, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    om = orc.OracleModel(pkg.seeded_model(seed=21, geometry=g, std=0.3))
    b = pkg.ragged_batch(seed=2, n=3, vocab=400)
    lists = [np.array([0, 50, 51, 300], np.uint32), np.array([77], np.uint32),
             np.array([0, 2, 3, 4, 5, 6, 39], np.uint32)]
    flat, offs, _ = sl.pack_candidates(lists)
    rows = orc.translate_shortlisted(om, b.tokens, b.offsets, [10] * 3, b.limits, flat, offs,
                                     flags=pkg.FLAG_IGNORE_EOS)
    for r, c in zip(rows, lists):
        assert set(r) <= set(c.tolist())
    assert rows[1] == [77] * 10
