"""Pins the oracle's Transformer-SSRU composition (the reference's own graph).

The SSRU op and the static-multiplier linear are pinned by the reference's
KATs (test_oracle.py).  These tests pin how oracle_translate_ssru wires them
(crates/marian-cpu/src/q8_engine.rs:511-558 encoder with separate Q/K/V
layers, :382-451 the SSRU decoder loop, :749-790 scoring over candidates):

1. A closed form.  With every dense weight zero except the SSRU candidate
   layer W, each other layer returns its bias: the encoder is
   x1 = LN(bo + x), x = LN(b2 + x1), and a decoder layer is
   s = g s + (1 - g) (W x) with g = 1 / (1 + exp(-bf)),
   x1 = LN(relu(s) + x), x2 = LN(bo + x1), x = LN(b2 + x2).
   Float64, positions and sqrt(d) included, against the oracle's encoder
   states, tokens and logits.
2. An independent float64 model (tests/fp64_model.py, Fp64SsruModel) with
   random weights and per-layer multipliers agrees within a small tolerance;
   each planted mistake (inverted gate, state not carried, missing ReLU or
   residual, wrong query source, K/V multipliers swapped, static output
   multiplier replaced by a dynamic one, ...) moves it far outside.
"""

import copy
import importlib

import numpy as np
import pytest

import fp64_model as F

GEOM = dict(source_vocab=300, target_vocab=280, dim=128, heads=2, ffn_dim=256,
            encoder_layers=2, decoder_layers=2)


@pytest.fixture(scope="module")
def syn(pkg):
    return importlib.import_module(pkg.__name__ + ".synthetic")


@pytest.fixture(scope="module")
def sl(pkg):
    return importlib.import_module(pkg.__name__ + ".shortlist")


def batch(n=5, seed=17, vocab=300):
    rng = np.random.default_rng(seed)
    lens = rng.integers(3, 14, size=n)
    seqs = [rng.integers(3, vocab, size=int(L)).astype(np.int32) for L in lens]
    offs = np.zeros(n + 1, np.uint32)
    offs[1:] = np.cumsum(lens)
    return np.concatenate(seqs), offs


def shortlist_for(sl, toks, offs, Vs, Vt, seed=3):
    """A random lexical shortlist (8 targets per source id, first 20 ids
    always allowed) and the candidate lists of the batch's sentences."""
    rng = np.random.default_rng(seed)
    targets = rng.integers(0, Vt, size=8 * Vs).astype(np.uint32)
    offsets = np.arange(Vs + 1, dtype=np.uint64) * 8
    s = sl.LexicalShortlist.from_bytes(sl.LexicalShortlist.to_bytes(20, offsets, targets), Vs, Vt)
    lists = [s.candidates(toks[offs[b]:offs[b + 1]]) for b in range(len(offs) - 1)]
    return sl.pack_candidates(lists)


def ln64(z, p):
    mean = z.mean(-1, keepdims=True)
    var = ((z - mean) ** 2).mean(-1, keepdims=True)
    return (z - mean) / np.sqrt(var + 1e-6) * p["scale"].astype(np.float64) + p["bias"].astype(np.float64)


def b64(lin):
    return lin["bias"].astype(np.float64)


@pytest.fixture(scope="module")
def zmodel(syn):
    m = syn.seeded_ssru_model(seed=9, geometry=syn.SsruGeometry(**GEOM), std=0.3)
    z = copy.deepcopy(m)
    for L in z.encoder + z.decoder:
        for name, part in L.items():
            if "weight" in part and name != "ssru_w":
                part["weight"][:] = 0
    return z


def closed_form_encoder(m, toks, offs):
    d = m.geometry.dim
    pos = F.positions(d, 4096)
    p = np.concatenate([np.arange(offs[i + 1] - offs[i]) for i in range(len(offs) - 1)])
    x = m.encoder_embedding[toks].astype(np.float64) / np.float64(m.encoder_embedding_mult)
    x = x * np.sqrt(d) + pos[p]
    for L in m.encoder:
        x1 = ln64(b64(L["wo"]) + x, L["attn_ln"])
        x = ln64(b64(L["w2"]) + x1, L["ffn_ln"])
    return x


def closed_form_decode(m, steps, flags=1):
    """Tokens and per-step logits of the zero-weight model (they do not depend
    on the source: cross-attention returns the value bias)."""
    d = m.geometry.dim
    pos = F.positions(d, 4096)
    scorer = F.Fp64SsruModel(m)
    state = [np.zeros(d) for _ in m.decoder]
    prev, toks, lgs = -1, [], []
    for t in range(steps):
        x = pos[t].copy()
        if prev >= 0:
            x += m.decoder_embedding[prev].astype(np.float64) / np.float64(m.decoder_embedding_mult) * np.sqrt(d)
        for i, L in enumerate(m.decoder):
            c = F.slinear(x[None, :], L["ssru_w"])[0]
            g = 1.0 / (1.0 + np.exp(-b64(L["ssru_wf"])))
            state[i] = g * state[i] + (1.0 - g) * c
            x1 = ln64(np.maximum(state[i], 0.0) + x, L["ssru_ln"])
            x2 = ln64(b64(L["wo"]) + x1, L["context_ln"])
            x = ln64(b64(L["w2"]) + x2, L["ffn_ln"])
        lg = scorer.logits(x, flags)
        prev = int(np.argmax(lg))
        toks.append(prev)
        lgs.append(lg)
    return toks, lgs


def test_zero_weight_closed_form(pkg, orc, zmodel):
    toks, offs = batch()
    steps = 9
    om = orc.OracleSsruModel(zmodel)
    rows, enc, lg, act = orc.translate_ssru(om, toks, offs, [steps] * 5, pkg.LIFTED_LIMITS,
                                            flags=1, probe_step=steps - 1)
    want = closed_form_encoder(zmodel, toks, offs)
    e_enc = np.abs(enc - want).max()
    want_toks, want_lg = closed_form_decode(zmodel, steps)
    live = np.isfinite(want_lg[-1])
    rel = np.abs(lg[0][live] - want_lg[-1][live]) / np.maximum(np.abs(want_lg[-1][live]), 1e-3)
    print(f"zero-weight SSRU model: encoder {e_enc:.2e}, logits rel {rel.max():.2e}, "
          f"tokens {want_toks}")
    assert e_enc < 2e-5
    assert all(r == want_toks for r in rows)
    assert np.array_equal(np.isfinite(lg[0]), live) and rel.max() < 1e-5
    moved = np.abs(want_lg[-1][live] - want_lg[0][live]).max()
    assert moved > 1e-2, "the recurrent state should change the logits between steps"


@pytest.fixture(scope="module")
def rmodel(syn):
    return syn.seeded_ssru_model(seed=12, geometry=syn.SsruGeometry(**GEOM), std=0.1,
                                 shared_input_mults=False)


@pytest.fixture(scope="module")
def oracle_runs(pkg, orc, sl, rmodel):
    toks, offs = batch(n=4, seed=23)
    om = orc.OracleSsruModel(rmodel)
    g = rmodel.geometry
    cand, coff, _ = shortlist_for(sl, toks, offs, g.source_vocab, g.target_vocab)
    runs = {}
    for name, c, co in (("full", None, None), ("shortlist", cand, coff)):
        rows, enc, lg, act = orc.translate_ssru(om, toks, offs, [6] * 4, pkg.LIFTED_LIMITS,
                                                flags=1, candidates=c, candidate_offsets=co,
                                                probe_step=3)
        runs[name] = (enc, rows, lg, c, co)
    return toks, offs, runs


def fp64_run(model, toks, offs, cand, coff, mistake=None):
    fm = F.Fp64SsruModel(model, mistake)
    enc = fm.encode(toks, offs)
    rows, lgs = [], []
    for b in range(len(offs) - 1):
        sl_ = slice(int(offs[b]), int(offs[b + 1]))
        c = None if cand is None else cand[coff[b]:coff[b + 1]]
        r, lg = fm.decode(enc[sl_], toks[sl_], 6, flags=1, candidates=c, probe_step=3)
        rows.append(r)
        lgs.append(lg)
    return enc, rows, np.stack(lgs)


ENC_TOL = 1e-4    # encoder states are O(1) after LayerNorm
LOGIT_TOL = 1e-4  # relative, on the scored logits


def distance(run, fp):
    enc, rows, lg = run[0], run[1], run[2]
    e_enc = float(np.abs(fp[0] - enc).max())
    live = np.isfinite(lg)
    assert np.array_equal(live, np.isfinite(fp[2])), "scored ids differ"
    e_lg = float((np.abs(fp[2][live] - lg[live]) / np.maximum(np.abs(lg[live]), 1e-2)).max())
    return e_enc, e_lg, fp[1] == rows


@pytest.mark.parametrize("scoring", ["full", "shortlist"])
def test_fp64_ssru_model_agrees_with_oracle(rmodel, oracle_runs, scoring):
    toks, offs, runs = oracle_runs
    run = runs[scoring]
    e_enc, e_lg, same = distance(run, fp64_run(rmodel, toks, offs, run[3], run[4]))
    print(f"{scoring}: encoder {e_enc:.2e}, logits {e_lg:.2e}, tokens same {same}")
    assert e_enc < ENC_TOL and e_lg < LOGIT_TOL and same


@pytest.mark.parametrize("mistake", F.SSRU_MISTAKES)
def test_planted_ssru_mistake_is_caught(rmodel, oracle_runs, mistake):
    toks, offs, runs = oracle_runs
    run = runs["shortlist"]
    fp = fp64_run(rmodel, toks, offs, run[3], run[4], mistake)
    e_enc = float(np.abs(fp[0] - run[0]).max())
    live = np.isfinite(run[2])
    e_lg = float((np.abs(fp[2][live] - run[2][live]) / np.maximum(np.abs(run[2][live]), 1e-2)).max())
    print(f"{mistake}: encoder {e_enc:.2e}, logits {e_lg:.2e}")
    assert e_enc > 100 * ENC_TOL or e_lg > 100 * LOGIT_TOL


def test_candidate_and_input_errors(pkg, orc, rmodel):
    om = orc.OracleSsruModel(rmodel)
    toks, offs = batch(n=2, seed=5)
    with pytest.raises(orc.OracleError):  # empty candidate list
        orc.translate_ssru(om, toks, offs, [3, 3], pkg.LIFTED_LIMITS, candidates=[0, 5],
                           candidate_offsets=[0, 2, 2])
    with pytest.raises(orc.OracleError):  # id outside the target vocabulary
        orc.translate_ssru(om, toks, offs, [3, 3], pkg.LIFTED_LIMITS, candidates=[0, 280],
                           candidate_offsets=[0, 1, 2])
    bad = toks.copy()
    bad[0] = rmodel.geometry.source_vocab  # source id checked against the source vocabulary
    with pytest.raises(orc.OracleError):
        orc.translate_ssru(om, bad, offs, [3, 3], pkg.LIFTED_LIMITS)


@pytest.mark.parametrize("scoring", ["full", "shortlist"])
@pytest.mark.parametrize("flags", [0, 1])
def test_reference_schedule_gives_the_same_tokens(pkg, orc, sl, rmodel, scoring, flags):
    """The padded, all-rows schedule (the timed CPU baseline: keys masked by
    length, finished rows still decoded, u8 AVX2 GEMMs) against the
    per-sentence restatement, with end-of-sentence stops on and off.  With
    stops on, the EOS id's bias is raised so that two sentences end at their
    first token while the others run to their limits."""
    m = rmodel
    if flags == 0:
        m = copy.deepcopy(rmodel)
        m.output_bias[0] += 1.5
    om = orc.OracleSsruModel(m)
    toks, offs = batch(n=7, seed=31)
    g = rmodel.geometry
    cand = coff = None
    if scoring == "shortlist":
        cand, coff, _ = shortlist_for(sl, toks, offs, g.source_vocab, g.target_vocab, seed=8)
    req = np.array([9, 3, 12, 1, 7, 12, 5], np.uint32)
    ragged = orc.translate_ssru(om, toks, offs, req, pkg.LIFTED_LIMITS, flags=flags,
                                candidates=cand, candidate_offsets=coff)
    padded = orc.translate_ssru(om, toks, offs, req, pkg.LIFTED_LIMITS, flags=flags,
                                candidates=cand, candidate_offsets=coff, threads=4,
                                schedule="reference")
    print(f"{scoring}, flags {flags}: lengths {[len(r) for r in ragged]}")
    assert padded == ragged
    stopped = [len(r) < int(n) and r[-1] == 0 for r, n in zip(ragged, req)]
    assert any(stopped) == (flags == 0) and not all(stopped)
    with pytest.raises(ValueError):
        orc.translate_ssru(om, toks, offs, req, pkg.LIFTED_LIMITS, schedule="reference", probe_step=1)
