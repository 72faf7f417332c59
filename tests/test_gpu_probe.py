"""GPU parity below the token level: encoder states and logits, bit for bit.

marian_hip_translate_probe copies out the engine's final encoder states and the
logits of one decode step; oracle.translate_probe computes the same on the CPU.
Both are compared bit-exactly (the kernels follow the reference's fp32
operation order), which also pins the fused decode kernels that tokens alone
exercise only indirectly: the attention blocks with their LayerNorm and
embedding prologues, the LayerNorm + FFN up-projection block, the FFN
down-projection that quantizes its fp32 input, the attention-output
projection with its 16-row groups, and the vocabulary kernel with and without
its LayerNorm prologue.  The cases straddle every row and key threshold at
which the engine switches kernels: 1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64 and
65 active rows; 128, 129 and 201 cached keys; 128, 129, 300, 512 and 513
source tokens (one wave per (row, head) up to 128 keys, eight waves up to
512, 64-key chunks past that), at head widths 64 and 48.

Limits are capped at probe_step + 1 on both sides: a row is active at the
probed step, and its logits there are the same, whatever happens afterwards.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


def probe_both(pkg, orc, engine, oracle_model, toks, offs, limits, flags, step, lim_cfg):
    lim = np.minimum(np.asarray(limits, np.int64), step + 1).astype(np.uint32)
    out, enc, lg, act = engine.translate_probe(toks, offs, lim, flags, probe_step=step)
    rows, enc_o, lg_o, act_o = orc.translate_probe(oracle_model, toks, offs, lim, lim_cfg, flags,
                                                   probe_step=step, threads=ORACLE_THREADS)
    plain = engine.translate_token_ids(toks, offs, lim, flags).rows()
    return out.rows(), enc, lg, act, rows, enc_o, lg_o, act_o, plain


def check(label, res):
    got, enc, lg, act, want, enc_o, lg_o, act_o, plain = res
    n_act = int(act.sum())
    print(f"{label}: {n_act} active rows at the probed step", flush=True)
    assert got == plain, "the probe changed the tokens"
    assert got == want, "tokens differ from the oracle"
    assert np.array_equal(act, act_o), "active rows differ"
    assert np.array_equal(enc.view(np.uint32), enc_o.view(np.uint32)), \
        f"encoder states differ (max |d| {np.abs(enc - enc_o).max():.3e})"
    a = act_o
    assert np.array_equal(lg[a].view(np.uint32), lg_o[a].view(np.uint32)), \
        f"logits differ (max |d| {np.nanmax(np.abs(lg[a] - lg_o[a])):.3e})"
    return n_act


def sentences(rng, n, lo, hi, vocab):
    lens = rng.integers(lo, hi + 1, size=n)
    seqs = [rng.integers(3, vocab, size=int(L)).astype(np.int32) for L in lens]
    offs = np.zeros(n + 1, np.uint32)
    offs[1:] = np.cumsum(lens)
    return np.concatenate(seqs), offs


@pytest.fixture(scope="module")
def small(pkg, orc, small_model):
    with pkg.HipEngine(small_model, limits=pkg.LIFTED_LIMITS) as e:
        yield e, orc.OracleModel(small_model), small_model.geometry.vocab


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64, 65])
def test_probe_row_thresholds(pkg, orc, small, rows):
    engine, om, V = small
    rng = np.random.default_rng(100 + rows)
    toks, offs = sentences(rng, rows, 5, 40, V)
    res = probe_both(pkg, orc, engine, om, toks, offs, [8] * rows, pkg.FLAG_IGNORE_EOS, 3,
                     pkg.LIFTED_LIMITS)
    assert check(f"rows={rows}", res) == rows


@pytest.mark.parametrize("step", [127, 128, 200])
def test_probe_self_key_threshold(pkg, orc, small, step):
    engine, om, V = small
    rng = np.random.default_rng(7)
    toks, offs = sentences(rng, 2, 10, 30, V)
    res = probe_both(pkg, orc, engine, om, toks, offs, [step + 1, step + 1], pkg.FLAG_IGNORE_EOS, step,
                     pkg.LIFTED_LIMITS)
    assert check(f"self keys={step + 1}", res) == 2


@pytest.mark.parametrize("src_len", [128, 129, 300, 512, 513])
def test_probe_cross_key_threshold(pkg, orc, small, src_len):
    engine, om, V = small
    rng = np.random.default_rng(src_len)
    toks, offs = sentences(rng, 3, 20, 60, V)
    long = rng.integers(3, V, size=src_len).astype(np.int32)
    toks = np.concatenate([toks, long])
    offs = np.append(offs, offs[-1] + src_len).astype(np.uint32)
    res = probe_both(pkg, orc, engine, om, toks, offs, [6] * 4, pkg.FLAG_IGNORE_EOS, 2,
                     pkg.LIFTED_LIMITS)
    assert check(f"source tokens={src_len}", res) == 4


@pytest.mark.parametrize("src_len, step", [(129, 2), (300, 2), (512, 2), (40, 150)])
def test_probe_long_keys_head_width_48(pkg, orc, src_len, step):
    """Eight heads of width 48 (d = 384): cross-attention over long sources and
    self-attention past 128 cached keys."""
    g = pkg.Geometry(vocab=3000, encoder_layers=1, decoder_layers=2, dim=384, heads=8, ffn_dim=768)
    model = pkg.seeded_model(seed=23, geometry=g)
    om = orc.OracleModel(model)
    rng = np.random.default_rng(src_len + step)
    toks, offs = sentences(rng, 3, 5, 30, g.vocab)
    long = rng.integers(3, g.vocab, size=src_len).astype(np.int32)
    toks = np.concatenate([toks, long])
    offs = np.append(offs, offs[-1] + src_len).astype(np.uint32)
    with pkg.HipEngine(model, limits=pkg.LIFTED_LIMITS) as e:
        res = probe_both(pkg, orc, e, om, toks, offs, [step + 1] * 4, pkg.FLAG_IGNORE_EOS, step,
                         pkg.LIFTED_LIMITS)
        assert check(f"head width 48, source tokens={src_len}, step {step}", res) == 4


def test_probe_without_generation_mask(pkg, orc, small):
    engine, om, V = small
    rng = np.random.default_rng(5)
    toks, offs = sentences(rng, 5, 5, 20, V)
    flags = pkg.FLAG_IGNORE_EOS | pkg.FLAG_NO_GENERATION_MASK
    res = probe_both(pkg, orc, engine, om, toks, offs, [4] * 5, flags, 1, pkg.LIFTED_LIMITS)
    check("no generation mask", res)
    assert np.all(np.isfinite(res[2][res[3]]))


@pytest.fixture(scope="module")
def full(pkg, orc, full_model):
    with pkg.HipEngine(full_model, limits=pkg.LIFTED_LIMITS) as e:
        yield e, orc.OracleModel(full_model)


@pytest.mark.parametrize("step", [0, 15, 31])
def test_probe_single_sentence(pkg, orc, full, step):
    engine, om = full
    b = pkg.single_sentence_batch()
    res = probe_both(pkg, orc, engine, om, b.tokens, b.offsets, b.max_output_tokens, b.flags, step,
                     b.limits)
    assert check(f"single sentence, step {step}", res) == 1


@pytest.mark.parametrize("step", [4, 40, 100])
def test_probe_ragged_64(pkg, orc, full, step):
    engine, om = full
    b = pkg.ragged_batch()
    res = probe_both(pkg, orc, engine, om, b.tokens, b.offsets, b.max_output_tokens, b.flags, step,
                     b.limits)
    check(f"ragged-64, step {step}", res)


def test_vocabulary_over_32768_ids_token_exact(pkg, orc):
    """A 40000-id vocabulary: 313 argmax partials per row, more than the
    finalizer's first pass of 4 x 64 per lane requests.  260 sentences, so the
    steps run every finalizer (the workgroup scan above 64 rows, over several
    64-row passes above 256, one wave per 8 rows up to 64, the 4- and 8-row
    single waves); tokens and one step's logits against the oracle."""
    g = pkg.Geometry(vocab=40000, dim=256, heads=4, ffn_dim=1024, encoder_layers=1,
                     decoder_layers=2)
    model = pkg.seeded_model(seed=17, geometry=g)
    om = orc.OracleModel(model)
    b = pkg.ragged_batch(seed=41, n=260, vocab=g.vocab)
    with pkg.HipEngine(model, limits=b.limits) as e:
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
        want = orc.translate(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags,
                             threads=ORACLE_THREADS)
        print(f"vocabulary 40000: {sum(map(len, got))} tokens", flush=True)
        assert got == want
        sub = b.subset(range(20))
        res = probe_both(pkg, orc, e, om, sub.tokens, sub.offsets, [4] * 20, pkg.FLAG_IGNORE_EOS,
                         3, b.limits)
        assert check("vocabulary 40000, 20 rows", res) == 20
        assert e.is_ready()


@pytest.mark.parametrize("geom", [dict(dim=256, heads=4, ffn_dim=1024),
                                  dict(dim=512, heads=8, ffn_dim=1536),
                                  dict(dim=128, heads=2, ffn_dim=320),
                                  dict(dim=384, heads=8, ffn_dim=1536),
                                  dict(dim=192, heads=4, ffn_dim=768),
                                  dict(dim=64, heads=1, ffn_dim=256),
                                  dict(dim=320, heads=5, ffn_dim=1280),
                                  dict(dim=448, heads=7, ffn_dim=1792)])
def test_other_geometries_token_exact(pkg, orc, geom):
    g = pkg.Geometry(vocab=3000, encoder_layers=2, decoder_layers=2, **geom)
    model = pkg.seeded_model(seed=13, geometry=g)
    om = orc.OracleModel(model)
    b = pkg.ragged_batch(seed=19, n=12, vocab=g.vocab)
    with pkg.HipEngine(model, limits=b.limits) as e:
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
        want = orc.translate(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags,
                             threads=ORACLE_THREADS)
        print(f"geometry {geom}: {sum(map(len, got))} tokens", flush=True)
        assert got == want
        for step, rows in ((2, 12), (3, 1), (3, 5)):
            sub = b.subset(range(rows))
            res = probe_both(pkg, orc, e, om, sub.tokens, sub.offsets, [step + 1] * rows,
                             pkg.FLAG_IGNORE_EOS, step, b.limits)
            assert check(f"geometry {geom}, {rows} rows", res) == rows
        assert e.is_ready()
