"""The opt-in fast-reduction mode (MARIAN_HIP_FLAG_FAST_REDUCTIONS) on the GPU.

The flag changes only the decoder's LayerNorm sums and softmax denominators,
to 64 lane partials combined by an xor butterfly; the oracle restates that
order as ORACLE_ORDER_FAST_DECODER.  Two checks:
  * against the oracle in that order: encoder states, one decode step's
    logits and every token bit for bit, at every row and key threshold at
    which the engine switches kernels (as tests/test_gpu_probe.py does for the
    exact mode), and token-exact on the 64-sentence and stress batches;
  * against the exact mode (the reference's order, itself bit-exact with the
    oracle): greedy sentences identical on at least 99.5% of sentences, the
    count printed, and the logits' relative L2 difference at three steps
    printed and held below 1e-2.  It is above the 1e-3 logit tolerance (an
    int8 re-quantization that flips moves a whole step), so the mode is
    opt-in and the exact mode remains the default.
"""

import numpy as np
import pytest

from test_gpu_probe import check, probe_both, sentences

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


def probe_fast(pkg, orc, engine, om, toks, offs, limits, flags, step, lim_cfg):
    """probe_both with the engine's fast flag and the oracle's fast order."""
    lim = np.minimum(np.asarray(limits, np.int64), step + 1).astype(np.uint32)
    fast = flags | pkg.FLAG_FAST_REDUCTIONS
    out, enc, lg, act = engine.translate_probe(toks, offs, lim, fast, probe_step=step)
    rows, enc_o, lg_o, act_o = orc.translate_probe(om, toks, offs, lim, lim_cfg, flags, probe_step=step,
                                                   order=orc.FAST_DECODER, threads=ORACLE_THREADS)
    plain = engine.translate_token_ids(toks, offs, lim, fast).rows()
    return out.rows(), enc, lg, act, rows, enc_o, lg_o, act_o, plain


@pytest.fixture(scope="module")
def small(pkg, orc, small_model):
    with pkg.HipEngine(small_model, limits=pkg.LIFTED_LIMITS) as e:
        yield e, orc.OracleModel(small_model), small_model.geometry.vocab


@pytest.fixture(scope="module")
def full(pkg, orc, full_model):
    with pkg.HipEngine(full_model, limits=pkg.LIFTED_LIMITS) as e:
        yield e, orc.OracleModel(full_model)


@pytest.mark.parametrize("rows", [1, 2, 4, 5, 8, 9, 32, 33, 64, 65])
def test_fast_probe_row_thresholds(pkg, orc, small, rows):
    engine, om, V = small
    rng = np.random.default_rng(300 + rows)
    toks, offs = sentences(rng, rows, 5, 40, V)
    res = probe_fast(pkg, orc, engine, om, toks, offs, [8] * rows, pkg.FLAG_IGNORE_EOS, 3,
                     pkg.LIFTED_LIMITS)
    assert check(f"fast, rows={rows}", res) == rows


@pytest.mark.parametrize("step", [127, 128, 200])
def test_fast_probe_self_key_threshold(pkg, orc, small, step):
    engine, om, V = small
    rng = np.random.default_rng(17)
    toks, offs = sentences(rng, 2, 10, 30, V)
    res = probe_fast(pkg, orc, engine, om, toks, offs, [step + 1, step + 1], pkg.FLAG_IGNORE_EOS, step,
                     pkg.LIFTED_LIMITS)
    assert check(f"fast, self keys={step + 1}", res) == 2


@pytest.mark.parametrize("src_len", [128, 129, 300, 512, 513])
def test_fast_probe_cross_key_threshold(pkg, orc, small, src_len):
    engine, om, V = small
    rng = np.random.default_rng(1000 + src_len)
    toks, offs = sentences(rng, 3, 20, 60, V)
    long = rng.integers(3, V, size=src_len).astype(np.int32)
    toks = np.concatenate([toks, long])
    offs = np.append(offs, offs[-1] + src_len).astype(np.uint32)
    res = probe_fast(pkg, orc, engine, om, toks, offs, [6] * 4, pkg.FLAG_IGNORE_EOS, 2,
                     pkg.LIFTED_LIMITS)
    assert check(f"fast, source tokens={src_len}", res) == 4


@pytest.mark.parametrize("step", [4, 40, 100])
def test_fast_probe_ragged_64(pkg, orc, full, step):
    engine, om = full
    b = pkg.ragged_batch()
    res = probe_fast(pkg, orc, engine, om, b.tokens, b.offsets, b.max_output_tokens, b.flags, step,
                     b.limits)
    check(f"fast, ragged-64, step {step}", res)


@pytest.mark.parametrize("name", ["ragged", "stress"])
def test_fast_mode_token_exact_and_close_to_exact_mode(pkg, orc, full, name):
    engine, om = full
    b = pkg.ragged_batch() if name == "ragged" else pkg.stress_batch()
    fast = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens,
                                      b.flags | pkg.FLAG_FAST_REDUCTIONS).rows()
    exact = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
    want = orc.translate(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags,
                         order=orc.FAST_DECODER, threads=ORACLE_THREADS)
    same = sum(f == e for f, e in zip(fast, exact))
    print(f"{name}: fast mode {same}/{len(exact)} sentences identical to the exact mode", flush=True)
    assert fast == want, "fast mode differs from the oracle's fast order"
    assert same / len(exact) >= 0.995


@pytest.mark.parametrize("step", [0, 20, 60])
def test_fast_logits_close_to_exact(pkg, full, step):
    """Logits of the fast mode against the exact mode at one decode step: the
    relative L2 difference over the finite logits (masked ids are -inf in
    both), printed, below 1e-2."""
    engine, _ = full
    b = pkg.ragged_batch()
    lim = np.minimum(b.max_output_tokens.astype(np.int64), step + 1).astype(np.uint32)
    _, enc_f, lg_f, act_f = engine.translate_probe(b.tokens, b.offsets, lim,
                                                   b.flags | pkg.FLAG_FAST_REDUCTIONS, probe_step=step)
    _, enc_e, lg_e, act_e = engine.translate_probe(b.tokens, b.offsets, lim, b.flags, probe_step=step)
    assert np.array_equal(act_f, act_e) and act_e.any()
    assert np.array_equal(enc_f.view(np.uint32), enc_e.view(np.uint32)), "the encoder must not change"
    f, e = lg_f[act_e], lg_e[act_e]
    fin = np.isfinite(e)
    assert np.array_equal(fin, np.isfinite(f))
    rel = np.linalg.norm(np.where(fin, f, 0.0) - np.where(fin, e, 0.0)) / np.linalg.norm(np.where(fin, e, 0.0))
    print(f"step {step}: {int(act_e.sum())} rows, relative L2 logit difference {rel:.3e}", flush=True)
    assert rel <= 1e-2


def test_fast_flag_is_rejected_by_the_ssru_engine(pkg):
    g = pkg.SsruGeometry(source_vocab=500, target_vocab=600, encoder_layers=1, decoder_layers=1,
                         dim=256, heads=4, ffn_dim=512)
    model = pkg.seeded_ssru_model(seed=3, geometry=g, std=0.05)
    with pkg.HipEngine(model, limits=pkg.LIFTED_LIMITS) as e:
        with pytest.raises(pkg.InvalidInput, match="transformer graph only"):
            e.translate_token_ids(np.array([5, 6, 7], np.int32), np.array([0, 3], np.uint32), [4],
                                  pkg.FLAG_FAST_REDUCTIONS)
        assert e.is_ready()
