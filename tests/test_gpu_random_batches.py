"""Randomized parity sweep: engine against the oracle, token-exact, on
seeded random draws of geometry, vocabulary size, decoder depth, batch size
(1-89 sentences, so steps cross every row threshold of the decode kernels)
and the EOS flag, for the Transformer graph and, every third case, the
Transformer-SSRU graph.  The draws come from a fixed seed, so a failure
names a reproducible case."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16
CASES = 40

GEOMS = [dict(dim=512, heads=8, ffn_dim=2048), dict(dim=256, heads=4, ffn_dim=1024),
         dict(dim=384, heads=6, ffn_dim=1536), dict(dim=512, heads=8, ffn_dim=1536),
         dict(dim=384, heads=8, ffn_dim=1536)]
SSRU_GEOMS = [dict(dim=384, heads=8, ffn_dim=1536), dict(dim=256, heads=4, ffn_dim=1024)]


def draws():
    rng = np.random.default_rng(20261202)
    for i in range(CASES):
        yield (i, int(rng.integers(len(GEOMS))), int(rng.integers(1, 10**6)), int(rng.integers(1, 90)),
               int(rng.choice([3000, 5000, 33000])), int(rng.integers(0, 2)), int(rng.integers(1, 3)))


def test_random_batches_token_exact(pkg, orc):
    bad = []
    for i, gi, seed, n, V, eos_off, layers in draws():
        flags = pkg.FLAG_IGNORE_EOS if eos_off else 0
        g = pkg.Geometry(vocab=V, encoder_layers=1, decoder_layers=layers, **GEOMS[gi])
        model = pkg.seeded_model(seed=seed, geometry=g)
        b = pkg.ragged_batch(seed=seed + 1, n=n, vocab=V)
        with pkg.HipEngine(model, limits=b.limits) as e:
            got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, flags).rows()
        want = orc.translate(orc.OracleModel(model), b.tokens, b.offsets, b.max_output_tokens, b.limits,
                             flags, threads=ORACLE_THREADS)
        case = f"case {i}: geometry {GEOMS[gi]}, V={V}, {n} sentences, seed {seed}, flags {flags}"
        print(f"{case}: {sum(map(len, got))} tokens", flush=True)
        if got != want:
            bad.append(case)
        if i % 3 == 0:
            sg = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=1, decoder_layers=2,
                                  **SSRU_GEOMS[i % 2])
            sm = pkg.seeded_ssru_model(seed=seed, geometry=sg, std=0.05)
            sb = pkg.ragged_batch(seed=seed + 2, n=n, vocab=sg.source_vocab)
            with pkg.HipEngine(sm, limits=sb.limits) as e:
                got = e.translate_token_ids(sb.tokens, sb.offsets, sb.max_output_tokens, flags).rows()
            want = orc.translate_ssru(orc.OracleSsruModel(sm), sb.tokens, sb.offsets, sb.max_output_tokens,
                                      sb.limits, flags, threads=ORACLE_THREADS)
            print(f"  ssru {SSRU_GEOMS[i % 2]}: {sum(map(len, got))} tokens", flush=True)
            if got != want:
                bad.append(f"ssru {case}")
    assert not bad, bad


def test_rows_ending_on_eos_stop_the_launches(pkg, orc):
    """A model whose output bias makes id 0 (EOS) every row's argmax: all
    rows end at step 0.  The decode loop learns it from the count the
    finalizer stores in pinned host memory every 8 steps and stops
    launching within a few poll periods (the engine's launched-step count),
    far below the step limit; the tokens match the oracle."""
    g = pkg.Geometry(vocab=2048, dim=256, heads=4, ffn_dim=1024, encoder_layers=1, decoder_layers=1)
    model = pkg.seeded_model(seed=9, geometry=g)
    model.output_bias = model.output_bias.copy()
    model.output_bias[0] = 1.0e4
    b = pkg.ragged_batch(seed=7, n=16, vocab=g.vocab)
    limit = 200
    mo = np.full(16, limit, np.uint32)
    with pkg.HipEngine(model, limits=pkg.LIFTED_LIMITS) as e:
        e.translate_token_ids(b.tokens, b.offsets, mo, 0)  # warm-up
        got = e.translate_token_ids(b.tokens, b.offsets, mo, 0).rows()
        eos = e.last_stats()
        forced = e.translate_token_ids(b.tokens, b.offsets, mo, pkg.FLAG_IGNORE_EOS).rows()
        full = e.last_stats()
    want = orc.translate(orc.OracleModel(model), b.tokens, b.offsets, mo, pkg.LIFTED_LIMITS, 0,
                         threads=ORACLE_THREADS)
    print(f"EOS at step 0: {eos['decode_steps']} step on rows, {eos['launched_steps']} launched, "
          f"decode {eos['decode_ms']:.3f} ms; all {limit} steps (EOS ignored): "
          f"{full['launched_steps']} launched, {full['decode_ms']:.3f} ms", flush=True)
    assert got == want
    assert all(len(r) <= 1 for r in got) and all(len(r) == limit for r in forced)
    assert eos["decode_steps"] == 1 and full["decode_steps"] == full["launched_steps"] == limit
    # the launches stop within a few poll periods of 8 steps (count stored at
    # step 7, seen when step 15 or a later poll step is enqueued)
    assert eos["launched_steps"] <= 5 * 8

