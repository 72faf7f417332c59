"""End-to-end greedy translation on the GPU against the oracle, through the C ABI.

Gate: greedy token sequences identical on >= 99.5% of sentences (the kernels
follow the oracle's canonical arithmetic, so every sentence is expected to be
identical and the tests say how many were not)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


def compare(got_rows, want_rows, label):
    same = sum(g == w for g, w in zip(got_rows, want_rows))
    frac = same / max(1, len(want_rows))
    print(f"{label}: {same}/{len(want_rows)} sentences identical, "
          f"{sum(map(len, got_rows))} tokens", flush=True)
    return frac


@pytest.fixture(scope="module")
def engine(pkg, full_model):
    with pkg.HipEngine(full_model, limits=pkg.LIFTED_LIMITS) as e:
        yield e


@pytest.fixture(scope="module")
def oracle_model(orc, full_model):
    return orc.OracleModel(full_model)


def run_both(orc, engine, oracle_model, b):
    out = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags)
    want = orc.translate(oracle_model, b.tokens, b.offsets, b.max_output_tokens, b.limits,
                         b.flags, threads=ORACLE_THREADS)
    return out.rows(), want


def test_small_model_batch(pkg, orc, small_model):
    b = pkg.ragged_batch(seed=21, n=8, vocab=small_model.geometry.vocab)
    print("small model, 8 sentences", flush=True)
    with pkg.HipEngine(small_model, limits=b.limits) as e:
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens).rows()
    want = orc.translate(orc.OracleModel(small_model), b.tokens, b.offsets, b.max_output_tokens,
                         b.limits)
    assert compare(got, want, "small") == 1.0


def test_single_sentence_exact_32_steps(pkg, orc, full_model, oracle_model):
    b = pkg.single_sentence_batch()
    print("single sentence, 32 steps, EOS ignored", flush=True)
    with pkg.HipEngine(full_model, limits=b.limits) as e:
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
    want = orc.translate(oracle_model, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags)
    assert len(got[0]) == 32
    assert compare(got, want, "single") == 1.0


def test_ragged_64_sentence_batch(pkg, orc, engine, oracle_model):
    b = pkg.ragged_batch()
    print(f"ragged batch: {len(b.lengths)} sentences, {b.tokens.size} source tokens", flush=True)
    got, want = run_both(orc, engine, oracle_model, b)
    assert compare(got, want, "ragged-64") >= 0.995
    assert got == want
    # every row stops at its forced step unless it produced EOS first
    for row, lim in zip(got, b.max_output_tokens):
        assert len(row) == int(lim) or (row and row[-1] == 0)


def test_stress_batch_compaction(pkg, orc, engine, oracle_model):
    b = pkg.stress_batch()
    print(f"stress batch: {len(b.lengths)} segments, {b.tokens.size} source tokens, "
          f"max stop {int(b.max_output_tokens.max())}", flush=True)
    got, want = run_both(orc, engine, oracle_model, b)
    assert compare(got, want, "stress") >= 0.995
    assert got == want
    st = engine.last_stats()
    # the loop runs exactly as many steps as the longest output row needs
    # (compaction down to a single live row); the host may enqueue a few
    # more before it sees the count reach zero, which run on no rows
    longest = max(map(len, want))
    print(f"stress: {st['decode_steps']} steps on rows, {st['launched_steps']} launched, "
          f"longest output {longest}", flush=True)
    assert st["decode_steps"] == longest
    assert longest <= st["launched_steps"] <= int(b.max_output_tokens.max())
    assert st["generated_tokens"] == sum(map(len, want))


def test_batch_invariance_on_device(pkg, engine):
    b = pkg.ragged_batch(seed=31, n=12)
    full = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens).rows()
    for idx in ([0], [5, 3], [11, 2, 7, 1]):
        s = b.subset(idx)
        part = engine.translate_token_ids(s.tokens, s.offsets, s.max_output_tokens).rows()
        assert part == [full[i] for i in idx]


def test_errors_and_readiness(pkg, engine):
    ok_toks = np.array([5, 6, 7], np.int32)
    with pytest.raises(pkg.InvalidInput):
        engine.translate_token_ids(ok_toks, np.array([0, 3, 3], np.uint32), [1, 1])
    with pytest.raises(pkg.InvalidInput):
        engine.translate_token_ids(np.array([5, 32000], np.int32), np.array([0, 2], np.uint32), [1])
    with pytest.raises(pkg.InvalidInput):
        engine.translate_token_ids(ok_toks, np.array([0, 2], np.uint32), [1])
    assert engine.is_ready()  # validation errors do not poison the engine
    # zero budget and a one-token budget
    out = engine.translate_token_ids(ok_toks, np.array([0, 1, 3], np.uint32), [0, 1])
    assert out.rows()[0] == [] and len(out.rows()[1]) == 1
    info = engine.info()
    assert info["name"] == "hip" and info["precision"] == "q8" and "gfx950" in info["device"]


def test_reference_caps_are_enforced_when_configured(pkg, full_model):
    with pkg.HipEngine(full_model, limits=pkg.REFERENCE_LIMITS) as e:
        toks = np.full(600, 5, np.int32)
        offs = np.arange(0, 601, 120).astype(np.uint32)
        with pytest.raises(pkg.InvalidInput):
            e.translate_token_ids(toks, offs, [1] * 5)
        # length factor 2 caps a 3-token source at 6 generated tokens
        out = e.translate_token_ids(np.array([5, 6, 7], np.int32), np.array([0, 3], np.uint32),
                                    [100], flags=pkg.FLAG_IGNORE_EOS)
        assert len(out.rows()[0]) == 6


def test_timing_modes_keep_outputs_and_trace_launches(pkg, engine):
    b = pkg.ragged_batch(seed=41, n=24)
    print("timing modes: 24 sentences, off / per step / per launch", flush=True)
    engine.set_timing(0)
    base = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
    try:
        engine.set_timing(engine.TIME_STEPS)
        stepped = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
        rows, step_end = engine.last_step_trace()
        engine.set_timing(engine.TIME_KERNELS)
        timed = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
        kt = engine.last_kernel_trace()
    finally:
        engine.set_timing(0)
    assert stepped == base and timed == base
    counts = np.array([len(r) for r in base])
    steps = len(rows)
    assert steps == counts.max()
    # rows active at step t = sentences that produced more than t tokens
    assert [int(r) for r in rows] == [int((counts > t).sum()) for t in range(steps)]
    assert np.all(np.diff(step_end) > 0)
    vocab = kt["kind"] == engine.KERNEL_VOCAB
    assert sorted(kt["step"][vocab].tolist()) == list(range(steps))
    assert np.all(kt["layer"][vocab] == 0)
    assert set(kt["layer"][~vocab].tolist()) <= {0, 1}  # two decoder layers
    blocks = np.isin(kt["kind"], [engine.KERNEL_SELF_BLOCK, engine.KERNEL_CROSS_BLOCK])
    attn = np.isin(kt["kind"], [engine.KERNEL_SELF_ATTN, engine.KERNEL_CROSS_ATTN])
    assert np.all(vocab | blocks | attn)
    assert np.all(kt["us"] > 0)
    # 24 sentences of at most 128 source tokens: while a step attends over at
    # most 128 cached keys, both attention sublayers of both layers run as
    # blocks; later steps run self-attention as the separate kernel
    per_step = np.bincount(kt["step"][blocks], minlength=steps)
    assert np.all(per_step[:128] == 4) and np.all(per_step <= 4)
    per_step_all = per_step + np.bincount(kt["step"][attn], minlength=steps)
    assert np.all(per_step_all == 4)
    assert set(kt["kind"][attn].tolist()) <= {engine.KERNEL_SELF_ATTN}


def test_backend_repetitions_on_device(pkg, engine):
    b = pkg.ragged_batch(seed=51, n=6)
    sents = [b.tokens[b.offsets[i]:b.offsets[i + 1]].tolist() for i in range(6)]
    lims = b.max_output_tokens.tolist()
    plain = pkg.HipBackend(engine).translate_token_batch(sents, lims)
    wide = pkg.HipBackend(engine, duplicate_batch_width=3)
    out = wide.translate_token_batch(sents, lims, repetitions=[1, 4, 2, 1, 3, 1])
    assert out == plain
    assert engine.last_stats()["max_active_rows"] == 1 + 3 + 2 + 1 + 3 + 1
