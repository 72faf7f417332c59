"""Serving-side behaviour of the engine on the GPU: the load-time warmup
(Q8CpuEngine::warmup, crates/marian-cpu/src/q8_engine.rs:349-351, called by the
backends at load, crates/marian-cpu/src/backend.rs:448, 812), the capacity
reservation that keeps requests free of allocations, and the call statistics
a serving worker reads.  Outputs are checked against the oracle."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


def test_warmup_runs_the_reference_batch(pkg, small_model):
    with pkg.HipEngine(small_model) as e:
        e.warmup()
        st = e.last_stats()
        print(f"warmup: {st['generated_tokens']} tokens, {st['decode_steps']} steps, "
              f"{st['allocations']} allocations", flush=True)
        assert 1 <= st["generated_tokens"] <= 4 and st["max_active_rows"] == 1
        assert st["allocations"] > 0  # the first call on a fresh engine sizes its buffers
        e.warmup()
        assert e.last_stats()["allocations"] == 0
        assert e.is_ready()


def test_reserved_engine_allocates_nothing_on_its_first_request(pkg, orc, full_model):
    """A worker sized for the 64-sentence ragged batch at load serves it, and
    any smaller batch, without a single device or pinned host allocation."""
    b = pkg.ragged_batch()
    small = b.subset(range(7))
    cap = pkg.capacity_for([b])
    print(f"capacity {cap}", flush=True)
    with pkg.HipEngine(full_model, limits=b.limits, capacity=cap) as e:
        e.warmup()
        assert e.last_stats()["allocations"] == 0
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags).rows()
        st = e.last_stats()
        print(f"first request: {st['generated_tokens']} tokens, {st['allocations']} allocations",
              flush=True)
        assert st["allocations"] == 0
        part = e.translate_token_ids(small.tokens, small.offsets, small.max_output_tokens,
                                     small.flags).rows()
        assert e.last_stats()["allocations"] == 0
    want = orc.translate(orc.OracleModel(full_model), b.tokens, b.offsets, b.max_output_tokens,
                         b.limits, b.flags, threads=ORACLE_THREADS)
    assert got == want
    assert part == want[:7]


def test_unreserved_engine_grows_once_then_reuses(pkg, orc, small_model):
    """Without a reservation the first call of a shape allocates, the same
    call again allocates nothing, and a larger batch grows the buffers and
    still matches the oracle."""
    om = orc.OracleModel(small_model)
    small = pkg.ragged_batch(seed=23, n=6, vocab=small_model.geometry.vocab)
    large = pkg.ragged_batch(seed=29, n=40, vocab=small_model.geometry.vocab)
    with pkg.HipEngine(small_model, limits=large.limits) as e:
        e.translate_token_ids(small.tokens, small.offsets, small.max_output_tokens, small.flags)
        first = e.last_stats()["allocations"]
        e.translate_token_ids(small.tokens, small.offsets, small.max_output_tokens, small.flags)
        again = e.last_stats()["allocations"]
        got = e.translate_token_ids(large.tokens, large.offsets, large.max_output_tokens,
                                    large.flags).rows()
        grown = e.last_stats()["allocations"]
        print(f"allocations: first {first}, repeat {again}, larger batch {grown}", flush=True)
        assert first > 0 and again == 0 and grown > 0
    want = orc.translate(om, large.tokens, large.offsets, large.max_output_tokens, large.limits,
                         large.flags, threads=ORACLE_THREADS)
    assert got == want


def test_backend_warms_up_at_load(pkg, small_model):
    with pkg.HipEngine(small_model) as e:
        pkg.HipBackend(e)
        st = e.last_stats()
        assert 1 <= st["generated_tokens"] <= 4 and st["max_active_rows"] == 1


def test_reserve_rejects_bad_capacities(pkg, small_model):
    with pkg.HipEngine(small_model) as e:
        with pytest.raises(pkg.InvalidInput):
            e.reserve(sentences=0, source_tokens=10, output_tokens=10, steps=10)
        with pytest.raises(pkg.InvalidInput):
            e.reserve(sentences=5000, source_tokens=10, output_tokens=10, steps=10)
        assert e.is_ready()
        e.reserve(sentences=4, source_tokens=64, output_tokens=64, steps=16)
        # a batch beyond the reservation grows the buffers and runs
        b = pkg.ragged_batch(seed=5, n=4, vocab=small_model.geometry.vocab)
        lim = np.minimum(b.max_output_tokens, 16)
        e.translate_token_ids(b.tokens, b.offsets, lim, b.flags)
        assert e.is_ready()
