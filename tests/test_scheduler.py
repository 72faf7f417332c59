"""The worker-loop model behind the HIP worker's scheduler settings
(marian-edge_amd/scheduler.py), no GPU.  Batch formation follows
crates/marian-core/src/scheduler.rs:494-659: the first request is taken, then
requests join until the batch is full or the window closes; a zero window
closes at once."""

import importlib

import pytest

TABLE = [dict(sentences=n, batch_ms=ms, target_tokens=31 * n, tokens_per_s=31 * n / (ms / 1e3))
         for n, ms in [(1, 2.5), (4, 4.5), (16, 6.5), (64, 9.5), (256, 16.0)]]


@pytest.fixture(scope="module")
def sch(pkg):
    return importlib.import_module(pkg.__name__ + ".scheduler")


def test_batch_time_interpolates_in_log2(sch):
    assert sch.batch_time_ms(TABLE, 1) == 2.5 and sch.batch_time_ms(TABLE, 256) == 16.0
    assert sch.batch_time_ms(TABLE, 8) == pytest.approx((4.5 + 6.5) / 2)
    assert sch.batch_time_ms(TABLE, 1000) == 16.0  # clamped


def test_zero_window_runs_every_request_alone(sch):
    r = sch.simulate(TABLE, 100.0, 256, 0, requests=500)
    assert r["mean_batch"] == 1.0


def test_full_batches_under_overload(sch):
    # far more requests per second than a 16-request batch can serve
    r = sch.simulate(TABLE, 50000.0, 16, 1500, requests=2000)
    assert r["mean_batch"] == 16.0


def test_light_load_waits_one_window(sch):
    # one request every ~100 ms: each batch holds one request and waits out the window
    r = sch.simulate(TABLE, 10.0, 256, 3000, requests=300)
    assert r["mean_batch"] == 1.0
    assert r["p50_ms"] == pytest.approx(3.0 + 2.5, abs=1e-6)


def test_recommendation_shape(sch):
    rec = sch.recommend(TABLE)
    assert rec["max_batch_size"] == 256 and rec["batch_window_us"] in sch.WINDOWS_US
    assert rec["max_padded_source_chars"] >= 256 * 256
    best = min((g for g in rec["grid"] if g["max_batch_size"] == 256), key=lambda g: g["mean_p50_ms"])
    assert best["batch_window_us"] == rec["batch_window_us"]
    # the reference CLI's 16-request batches cannot keep up with 90% of a 256-batch's rate
    assert rec["reference_cli_defaults"]["load_90"]["p50_ms"] > rec["recommended"]["load_90"]["p50_ms"]
