"""Scheduler settings for a HIP translation worker, derived from measured
batch times.

The reference's dynamic batcher (crates/marian-core/src/scheduler.rs:494-659,
`worker_loop`) takes the first queued request, then keeps collecting requests
with the same batch key until it holds `batch_limit` of them or
`batch_window` has passed since it started the batch; `batch_limit` is
min(max_batch_size, max_padded_source_chars / length bucket) (:544-548).  It
then runs the whole batch and answers every request of it at once.  Its
defaults are 16 requests and a 1500 us window (:33-44); the server's CLI uses
16 and 750 us (crates/marian-server/src/main.rs:49-66).

`simulate` replays that loop for one worker over Poisson arrivals, with each
batch taking the device time measured for a batch of that size (the
measured table interpolated in log2 of the size).  `recommend` picks the
worker's settings from a measured table.  The figures it returns are a model
of the scheduler over measured batch times, not a measurement of a server.
"""

from __future__ import annotations

import math

import numpy as np

# The reference batcher's own ceiling (scheduler.rs:20).
MAX_BATCH_SIZE = 256
# The length bucket of one request is its character count rounded up to a
# power of two (types.rs:28-37); 1024 covers the 256-token segments the text
# adapter cuts long inputs into.
BUCKET_CHARS = 1024

WINDOWS_US = (0, 100, 250, 500, 750, 1500, 3000)
BATCH_SIZES = (16, 64, 128, 256)
LOADS = (0.1, 0.5, 0.9)  # fractions of the largest batch's request rate


def batch_time_ms(table, n: int) -> float:
    """Device time of a batch of n sentences: the measured table interpolated
    linearly in log2 of the batch size (clamped to the measured range)."""
    xs = np.log2([r["sentences"] for r in table])
    ys = [r["batch_ms"] for r in table]
    return float(np.interp(math.log2(max(n, 1)), xs, ys))


def simulate(table, rate_per_s: float, max_batch: int, window_us: float, requests: int = 4000,
             seed: int = 0) -> dict:
    """One worker over `requests` Poisson arrivals at `rate_per_s`, batches
    formed as worker_loop forms them: the first queued request is taken when
    the worker is free; further requests join while fewer than max_batch are
    held and they arrive before the window closes (with a zero window the
    loop stops at once, so every batch is one request); the batch runs when
    it is full (at the arrival of its last request) or when the window
    closes, and takes batch_time_ms.  Returns the requests' latency (arrival
    to answer) p50 / p99 and the mean batch size."""
    rng = np.random.default_rng(seed)
    arrivals = np.cumsum(rng.exponential(1000.0 / rate_per_s, size=requests))  # ms
    lat = np.empty(requests)
    sizes = []
    free = 0.0  # when the worker is next free
    i = 0
    while i < requests:
        start = max(free, arrivals[i])
        deadline = start + window_us / 1000.0
        j = i + 1
        while window_us > 0 and j < requests and j - i < max_batch and arrivals[j] < deadline:
            j += 1
        if window_us == 0:
            run = start
        elif j - i == max_batch:
            run = max(start, arrivals[j - 1])
        else:
            run = deadline
        done = run + batch_time_ms(table, j - i)
        lat[i:j] = done - arrivals[i:j]
        sizes.append(j - i)
        free = done
        i = j
    return {"p50_ms": round(float(np.median(lat)), 3), "p99_ms": round(float(np.percentile(lat, 99)), 3),
            "mean_batch": round(float(np.mean(sizes)), 1)}


def recommend(table) -> dict:
    """HIP worker settings from a measured batch-size table (rows with
    sentences, batch_ms, target_tokens, tokens_per_s).

    max_batch_size: the reference's ceiling, 256.  A decode step costs nearly
    the same from 1 to 64 rows here, so the largest batch serves the most
    requests per second, and a batch only grows that large when requests are
    queued anyway: at light load the window, not the size, bounds waiting.
    batch_window: the window with the lowest median latency averaged over
    light, medium and heavy load (10%, 50% and 90% of the request rate the
    largest measured batch sustains), each load simulated with every window.
    max_padded_source_chars: large enough that the length bucket never caps
    the batch below max_batch_size (the engine packs rows without padding)."""
    big = max(table, key=lambda r: r["sentences"])
    tokens_per_req = big["target_tokens"] / big["sentences"]
    capacity_rps = big["sentences"] / (big["batch_ms"] / 1000.0)
    grid = []
    for mb in BATCH_SIZES:
        for w in WINDOWS_US:
            row = {"max_batch_size": mb, "batch_window_us": w}
            for load in LOADS:
                row[f"load_{int(load * 100)}"] = simulate(table, load * capacity_rps, mb, w)
            row["mean_p50_ms"] = round(float(np.mean([row[f"load_{int(x * 100)}"]["p50_ms"] for x in LOADS])), 3)
            grid.append(row)
    best_w = min((r for r in grid if r["max_batch_size"] == MAX_BATCH_SIZE), key=lambda r: r["mean_p50_ms"])
    ref = next(r for r in grid if r["max_batch_size"] == 16 and r["batch_window_us"] == 750)
    return {
        "max_batch_size": MAX_BATCH_SIZE,
        "batch_window_us": best_w["batch_window_us"],
        "max_padded_source_chars": MAX_BATCH_SIZE * BUCKET_CHARS,
        "basis": (f"one worker, Poisson single-sentence requests ({tokens_per_req:.1f} target tokens each "
                  f"on average) at 10/50/90% of {capacity_rps:.0f} requests/s (what a "
                  f"{big['sentences']}-sentence batch sustains), batch device times interpolated from "
                  "the measured table; a model of scheduler.rs's worker_loop, not a server measurement"),
        "recommended": {k: best_w[k] for k in best_w if k.startswith("load_")},
        "reference_cli_defaults": {"max_batch_size": 16, "batch_window_us": 750,
                                   **{k: ref[k] for k in ref if k.startswith("load_")}},
        "grid": grid,
    }
