#!/usr/bin/env python3
"""Op-level measurements of the marian-hip kernels on the Q8 GEMM sweep and the
varlen attention workload, timed from a rocprofv3 kernel trace of this script
(per-call Python overhead would otherwise dominate small kernels).

    rocprofv3 --kernel-trace --output-format csv -d DIR -o ops -- \\
        python3 marian-edge_amd/bench_ops.py run --out DIR/ops_run.json
    python3 marian-edge_amd/bench_ops.py summarize DIR/ops_run.json DIR/ops_kernel_trace.csv

`run` executes every case `reps` times back to back and records, in call
order, how many kernels each call dispatches.  `summarize` walks the trace's
marian-hip dispatches in start order, attributes them to the recorded calls,
and reports per case the median device time of one call (the sum of its
kernels' durations), the algorithmic bytes and the achieved fraction of the
MI355X's 8 TB/s HBM peak (and of the 5.0 POP/s dense int8 MFMA peak).

Cases:
  * GEMM sweep: fp32 A ~ N(0,1) [M, K] quantized per row, int8 W [N, K] with
    per-column scales, bias; outputs i32 accumulators and fp32.  Shapes (K, N)
    in (512,1536) (512,512) (512,2048) (2048,512) (512,32000), M in 1, 8, 64,
    256, 4096.  Algorithmic bytes 4MK + KN + 4N + 8MN (fp32 A, int8 W, one
    per-column scale, i32 + fp32 out); bias reads are 4N more and counted.
  * Varlen attention: 256 packed sentences with lengths ~ lognormal(3.2, 0.6)
    clipped to [4, 256], 8 heads x 64, Q/K/V fp32 and bf16, as packed
    self-attention (the query-tile list, then the key-staging kernel).
    Algorithmic bytes 3 * T * d * b + 4 * T * d (Q, K, V in their type, fp32
    O out).
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys
from pathlib import Path

import numpy as np

HBM_PEAK = 8.0e12
INT8_PEAK = 5.0e15


def _load_package():
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    import __graft_entry__ as ge

    return ge.load_package()


def run(out_path: str, reps: int) -> None:
    pkg = _load_package()
    from importlib import import_module

    dev = import_module(pkg.__name__ + ".device")
    D = dev.DeviceArray
    cases = []

    for K, N in pkg.GEMM_SHAPES:
        for M in pkg.GEMM_ROWS:
            a, w, mult, bias = pkg.gemm_inputs(M, K, N)
            x, dw, dm, db = (D.from_host(t) for t in (a, w, mult, bias))
            oi, of = D((M, N), np.int32), D((M, N), np.float32)
            for _ in range(reps):
                dev.q8_linear(x, dw, dm, db, oi, of)
            dev.synchronize()
            cases.append(dict(label=f"q8_linear K={K} N={N} M={M}", kind="gemm", M=M, K=K, N=N,
                              calls=reps, kernels_per_call=2,
                              bytes=4 * M * K + K * N + 8 * N + 8 * M * N, flops=2 * M * N * K))
            for t in (x, dw, dm, db, oi, of):
                t.free()

    q, k, v, cu = pkg.attention_inputs()
    T, d = q.shape
    seq = np.repeat(np.arange(len(cu) - 1, dtype=np.int32), np.diff(cu.astype(np.int64)))
    lmax = int(np.diff(cu.astype(np.int64)).max())
    for bf16 in (False, True):
        if bf16:
            hq, hk, hv = (pkg.synthetic.bf16_round(t) for t in (q, k, v))
            b = 2
        else:
            hq, hk, hv = q, k, v
            b = 4
        dq, dk, dv = (D.from_host(t) for t in (hq, hk, hv))
        dseq, dcu = D.from_host(seq), D.from_host(cu)
        do = D((T, d), np.float32)
        for _ in range(reps):
            dev.attention(dq, dk, dv, dseq, dcu, do, heads=d // 64, max_keys=lmax, bf16=bf16)
        dev.synchronize()
        # Q, K, V read in their type, O written in fp32.
        # Two kernels per call: the query-tile list, then the attention.
        cases.append(dict(label=f"attention {'bf16' if bf16 else 'fp32'} T={T}", kind="attention",
                          T=T, calls=reps, kernels_per_call=2,
                          bytes=3 * T * d * b + 4 * T * d, flops=4 * d * int((np.diff(cu.astype(np.int64)) ** 2).sum())))
        for t in (dq, dk, dv, dseq, dcu, do):
            t.free()
    Path(out_path).parent.mkdir(parents=True, exist_ok=True)
    Path(out_path).write_text(json.dumps({"reps": reps, "cases": cases}, indent=1))
    print(f"wrote {len(cases)} cases to {out_path}", flush=True)


def summarize(run_path: str, trace_path: str) -> str:
    spec = json.loads(Path(run_path).read_text())
    rows = []
    with open(trace_path, newline="") as f:
        for r in csv.DictReader(f):
            if "mh::" in r["Kernel_Name"]:
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    need = sum(c["calls"] * c["kernels_per_call"] for c in spec["cases"])
    if len(rows) != need:
        raise SystemExit(f"trace holds {len(rows)} marian-hip dispatches, the run made {need}")
    out = ["| case | kernels | median us / call | algorithmic MB | GB/s | frac of 8 TB/s | int8 MFMA frac |",
           "|---|---|---:|---:|---:|---:|---:|"]
    i = 0
    for c in spec["cases"]:
        per_call = []
        names = set()
        for _ in range(c["calls"]):
            ks = rows[i:i + c["kernels_per_call"]]
            i += c["kernels_per_call"]
            per_call.append(sum(e - s for s, e, _ in ks) / 1000.0)
            names.update(n.replace("mh::(anonymous namespace)::", "").replace("void ", "").split("(")[0]
                         for _, _, n in ks)
        us = statistics.median(per_call[1:] if len(per_call) > 1 else per_call)
        gbs = c["bytes"] / (us * 1e-6) / 1e9
        mf = c["flops"] / (us * 1e-6) / INT8_PEAK if c["kind"] == "gemm" else float("nan")
        out.append(f"| {c['label']} | {', '.join(sorted(names))} | {us:.2f} | {c['bytes'] / 1e6:.3f} | "
                   f"{gbs:.0f} | {gbs * 1e9 / HBM_PEAK:.3f} | "
                   + (f"{mf:.4f} |" if c["kind"] == "gemm" else "- |"))
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--out", required=True)
    r.add_argument("--reps", type=int, default=20)
    s = sub.add_parser("summarize")
    s.add_argument("run_json")
    s.add_argument("trace_csv")
    a = ap.parse_args(argv)
    if a.cmd == "run":
        run(a.out, a.reps)
    else:
        print(summarize(a.run_json, a.trace_csv))
    return 0


if __name__ == "__main__":
    sys.exit(main())
