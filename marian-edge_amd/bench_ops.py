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
    O out).  Also as cross-attention at decode shape: one query per sentence
    (its first row's Q) over the sentence's packed K/V, one wave per (query,
    head); bytes 2 * T * d * b + B * d * b + 4 * B * d.
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
        # Cross-attention at decode shape: one query per sentence over its
        # packed keys and values (one wave per (query, head)).
        B = len(cu) - 1
        qc = hq[cu[:-1].astype(np.int64)]
        dq, dk, dv = (D.from_host(t) for t in (qc, hk, hv))
        dseq, dcu = D.from_host(np.arange(B, dtype=np.int32)), D.from_host(cu)
        do = D((B, d), np.float32)
        for _ in range(reps):
            dev.attention(dq, dk, dv, dseq, dcu, do, heads=d // 64, max_keys=lmax, bf16=bf16,
                          packed_self=False)
        dev.synchronize()
        # K and V of every sentence read once, B queries in, B fp32 rows out.
        cases.append(dict(label=f"cross-attention {'bf16' if bf16 else 'fp32'} B={B} T={T}",
                          kind="attention", T=T, calls=reps, kernels_per_call=1,
                          bytes=2 * T * d * b + B * d * b + 4 * B * d, flops=4 * d * T))
        for t in (dq, dk, dv, dseq, dcu, do):
            t.free()
    Path(out_path).parent.mkdir(parents=True, exist_ok=True)
    Path(out_path).write_text(json.dumps({"reps": reps, "cases": cases}, indent=1))
    print(f"wrote {len(cases)} cases to {out_path}", flush=True)


def copy_calibration(mb: int, reps: int) -> None:
    """Device-to-device copies of `mb` MiB (the runtime's copy kernel): the
    reference for what the memory-traffic counters read per byte moved."""
    pkg = _load_package()
    from importlib import import_module

    dev = import_module(pkg.__name__ + ".device")
    n = mb * 1024 * 1024
    src = dev.DeviceArray.from_host(np.ones(n // 4, np.float32))
    dst = dev.DeviceArray((n // 4,), np.float32)
    for _ in range(reps):
        dev.copy(dst, src)
    dev.synchronize()
    print(f"copied {mb} MiB x {reps}", flush=True)


def memory_rates(mb: int, reps: int) -> dict:
    """The runtime's fill and device-to-device copy kernels on `mb` MiB
    buffers, `reps` calls each between two events: the practical write-only
    and read+write rates of this device, next to the 8 TB/s peak."""
    pkg = _load_package()
    from importlib import import_module

    dev = import_module(pkg.__name__ + ".device")
    n = mb * 1024 * 1024
    a = dev.DeviceArray((n // 4,), np.float32)
    b = dev.DeviceArray((n // 4,), np.float32)
    out = {"mib": mb, "calls": reps}
    for name, fn, moved in (("fill", lambda: a.fill_bytes(1), n), ("copy", lambda: dev.copy(b, a), 2 * n)):
        fn()
        fn()
        dev.synchronize()
        e0, e1 = dev.Event(), dev.Event()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.sync()
        us = e0.elapsed_ms(e1) / reps * 1000.0
        out[name] = {"us_per_call": round(us, 1), "bytes_moved": moved,
                     "gb_per_s": round(moved / us / 1e3, 0), "frac_of_8tbs": round(moved / us / 1e3 / 8000, 3)}
        e0.close()
        e1.close()
    a.free()
    b.free()
    return out


def pmc_summary(fetch_csv: str, write_csv: str, copy_fetch_csv: str, copy_write_csv: str,
                copy_mb: int, workload: str) -> dict:
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the decode kernels from
    two rocprofv3 --pmc runs of bench.py, scaled by what the same counters
    read for the copy kernel per byte it moves."""
    def per_kernel(path, counter):
        out = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") != counter:
                    continue
                name = r["Kernel_Name"].replace("mh::(anonymous namespace)::", "").replace("void ", "")
                out.setdefault(name.split("(")[0], []).append(float(r["Counter_Value"]))
        return out

    fetch, write = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    cf, cw = per_kernel(copy_fetch_csv, "FETCH_SIZE"), per_kernel(copy_write_csv, "WRITE_SIZE")
    copy_kib = copy_mb * 1024.0

    def copy_factor(d):
        vals = [v for k, vs in d.items() if "copyBuffer" in k for v in vs]
        return copy_kib / statistics.median(vals) if vals else float("nan")

    ff, fw = copy_factor(cf), copy_factor(cw)
    res = {
        "workload": workload,
        "counters": "FETCH_SIZE and WRITE_SIZE (KiB per dispatch), one rocprofv3 --pmc run each",
        "calibration": {
            "copy_mib": copy_mb,
            "fetch_factor": round(ff, 4),
            "write_factor": round(fw, 4),
            "note": f"the runtime's copy kernel moving {copy_mb} MiB reads FETCH_SIZE = "
                    f"{copy_mb / ff:.0f} MiB and WRITE_SIZE = {copy_mb / fw:.0f} MiB; kernel counts are "
                    f"scaled by {copy_mb} MiB / those readings",
        },
        "kernels": {},
    }
    for k in sorted(set(fetch) | set(write)):
        if not k.startswith("k_"):
            continue
        fk = statistics.mean(fetch.get(k, [0.0])) * ff * 1024.0
        wk = statistics.mean(write.get(k, [0.0])) * fw * 1024.0
        res["kernels"][k] = {"fetch_bytes_per_dispatch": round(fk), "write_bytes_per_dispatch": round(wk),
                             "dispatches": len(fetch.get(k, []))}
    return res


def counter_summary(csv_paths: list[str], trace_csv: str | None = None) -> dict:
    """Dispatch-averaged counter values per kernel from rocprofv3 --pmc
    counter_collection.csv files (any counters), with two derived figures
    where their counters were collected:
      * dram_read_share: TCC_EA0_RDREQ_DRAM_sum / TCC_EA0_RDREQ_sum, the share
        of the L2's read requests that go out to the memory controller;
      * mfma_util: SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs), the
        matrix cores' busy fraction over the dispatch (1024 SIMDs: 256 CUs x 4);
    and, with a kernel trace of the same command, the int8 MFMA throughput
    SQ_INSTS_VALU_MFMA_MOPS_I8 x 512 ops / average duration."""
    vals: dict = {}
    for path in csv_paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"].replace("mh::(anonymous namespace)::", "").replace("void ", "")
                name = name.split("(")[0]
                key = (r.get("Dispatch_Id") or r.get("Correlation_Id"), r["Counter_Name"])
                vals.setdefault(name, {}).setdefault(r["Counter_Name"], {})
                d = vals[name][r["Counter_Name"]]
                d[key] = d.get(key, 0.0) + float(r["Counter_Value"])
    durations: dict = {}
    if trace_csv:
        with open(trace_csv, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"].replace("mh::(anonymous namespace)::", "").replace("void ", "")
                durations.setdefault(name.split("(")[0], []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    out = {}
    for name, counters in sorted(vals.items()):
        row = {c: round(statistics.mean(v.values()), 1) for c, v in counters.items()}
        row["dispatches"] = max(len(v) for v in counters.values())
        if "TCC_EA0_RDREQ_DRAM_sum" in row and row.get("TCC_EA0_RDREQ_sum"):
            row["dram_read_share"] = round(row["TCC_EA0_RDREQ_DRAM_sum"] / row["TCC_EA0_RDREQ_sum"], 4)
        if "SQ_VALU_MFMA_BUSY_CYCLES" in row and row.get("GRBM_GUI_ACTIVE"):
            row["mfma_util"] = round(row["SQ_VALU_MFMA_BUSY_CYCLES"] / (row["GRBM_GUI_ACTIVE"] * 1024), 5)
        if "SQ_INSTS_VALU_MFMA_MOPS_I8" in row and durations.get(name):
            us = statistics.mean(durations[name])
            ops = row["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512
            row["avg_us"] = round(us, 3)
            row["int8_tops"] = round(ops / (us * 1e-6) / 1e12, 2)
            row["int8_frac_of_5pops"] = round(ops / (us * 1e-6) / INT8_PEAK, 5)
        out[name] = row
    return out


def _short(name: str) -> str:
    return name.replace("mh::(anonymous namespace)::", "").replace("void ", "").split("(")[0]


def stats_table(stats_csv: str, batches: int) -> str:
    """Markdown table of a rocprofv3 --stats kernel_stats.csv."""
    with open(stats_csv, newline="") as f:
        rows = list(csv.DictReader(f))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    out = ["| kernel | calls | calls / batch | avg us | min us | max us | total ms | % |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {int(r['Calls']) / batches:.1f} | "
                   f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                   f"{float(r['Percentage']):.1f} |")
    out.append(f"\nTotal kernel time {tot / 1e6:.3f} ms over {batches} batches = "
               f"{tot / 1e6 / batches:.3f} ms per batch.")
    return "\n".join(out)


def stats_json(stats_csv: str, batches: int) -> dict:
    """Per-kernel calls and average traced duration of a rocprofv3 --stats
    kernel_stats.csv, for bench.py to set beside its event-timed averages."""
    with open(stats_csv, newline="") as f:
        rows = list(csv.DictReader(f))
    return {"source": "rocprofv3 --kernel-trace --stats", "batches": batches,
            "kernels": {_short(r["Name"]): {"calls": int(r["Calls"]),
                                            "avg_us": round(float(r["AverageNs"]) / 1e3, 4)}
                        for r in rows}}


def step_breakdown(trace_csv: str, steps_per_batch: int, batches: int, rows_at: list[int],
                   first_batch: int = 0) -> str:
    """Per decode step of a bench.py kernel trace: the kernels in launch order
    and their average durations, grouped by the number of active rows.  A
    step ends with k_finalize; the encoder's kernels are dropped."""
    with open(trace_csv, newline="") as f:
        ks = [( _short(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
              for r in csv.DictReader(f)]
    ks.sort(key=lambda k: k[1])
    steps, cur = [], []
    for k in ks:
        if k[0].startswith("__amd"):
            continue
        cur.append(k)
        if k[0].startswith("k_finalize"):
            steps.append(cur)
            cur = []
    enc = ("k_gemm_tile", "k_attn_tiles", "k_seq_tiles", "k_embed", "k_quantize_rows_v4<2>")
    groups = [(1, 1), (2, 4), (5, 8), (9, 16), (17, 32), (33, 64), (65, 128), (129, 256), (257, 4096)]
    agg: dict = {}
    for b in range(first_batch, first_batch + batches):
        for t in range(steps_per_batch):
            st = steps[b * steps_per_batch + t]
            if t == 0:  # the encoder runs before step 0
                i = max(j for j, k in enumerate(st) if k[0].startswith(enc)) + 1 if any(
                    k[0].startswith(enc) for k in st) else 0
                st = st[i:]
            g = next(g for g in groups if g[0] <= rows_at[t] <= g[1])
            a = agg.setdefault(g, {"steps": 0, "sum": 0.0, "kernels": {}})
            a["steps"] += 1
            a["sum"] += sum(k[2] - k[1] for k in st) / 1000.0
            for i, k in enumerate(st):
                a["kernels"].setdefault((i, k[0]), []).append((k[2] - k[1]) / 1000.0)
    out = []
    for g in groups:
        if g not in agg:
            continue
        a = agg[g]
        label = f"{g[0]}" if g[0] == g[1] else f"{g[0]}-{g[1]}"
        out.append(f"\n**{label} active rows** ({a['steps']} steps; kernel time per step "
                   f"{a['sum'] / a['steps']:.1f} us)\n")
        out.append("| # | kernel | avg us | launches |")
        out.append("|---:|---|---:|---:|")
        for (i, name), d in sorted(a["kernels"].items()):
            out.append(f"| {i} | `{name}` | {statistics.mean(d):.2f} | {len(d)} |")
    return "\n".join(out)


def _mfma_ops_per_dispatch(counter_csv: str) -> list:
    """int8 MFMA operations (SQ_INSTS_VALU_MFMA_MOPS_I8 x 512) of every
    marian-hip dispatch of a rocprofv3 --pmc run, in dispatch order."""
    per: dict = {}
    with open(counter_csv, newline="") as f:
        for r in csv.DictReader(f):
            if "mh::" not in r["Kernel_Name"] or r["Counter_Name"] != "SQ_INSTS_VALU_MFMA_MOPS_I8":
                continue
            d = int(r.get("Dispatch_Id") or r.get("Correlation_Id"))
            per[d] = per.get(d, 0.0) + float(r["Counter_Value"])
    return [per[d] * 512 for d in sorted(per)]


def summarize(run_path: str, trace_path: str, counter_csv: str | None = None) -> str:
    """The op sweep's table from the run's case list and a kernel trace of
    the same command; with the counter file of a `--pmc
    SQ_INSTS_VALU_MFMA_MOPS_I8` run of it, also the int8 operations the
    matrix cores executed per call and the fraction of the dense peak they
    make at the traced time (the counted operations include the tiles' zero
    padding past M and N)."""
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
    ops = _mfma_ops_per_dispatch(counter_csv) if counter_csv else None
    if ops is not None and len(ops) != need:
        raise SystemExit(f"counter file holds {len(ops)} marian-hip dispatches, the run made {need}")
    head = "| case | kernels | median us / call | algorithmic MB | GB/s | frac of 8 TB/s | int8 MFMA frac |"
    rule = "|---|---|---:|---:|---:|---:|---:|"
    if ops is not None:
        head += " counted int8 GOP / call | counted MFMA frac |"
        rule += "---:|---:|"
    out = [head, rule]
    i = 0
    for c in spec["cases"]:
        per_call, per_ops = [], []
        names = set()
        for _ in range(c["calls"]):
            ks = rows[i:i + c["kernels_per_call"]]
            if ops is not None:
                per_ops.append(sum(ops[i:i + c["kernels_per_call"]]))
            i += c["kernels_per_call"]
            per_call.append(sum(e - s for s, e, _ in ks) / 1000.0)
            names.update(n.replace("mh::(anonymous namespace)::", "").replace("void ", "").split("(")[0]
                         for _, _, n in ks)
        us = statistics.median(per_call[1:] if len(per_call) > 1 else per_call)
        gbs = c["bytes"] / (us * 1e-6) / 1e9
        mf = c["flops"] / (us * 1e-6) / INT8_PEAK if c["kind"] == "gemm" else float("nan")
        line = (f"| {c['label']} | {', '.join(sorted(names))} | {us:.2f} | {c['bytes'] / 1e6:.3f} | "
                f"{gbs:.0f} | {gbs * 1e9 / HBM_PEAK:.3f} | "
                + (f"{mf:.4f} |" if c["kind"] == "gemm" else "- |"))
        if ops is not None:
            if c["kind"] == "gemm":
                o = statistics.median(per_ops)
                line += f" {o / 1e9:.3f} | {o / (us * 1e-6) / INT8_PEAK:.4f} |"
            else:
                line += " - | - |"
        out.append(line)
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
    s.add_argument("--counters", default=None,
                   help="counter_collection.csv of a --pmc SQ_INSTS_VALU_MFMA_MOPS_I8 run of the same command")
    c = sub.add_parser("copy")
    c.add_argument("--mb", type=int, default=64)
    c.add_argument("--reps", type=int, default=5)
    mr = sub.add_parser("rates", help="the runtime's fill and copy rates (events around the calls)")
    mr.add_argument("--mb", type=int, default=512)
    mr.add_argument("--reps", type=int, default=10)
    pm = sub.add_parser("pmc")
    pm.add_argument("fetch_csv")
    pm.add_argument("write_csv")
    pm.add_argument("copy_fetch_csv")
    pm.add_argument("copy_write_csv")
    pm.add_argument("--copy-mb", type=int, default=64)
    pm.add_argument("--workload", default="64-sentence ragged greedy batch (bench.py --steps 2 --warmup 1 "
                                          "--no-cpu-baseline: 5 translations)",
                    help="what the counted command ran")
    st = sub.add_parser("stats")
    st.add_argument("stats_csv")
    st.add_argument("--batches", type=int, required=True)
    st.add_argument("--json", action="store_true", help="per-kernel calls and averages as JSON")
    sb = sub.add_parser("steps", help="per-step kernel breakdown of a bench.py trace")
    sb.add_argument("trace_csv")
    sb.add_argument("--batches", type=int, default=6, help="untimed-event batches at the start")
    sb.add_argument("--workload", choices=["ragged", "stress"], default="ragged",
                    help="the bench.py workload the trace ran (its forced stops give the row counts)")
    cc = sub.add_parser("counters")
    cc.add_argument("csv", nargs="+")
    cc.add_argument("--trace", default=None)
    a = ap.parse_args(argv)
    if a.cmd == "run":
        run(a.out, a.reps)
    elif a.cmd == "copy":
        copy_calibration(a.mb, a.reps)
    elif a.cmd == "rates":
        print(json.dumps(memory_rates(a.mb, a.reps)))
    elif a.cmd == "pmc":
        print(json.dumps(pmc_summary(a.fetch_csv, a.write_csv, a.copy_fetch_csv, a.copy_write_csv,
                                     a.copy_mb, a.workload), indent=1))
    elif a.cmd == "stats":
        print(json.dumps(stats_json(a.stats_csv, a.batches), indent=1) if a.json
              else stats_table(a.stats_csv, a.batches))
    elif a.cmd == "steps":
        pkg = _load_package()
        b = pkg.ragged_batch() if a.workload == "ragged" else pkg.stress_batch()
        lim = b.max_output_tokens.astype(np.int64)
        n = int(lim.max())
        print(step_breakdown(a.trace_csv, n, a.batches, [int((lim > t).sum()) for t in range(n)]))
    elif a.cmd == "counters":
        print(json.dumps(counter_summary(a.csv, a.trace), indent=1))
    else:
        print(summarize(a.run_json, a.trace_csv, a.counters))
    return 0


if __name__ == "__main__":
    sys.exit(main())
