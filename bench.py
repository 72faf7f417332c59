#!/usr/bin/env python3
"""Benchmark of the marian-hip Q8 greedy translation path on one MI355X.

Default workload: the 64-sentence ragged batch (lengths ~ lognormal(3.0, 0.5)
clipped to [5, 128], forced stops ~U[0.8 L, 1.5 L + 10]) on the seeded
6-encoder / 2-decoder, d=512 Transformer.  A "step" is one greedy translation
of the whole batch.  `value` = generated target tokens / device time from
packed inputs resident in HBM to generated tokens in host memory.

Also reported on the same line: p50 sentence completion latency, the decode
step time by active-row count, the roofline of the workload's dominant kernel
(the kernel family with the most event-timed device time: on the default
batch the decoder attention block, LayerNorm or embedding + head projection +
attention; on the stress batch the decode attention kernel over the fp32 K/V
rows), the roofline of the vocabulary projection + fused argmax (the decode
GEMM with the largest weight stream), both timed with HIP events that each
launch's own dispatch records on the engine's stream, and the CPU baseline
(the oracle's reference-schedule port, timed on this host's cores).  For
information, `reference_ssru` gives the same batch through the reference's
own graph (`--workload reference-ssru` prints its full line).

`--workload batch-sweep` measures batches of 1 to 256 sentences drawn from the
default batch's distribution and derives the HIP worker's scheduler settings
from them.
"""

from __future__ import annotations

import argparse
import json
import multiprocessing as mp
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "target tokens/sec, 64-sentence ragged greedy batch, 1 MI355X; p50 request latency"


def load():
    import __graft_entry__ as ge

    return ge.load_package()


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's reference-schedule port (padded sub-batches,
# all-rows decode, AVX2 madd GEMM, scalar scoring), 4 threads per process, one
# process per 4 cores.  Runs before anything touches the GPU.
# ---------------------------------------------------------------------------
_CPU_STATE = {}


def _reference_sub_batches(lengths, cell_cap=65536, batch_cap=256):
    """Input-order packing under batch * Lmax^2 <= cell_cap (backend.rs:206-315)."""
    batches, cur, lmax = [], [], 0
    for i, L in enumerate(lengths):
        nl = max(lmax, int(L))
        if cur and ((len(cur) + 1) * nl * nl > cell_cap or len(cur) + 1 > batch_cap):
            batches.append(cur)
            cur, nl = [], int(L)
        cur.append(i)
        lmax = nl
    if cur:
        batches.append(cur)
    return batches


def _cpu_worker(rows):
    """One process's share of the batch, in the reference's padded
    sub-batches, translated by _CPU_STATE["run"](sub_batch, batch_rows)."""
    run, batch = _CPU_STATE["run"], _CPU_STATE["batch"]
    sub = batch.subset(rows)
    t0 = time.perf_counter()
    done_ms, ntok = [], 0
    for part in _reference_sub_batches(sub.lengths):
        out = run(sub.subset(part), [rows[i] for i in part])
        ntok += sum(map(len, out))
        t = (time.perf_counter() - t0) * 1000.0
        done_ms += [t] * len(part)
    return ntok, time.perf_counter() - t0, done_ms


def _reference_schedule_port(batch, cores: int, threads: int, run):
    """The batch spread over cores // threads processes (greedy partition by
    expected work: source plus forced output length), each running `run` on
    its padded sub-batches with `threads` threads.  Returns the generated
    tokens, the slowest process's wall time, the sentences' completion times
    and the process count."""
    procs = max(1, cores // threads)
    lens = batch.lengths
    work = [(int(lens[i]) + int(batch.max_output_tokens[i]), i) for i in range(len(lens))]
    parts = [[] for _ in range(procs)]
    load_ = [0] * procs
    for w, i in sorted(work, reverse=True):
        j = int(np.argmin(load_))
        parts[j].append(i)
        load_[j] += w
    parts = [sorted(p) for p in parts if p]
    _CPU_STATE.update(run=run, batch=batch)
    ctx = mp.get_context("fork")
    with ctx.Pool(len(parts)) as pool:
        res = pool.map(_cpu_worker, parts)
    return (sum(r[0] for r in res), max(r[1] for r in res), [t for r in res for t in r[2]],
            len(parts))


def host_info(cores_used: int) -> dict:
    """The CPU the baseline ran on: visible cores, model, and the oracle's compiler."""
    import __graft_entry__ as ge

    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"nproc": usable, "cpu_count": os.cpu_count(), "cpu_model": model,
            "cores_used": cores_used, "compiler": ge.load_oracle().build_info()}


def cpu_baseline(pkg, model, batch, cores: int, threads: int = 4):
    import __graft_entry__ as ge

    orc = ge.load_oracle()
    om = orc.OracleModel(model)

    def run(b, _rows):
        return orc.translate(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags,
                             threads=threads, schedule="reference")

    tokens, wall, lat, nproc = _reference_schedule_port(batch, cores, threads, run)
    lens = batch.lengths
    return {
        "value": round(tokens / wall, 2),
        "unit": "tokens/s",
        "cores": nproc * threads,
        "kind": "port",
        "sample": (f"the full {len(lens)}-sentence batch ({tokens} target tokens) on "
                   f"{nproc} processes x {threads} threads; reference schedule: padded "
                   "sub-batches (batch*Lmax^2 <= 65536), all rows every step, AVX2 madd "
                   "GEMM, scalar output scoring; generation caps lifted as on the GPU"),
        "p50_ms": round(statistics.median(lat), 2),
        "wall_s": round(wall, 3),
    }


# ---------------------------------------------------------------------------
# GPU leg
# ---------------------------------------------------------------------------
# Steps with at most this many rows build the last residual LayerNorm inside
# the vocabulary kernel (kVocabLnMaxRows in csrc/kernels.h).
VOCAB_LN_MAX_ROWS = 4


def vocab_bytes(V, K, rows):
    """Algorithmic bytes of one vocabulary launch over `rows` active rows:
    int8 weights + fp32 multipliers + fp32 bias + the 8-byte argmax partial
    per row and 128-column workgroup + the rows: int8 activations and fp32
    row multipliers, or, on steps that build the LayerNorm in the kernel, the
    fp32 sublayer output and residual rows and the fp32 scale and bias."""
    groups = (V + 127) // 128
    row_in = rows * 8 * K + 8 * K if rows <= VOCAB_LN_MAX_ROWS else rows * (K + 4)
    return V * K + 8 * V + rows * 8 * groups + row_in


# Workloads of the bench line: (config name, profile tag, batch generator).
WORKLOADS = {
    "ragged": ("64-sentence ragged greedy batch", "ragged64", "ragged_batch"),
    "stress": ("256-item scheduler-stress batch", "stress256", "stress_batch"),
    "single": ("single sentence, 24 tokens, 32 steps", "single", "single_sentence_batch"),
}


def profile_path(tag, kind):
    """profiles/decode_kernels_<tag>_<kind>.json: the rocprofv3 summaries of
    this workload's bench command (kind "stats": --kernel-trace --stats;
    "traffic": FETCH_SIZE / WRITE_SIZE)."""
    return ROOT / "profiles" / f"decode_kernels_{tag}_{kind}.json"


def _profile_kernels(tag, kind):
    try:
        return json.loads(profile_path(tag, kind).read_text())["kernels"]
    except (OSError, ValueError, KeyError):
        return None


def measured_traffic(prefix, tag):
    """HBM-side bytes per dispatch (fetched + written) of the kernels whose
    name starts with `prefix`, dispatch-weighted, from this workload's
    FETCH_SIZE / WRITE_SIZE rocprofv3 runs summarized in profiles/
    (copy-calibrated); None when no such profile of this workload exists."""
    kernels = _profile_kernels(tag, "traffic")
    if not kernels:
        return None
    ks = [v for k, v in kernels.items() if k.startswith(prefix)]
    n = sum(v["dispatches"] for v in ks)
    if not n:
        return None
    return round(sum((v["fetch_bytes_per_dispatch"] + v["write_bytes_per_dispatch"]) * v["dispatches"]
                     for v in ks) / n)


def traced_launch_us(prefix, tag):
    """Average traced duration (us) of the kernels whose name starts with
    `prefix`, call-weighted, from the rocprofv3 --kernel-trace --stats run of
    this workload summarized in profiles/; None without one."""
    kernels = _profile_kernels(tag, "stats")
    if not kernels:
        return None
    ks = [v for k, v in kernels.items() if k.startswith(prefix)]
    n = sum(v["calls"] for v in ks)
    return round(sum(v["avg_us"] * v["calls"] for v in ks) / n, 4) if n else None


def traced_fields(algo_bytes_per_launch, prefix, tag):
    us = traced_launch_us(prefix, tag)
    if not us:
        return {"traced_avg_launch_us": None, "traced_achieved": None, "traced_frac": None,
                "traced_source": None}
    gbs = algo_bytes_per_launch / (us * 1e-6) / 1e9
    return {"traced_avg_launch_us": us, "traced_achieved": round(gbs, 1),
            "traced_frac": round(gbs / HBM_PEAK_GBS, 4),
            "traced_source": f"profiles/{profile_path(tag, 'stats').name} (rocprofv3 --kernel-trace --stats)"}


def traffic_fields(prefix, tag):
    t = measured_traffic(prefix, tag)
    return {"traffic": t,
            "traffic_source": (f"profiles/{profile_path(tag, 'traffic').name} (rocprofv3 FETCH_SIZE + "
                               "WRITE_SIZE, bytes per launch)") if t is not None else None}


def block_bytes(kind, step, layer, src_lens, d, heads):
    """Algorithmic bytes of one attention-block launch at decode step `step`
    over the active rows whose source lengths are `src_lens`:
      head projection weights (int8) + their fp32 multipliers and biases;
      the input rows (decoder layer 0 self-attention: the previous token's
      int8 embedding row, its multiplier and the token id, plus the shared
      fp32 position row; otherwise the two fp32 rows y and r of the residual
      LayerNorm plus gamma and beta);
      keys and values read (self: `step` cached rows; cross: the sentence's
      encoder rows), fp32, 64 x heads = d wide;
      writes: the fp32 attention output, the per-head maxima, the fp32 input
      row (the residual stream) and, for self-attention, this step's key and
      value rows; plus the per-row metadata (first key row, key count)."""
    m = len(src_lens)
    out = m * (4 * d + 4 * heads + 4 * d)
    if kind == 1:  # self-attention block
        w = 3 * d * (d + 8)
        rows_in = m * (d + 8) + 4 * d if layer == 0 else m * 8 * d + 8 * d
        keys = m * 2 * step * d * 4
        out += m * (8 * d + 8)
    else:  # cross-attention block
        w = d * (d + 8)
        rows_in = m * 8 * d + 8 * d
        keys = 8 * d * int(np.sum(src_lens))
        out += m * 12
    return w + rows_in + keys + out


def attn_bytes(kind, step, src_lens, d, heads):
    """Algorithmic bytes of one decode attention launch (k_attention or
    k_attn_long, the steps the blocks do not cover) over the active rows whose source lengths
    are `src_lens`: per row the fp32 query, the keys and values it reads
    (self: the `step` + 1 cached rows, this step's written by the projection
    before; cross: the sentence's encoder rows), d floats each, the fp32
    output, the per-head maxima and the row's key metadata."""
    m = len(src_lens)
    keys = m * (step + 1) if kind == 3 else int(np.sum(src_lens))
    return m * (4 * d + 4 * d + 4 * heads + 8) + 8 * d * keys + (m * 4 if kind == 4 else 0)


# Kernel families timed by their own dispatches (marian_hip_last_kernel_trace
# kinds), the prefix of their kernels' names in the rocprof summaries, and
# what the roofline calls them.
FAMILIES = {
    "vocab": ((0,), "k_vocab_argmax", "k_vocab_argmax (vocab projection + bias + mask + argmax partials)"),
    "block": ((1, 2), "k_attn_block", "k_attn_block (LayerNorm/embedding + head projection + attention)"),
    "attention": ((3, 4), ("k_attention", "k_attn_long"),
                  "k_attention / k_attn_long (decode self- and cross-attention over fp32 K/V rows)"),
}

# Active-row buckets of the step table.
ROW_BUCKETS = [(1, 1), (2, 4), (5, 8), (9, 16), (17, 32), (33, 64), (65, 128), (129, 256), (257, 4096)]


def step_table(rows, step_ms, encoder_ms):
    """Decode step time by active rows, from one translation with an event at
    the end of every step (those events add about 2% of device time)."""
    rows = np.asarray(rows, np.int64)
    ends = np.asarray(step_ms, np.float64)
    dur = np.diff(np.concatenate([[encoder_ms], ends]))
    total = float(dur.sum())
    out = []
    for lo, hi in ROW_BUCKETS:
        sel = (rows >= lo) & (rows <= hi)
        if not sel.any():
            continue
        out.append({"rows": f"{lo}" if lo == hi else f"{lo}-{hi}", "steps": int(sel.sum()),
                    "us_per_step": round(float(dur[sel].mean()) * 1000.0, 1),
                    "share_of_decode": round(float(dur[sel].sum()) / total, 3)})
    return out


def run_translate_bench(pkg, model, batch, steps, warmup, extra_passes=2):
    """`warmup` untimed batches, then `steps` timed batches (device events at
    the batch start, after the encoder and after the decode loop only), then
    `extra_passes` batches with an event at the end of every decode step (the
    sentence completion latencies; these events add about 2% of device time)
    and `extra_passes` batches whose vocabulary and attention-block launches
    record events from their own dispatches (several microseconds of device
    time per launch).  The batch, the launches and their row counts are the
    same in every pass."""
    eng = pkg.HipEngine(model, limits=batch.limits)
    for _ in range(warmup):
        eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens, batch.flags)
    H = model.geometry.heads
    V, K = model.geometry.vocab, model.geometry.dim
    src_len = np.asarray(batch.lengths, np.int64)
    dev_ms, wall_ms, lat, enc_ms, dec_ms, n_steps = [], [], [], [], [], []
    ntok = None
    eng.set_timing(0)
    for _ in range(steps):
        t0 = time.perf_counter()
        out = eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens,
                                      batch.flags)
        wall_ms.append((time.perf_counter() - t0) * 1000.0)
        st = eng.last_stats()
        dev_ms.append(st["total_ms"])
        enc_ms.append(st["encoder_ms"])
        dec_ms.append(st["decode_ms"])
        n_steps.append(st["decode_steps"])
        ntok = int(out.tokens.size)

    eng.set_timing(eng.TIME_STEPS)
    table = None
    for _ in range(extra_passes):
        out = eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens,
                                      batch.flags)
        rows, step_end = eng.last_step_trace()
        # A sentence that produced c tokens ran decode steps 0..c-1.
        counts = np.diff(out.offsets.astype(np.int64))
        lat += [float(step_end[c - 1]) for c in counts if c > 0]
        if table is None:
            table = step_table(rows, step_end, eng.last_stats()["encoder_ms"])

    fam = {k: dict(us=0.0, launches=0, algo=0.0) for k in FAMILIES}
    kind_family = {kind: k for k, (kinds, _, _) in FAMILIES.items() for kind in kinds}
    eng.set_timing(eng.TIME_KERNELS)
    for _ in range(extra_passes):
        out = eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens,
                                      batch.flags)
        rows, _ = eng.last_step_trace()
        counts = np.diff(out.offsets.astype(np.int64))
        kt = eng.last_kernel_trace()
        for kind, t, layer, us in zip(kt["kind"], kt["step"], kt["layer"], kt["us"]):
            active = src_len[counts > t]
            if len(active) != int(rows[t]):
                raise RuntimeError(f"step {t}: {len(active)} sentences active, the engine ran {rows[t]}")
            f = fam[kind_family[int(kind)]]
            f["us"] += float(us)
            f["launches"] += 1
            if kind == eng.KERNEL_VOCAB:
                f["algo"] += vocab_bytes(V, K, len(active))
            elif kind in (eng.KERNEL_SELF_BLOCK, eng.KERNEL_CROSS_BLOCK):
                f["algo"] += block_bytes(int(kind), int(t), int(layer), active, K, H)
            else:
                f["algo"] += attn_bytes(int(kind), int(t), active, K, H)
    eng.set_timing(0)
    info = eng.info()
    eng.close()
    return dict(dev_ms=dev_ms, wall_ms=wall_ms, lat=lat, ntok=ntok, info=info, families=fam,
                enc_ms=enc_ms, dec_ms=dec_ms, n_steps=n_steps, step_table=table, rows=out.rows())


def fast_mode(pkg, model, batch, steps, warmup, exact_rows, probe_steps=(0, 20, 60)):
    """The same batch with MARIAN_HIP_FLAG_FAST_REDUCTIONS (the decoder's
    LayerNorm and softmax sums in the tree order): tokens/s over `steps`
    timed translations, how many sentences equal the exact mode's, and the
    relative L2 difference of the logits from the exact mode's at a few
    decode steps (over the rows active there, masked ids excluded)."""
    flags = batch.flags | pkg.FLAG_FAST_REDUCTIONS
    eng = pkg.HipEngine(model, limits=batch.limits)
    for _ in range(warmup):
        eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens, flags)
    ms, rows = [], None
    for _ in range(steps):
        out = eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens, flags)
        ms.append(eng.last_stats()["total_ms"])
        rows = out.rows()
    same = sum(a == b for a, b in zip(rows, exact_rows))
    rel = []
    for step in probe_steps:
        lim = np.minimum(batch.max_output_tokens.astype(np.int64), step + 1).astype(np.uint32)
        _, _, lf, act = eng.translate_probe(batch.tokens, batch.offsets, lim, flags, probe_step=step)
        _, _, le, _ = eng.translate_probe(batch.tokens, batch.offsets, lim, batch.flags, probe_step=step)
        if not act.any():
            continue
        f, e = lf[act], le[act]
        fin = np.isfinite(e)
        rel.append(float(np.linalg.norm(np.where(fin, f, 0.0) - np.where(fin, e, 0.0)) /
                         np.linalg.norm(np.where(fin, e, 0.0))))
    eng.close()
    ntok = sum(map(len, rows))
    m = statistics.mean(ms)
    return {"value": round(ntok / (m / 1000.0), 1), "unit": "tokens/s", "ms_per_step": round(m, 4),
            "identical_sentences": f"{same}/{len(rows)}",
            "max_logit_rel_l2": round(max(rel), 6) if rel else None,
            "probe_steps": list(probe_steps),
            "note": "opt-in MARIAN_HIP_FLAG_FAST_REDUCTIONS: the decoder's LayerNorm sums and softmax "
                    "denominators as lane partials + xor butterfly (bit-exact with the oracle's restatement "
                    "of that order); compared here with the exact mode of the same build"}


def roofline_of(family, f, tag, timing_note):
    """The roofline object of one kernel family from its event-timed launches."""
    _, prefix, name = FAMILIES[family]
    n = max(1, f["launches"])
    avg_us = f["us"] / n
    per_launch = f["algo"] / n
    achieved = per_launch / max(avg_us * 1e-6, 1e-12) / 1e9 if f["launches"] else 0.0
    return {
        "kernel": name,
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "avg_launch_us": round(avg_us, 3),
        "algorithmic_bytes_per_launch": round(per_launch),
        "launches": f["launches"],
        "timing": timing_note,
        **traced_fields(per_launch, prefix, tag),
        **traffic_fields(prefix, tag),
    }


def ssru_cpu_baseline(model, batch, cand, coff, cores: int, threads: int = 4):
    """The oracle's Transformer-SSRU restatement on the reference x86
    schedule over the same batch and shortlist: one process per `threads`
    cores, each translating its sentences in the reference's padded
    sub-batches (every row decoded every step, keys masked by length, u8 AVX2
    GEMMs split over `threads` threads, scalar scoring of the unfinished rows
    over their candidates), timed on this host."""
    import __graft_entry__ as ge

    orc = ge.load_oracle()
    om = orc.OracleSsruModel(model)
    lists = [np.asarray(cand[coff[b]:coff[b + 1]], np.uint32) for b in range(len(coff) - 1)]

    def run(b, rows):
        c = np.concatenate([lists[r] for r in rows])
        co = np.zeros(len(rows) + 1, np.uint32)
        co[1:] = np.cumsum([lists[r].size for r in rows])
        return orc.translate_ssru(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, b.flags,
                                  candidates=c, candidate_offsets=co, threads=threads,
                                  schedule="reference")

    tokens, wall, lat, nproc = _reference_schedule_port(batch, cores, threads, run)
    return {
        "value": round(tokens / wall, 2),
        "unit": "tokens/s",
        "cores": nproc * threads,
        "kind": "port",
        "sample": (f"the full {len(batch.lengths)}-sentence batch ({tokens} target tokens) with the same "
                   f"shortlist on {nproc} processes x {threads} threads; reference schedule: padded "
                   "sub-batches (batch*Lmax^2 <= 65536), all rows every step, AVX2 madd GEMM, scalar "
                   "shortlist scoring; generation caps lifted as on the GPU"),
        "p50_ms": round(statistics.median(lat), 2),
        "wall_s": round(wall, 3),
        "host": host_info(nproc * threads),
    }


def ssru_bench(pkg, args):
    print(json.dumps(ssru_line(pkg, args)), flush=True)
    return 0


def ssru_line(pkg, args):
    """The reference's own graph (Transformer encoder + 4 SSRU decoder layers,
    d = 384 with 8 heads of 48, FFN 1536, 32000-id vocabularies, static
    per-tensor multipliers; seeded random weights) on the same 64-sentence
    ragged batch, scored over lexical-shortlist candidates (the reference's
    production mode) and over the full vocabulary.  Informational: the
    headline metric is the default workload's."""
    import importlib
    sl = importlib.import_module(pkg.__name__ + ".shortlist")
    g = pkg.SsruGeometry()
    model = pkg.seeded_ssru_model(geometry=g)
    batch = pkg.ragged_batch()
    # A synthetic shortlist: 40 targets per source id, ids below 100 always allowed.
    rng = np.random.Generator(np.random.PCG64(11))
    per = 40
    targets = rng.integers(0, g.target_vocab, size=per * g.source_vocab).astype(np.uint32)
    shortlist = sl.LexicalShortlist.from_bytes(
        sl.LexicalShortlist.to_bytes(100, np.arange(g.source_vocab + 1, dtype=np.uint64) * per, targets),
        g.source_vocab, g.target_vocab)
    offs = batch.offsets
    cand, coff, maxc = sl.pack_candidates([shortlist.candidates(batch.tokens[offs[b]:offs[b + 1]])
                                           for b in range(len(offs) - 1)])
    cpu = None
    if not args.no_cpu_baseline:
        cpu = ssru_cpu_baseline(model, batch, cand, coff, args.cpu_cores)
    eng = pkg.HipEngine(model, limits=batch.limits)

    def run(with_shortlist):
        kw = dict(candidates=cand, candidate_offsets=coff) if with_shortlist else {}
        for _ in range(args.warmup):
            eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens, batch.flags, **kw)
        ms, ntok = [], 0
        for _ in range(args.steps):
            out = eng.translate_token_ids(batch.tokens, batch.offsets, batch.max_output_tokens,
                                          batch.flags, **kw)
            ms.append(eng.last_stats()["total_ms"])
            ntok = int(out.tokens.size)
        st = eng.last_stats()
        return ntok, statistics.mean(ms), st

    ntok, ms, st = run(True)
    ntok_f, ms_f, _ = run(False)
    line = {
        "metric": "target tokens/sec, 64-sentence ragged greedy batch, reference Transformer-SSRU graph, 1 MI355X",
        "value": round(ntok / (ms / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init weights, seeded token ids, synthetic shortlist)",
        "config": {"workload": "64-sentence ragged greedy batch, shortlist scoring",
                   "model": "transformer-ssru-q8 6 enc / 4 SSRU dec, d=384, 8 heads of 48, ffn 1536, "
                            "vocab 32000/32000, static per-tensor multipliers",
                   "shortlist": f"{per} targets per source id, first 100 ids; longest list {maxc}",
                   "target_tokens": ntok, "decode_steps": st["decode_steps"]},
        "encoder_ms": round(st["encoder_ms"], 4),
        "decode_ms": round(st["decode_ms"], 4),
        "full_vocabulary": {"value": round(ntok_f / (ms_f / 1000.0), 1), "ms_per_step": round(ms_f, 4),
                            "target_tokens": ntok_f},
        "device": eng.info()["device"],
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
        line["speedup_vs_cpu"] = round(line["value"] / cpu["value"], 1)
    eng.close()
    return line


def batch_sweep(pkg, args):
    """Batches of 1 to 256 sentences drawn from the default batch's
    distribution (lognormal(3.0, 0.5) lengths clipped to [5, 128], forced
    stops ~U[0.8 L, 1.5 L + 10]), each translated `steps` times after a
    warmup: device time per batch, target tokens/s, and the sentences'
    completion latencies from the batch start (one pass with step events).
    The HIP worker's scheduler settings follow from the table (`scheduler`)."""
    import importlib
    sched = importlib.import_module(pkg.__name__ + ".scheduler")
    model = pkg.seeded_model()
    sizes = [int(x) for x in args.sizes.split(",")]
    draws = 4  # batches drawn per size: a batch lasts as long as its longest sentence
    batches = {n: [pkg.ragged_batch(seed=1000 + 10 * n + k, n=n) for k in range(draws)] for n in sizes}
    allb = [b for bs in batches.values() for b in bs]
    eng = pkg.HipEngine(model, limits=allb[0].limits, capacity=pkg.capacity_for(allb))
    eng.warmup()
    table = []
    for n in sizes:
        ms, ntok, steps, lat, allocs = [], 0, [], [], 0
        for b in batches[n]:
            for _ in range(args.warmup):
                eng.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags)
            for _ in range(args.steps):
                eng.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags)
                st = eng.last_stats()
                ms.append(st["total_ms"])
                allocs += int(st["allocations"])
            steps.append(int(st["decode_steps"]))
            eng.set_timing(eng.TIME_STEPS)
            out = eng.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags)
            _, step_end = eng.last_step_trace()
            eng.set_timing(0)
            counts = np.diff(out.offsets.astype(np.int64))
            lat += [float(step_end[c - 1]) for c in counts if c > 0]
            ntok += int(out.tokens.size)
        bm = statistics.mean(ms)
        table.append({"sentences": n, "draws": draws, "target_tokens": round(ntok / draws, 1),
                      "decode_steps": round(statistics.mean(steps), 1), "batch_ms": round(bm, 3),
                      "tokens_per_s": round(ntok / draws / (bm / 1000.0), 1),
                      "p50_ms": round(float(np.median(lat)), 3),
                      "p90_ms": round(float(np.percentile(lat, 90)), 3),
                      "allocations": allocs})
        print(f"batch-sweep: {n} sentences, {bm:.3f} ms, {ntok / draws / (bm / 1000.0):.0f} tokens/s",
              file=sys.stderr, flush=True)
    info = eng.info()
    eng.close()
    rec = sched.recommend(table)
    line = {
        "metric": "target tokens/sec and p50 sentence latency by batch size, ragged greedy batches, 1 MI355X",
        "value": max(r["tokens_per_s"] for r in table),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init weights, seeded token ids)",
        "config": {"workload": "batches of " + ", ".join(map(str, sizes)) + " sentences drawn like the "
                               "64-sentence ragged batch, 4 draws per size (seeds 1000 + 10 size + k)",
                   "model": "transformer-q8 6 enc / 2 dec, d=512, 8 heads, ffn 2048, vocab 32000"},
        "batch_sweep": table,
        "scheduler": rec,
        "device": info["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=["ragged", "stress", "single", "reference-ssru", "batch-sweep"],
                    default="ragged")
    ap.add_argument("--sizes", default="1,4,16,64,128,256",
                    help="batch-sweep: the batch sizes (sentences)")
    ap.add_argument("--passes", type=int, default=2,
                    help="translations with step events and with launch events (each); 0 skips "
                         "the p50, step table and rooflines (for counter runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fast-mode", action="store_true",
                    help="skip the opt-in fast-reduction mode's line items")
    ap.add_argument("--no-reference-ssru", action="store_true",
                    help="skip the informational Transformer-SSRU run on the default workload")
    ap.add_argument("--cpu-cores", type=int, default=min(16, os.cpu_count() or 4))
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this backend's path needs no collectives and the run "
              "uses a single MI355X (sentences shard across GPUs with no exchange; see "
              "DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    pkg = load()
    if args.workload == "reference-ssru":
        return ssru_bench(pkg, args)
    if args.workload == "batch-sweep":
        return batch_sweep(pkg, args)
    model = pkg.seeded_model()
    workload_name, tag, make = WORKLOADS[args.workload]
    batch = getattr(pkg, make)()

    cpu = None
    if not args.no_cpu_baseline and args.workload == "ragged":
        cpu = cpu_baseline(pkg, model, batch, args.cpu_cores)
        # The same batch under the reference's own limits (length factor 2, at
        # most 256 steps, padded-cell cap): fewer generated tokens per row.
        capped = pkg.synthetic.Batch(batch.name, batch.tokens, batch.offsets,
                                     batch.max_output_tokens, batch.flags,
                                     dict(pkg.REFERENCE_LIMITS))
        cap = cpu_baseline(pkg, model, capped, args.cpu_cores)
        cpu["capped_limits"] = {"value": cap["value"], "unit": "tokens/s", "p50_ms": cap["p50_ms"],
                                "wall_s": cap["wall_s"],
                                "limits": "reference caps: factor 2, 256 steps, batch 256, "
                                          "256 source tokens, 65536 padded cells"}
        cpu["host"] = host_info(cpu["cores"])

    r = run_translate_bench(pkg, model, batch, args.steps, args.warmup, max(0, args.passes))
    ms = statistics.mean(r["dev_ms"])
    value = r["ntok"] / (ms / 1000.0)
    wall = statistics.mean(r["wall_ms"])
    timing = "events recorded by each launch's dispatch, in a separate pass over the same batch"
    fams = r["families"]
    # The roofline names the kernel family with the most event-timed device
    # time on this workload; the vocabulary kernel is the decode GEMM line.
    dominant = max(FAMILIES, key=lambda k: fams[k]["us"])
    line = {
        "metric": METRIC if args.workload == "ragged" else
        f"target tokens/sec, {workload_name}, 1 MI355X; p50 request latency",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init weights, seeded token ids)",
        "config": {
            "workload": workload_name,
            "model": "transformer-q8 6 enc / 2 dec, d=512, 8 heads, ffn 2048, vocab 32000",
            "sentences": int(len(batch.lengths)),
            "source_tokens": int(batch.tokens.size),
            "target_tokens": r["ntok"],
            "decode_steps": int(statistics.median(r["n_steps"])),
            "parallelism": "single GPU",
        },
        "p50_latency_ms": round(statistics.median(r["lat"]), 4) if r["lat"] else None,
        "batch_ms": round(ms, 4),
        "encoder_ms": round(statistics.mean(r["enc_ms"]), 4),
        "decode_ms": round(statistics.mean(r["dec_ms"]), 4),
        "pcie_inclusive_tokens_per_s": round(r["ntok"] / (wall / 1000.0), 1),
        "roofline": roofline_of(dominant, fams[dominant], tag, timing),
        "decode_gemm_roofline": roofline_of("vocab", fams["vocab"], tag, timing),
        # per translation of the batch, from the event-timed passes
        "event_timed_kernel_ms": ({k: round(v["us"] / 1000.0 / args.passes, 3) for k, v in fams.items()}
                                  if args.passes > 0 else None),
        "step_table": r["step_table"],
        "cpu_baseline": cpu,
        "device": r["info"]["device"],
    }
    if not args.no_fast_mode:
        line["fast_reductions"] = fast_mode(pkg, model, batch, args.steps, args.warmup, r["rows"])
    if cpu:
        line["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    if args.workload == "ragged" and not args.no_reference_ssru:
        # The reference's own graph on the same batch, for information.
        sr = ssru_line(pkg, args)
        line["reference_ssru"] = {
            "metric": sr["metric"], "value": sr["value"], "unit": sr["unit"],
            "ms_per_step": sr["ms_per_step"], "config": sr["config"],
            "full_vocabulary": sr["full_vocabulary"],
            "cpu_baseline": ({"value": sr["cpu_baseline"]["value"], "unit": "tokens/s",
                              "cores": sr["cpu_baseline"]["cores"], "kind": "port",
                              "sample": sr["cpu_baseline"]["sample"]} if "cpu_baseline" in sr else None),
        }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
