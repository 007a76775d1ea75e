"""Throughput of the rocm backend's encoder forward pass on one MI355X.

Default workload: the BERT-base-shaped encoder (12 layers, hidden 768, 12
heads, FFN 3072, vocab 30522), weights stored F32 and run in the FASTEST
tier (F16 operands, F32 sums), 64 rows x 512 tokens all live, CLS pooling +
L2. A step is one session run over the batch (pack, embeddings, 12 layers,
pool), with the rows already resident on the device. Prints one JSON line.

The CPU baseline is the oracle (this repository's C++ restatement of the
reference's CPU encoder) on a bounded sample of the same rows, on the host's
cores; the same sample gives the cosine of the GPU's vectors against it.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import turboembed_amd as T  # noqa: E402
from turboembed_amd import seam as S  # noqa: E402
from turboembed_amd import workloads as W  # noqa: E402

PEAK = {"f16": 2.5e15, "bf16": 2.5e15, "f32": 157.3e12, "i8": 5.0e15}   # dense MFMA, MI355X (int8: ops/s)


def kernel_flops(shape, tokens, lengths):
    """Algorithmic FLOPs of one launch of each kernel, by the names the
    session's timing hook reports."""
    H, I = shape.hidden, shape.intermediate
    gated = shape.family == S.TURBO_FAMILY_MODERNBERT
    f = {
        "gemm_qkv": 2.0 * tokens * 3 * H * H,
        "gemm_out": 2.0 * tokens * H * H,
        "gemm_ffn_in": 2.0 * tokens * (2 * I if gated else I) * H,
        "gemm_ffn_out": 2.0 * tokens * H * I,
        "attention": W.attention_flops(shape, lengths) / shape.layers,
    }
    # The out and FFN-out products with the add + LayerNorm in their
    # epilogue: the same products (the norm's few operations a value are not
    # counted).
    f["gemm_out_ln"] = f["gemm_out"]
    f["gemm_ffn_out_ln"] = f["gemm_ffn_out"]
    return f


HBM_PEAK = 8.0e12   # MI355X HBM3E, bytes/s (published)


def busy_union(intervals, names):
    """The time at least one of these kernels' launches was running: the
    union of their (name, start, end) intervals, over every stream."""
    total, end = 0.0, float("-inf")
    for a, b in sorted((a, b) for n, a, b in intervals if n in names):
        if b > end:
            total += b - max(a, end)
            end = b
    return total


def run_slice(items, index, name):
    """The items (kernel dispatches, in order) of the process's run number
    `index`: each run begins with pack_rows_kernel and ends with its pooling
    (what follows, up to the next run, is the bench's own), or None when the
    process ran fewer runs. `name` gives an item's kernel name."""
    starts = [i for i, x in enumerate(items) if "pack_rows_kernel" in name(x)]
    if index >= len(starts):
        return None
    run = items[starts[index]:starts[index + 1] if index + 1 < len(starts) else len(items)]
    ends = [i for i, x in enumerate(run) if "pool_kernel" in name(x)]
    return run[:ends[-1] + 1] if ends else run


def tail_bytes(shape, dtype, tokens, rows, od):
    """Algorithmic HBM bytes of the memory-bound kernels' launches in one
    run, by the timing hook's names: each operand read once and each result
    written once (a table row once per token that reads it).

    embed_ln per token: the word row in F32, the ids (and types), x written
    in F32 (not on post-norm F16 and int8 sessions, whose residual starts in
    the 16-bit rows) and its 16-bit operand copy; off the rotary families the
    position and type rows once a run (they stay in L2). add_layer_norm per
    token: the residual and the product y read, the normalized rows written.
    Post-norm F16 and int8 sessions carry the residual in the 16-bit rows (2
    bytes read and 2 written an element; the last layer's norm also writes F32
    rows, and on int8 every norm feeding a product writes its int8 codes and
    scale); others read and write x in F32 and write the normalized operand
    copy (16-bit, or F32 on a pre-norm F32 session) except on post-norm F32
    sessions and after a pre-norm model's last layer. pool: each pooled
    token's F32 row (one per output row for CLS and LAST), then the output
    rows."""
    H = shape.hidden
    modern = shape.family == S.TURBO_FAMILY_MODERNBERT
    act = 4 if dtype == "f32" else 2
    ysz = 2 if dtype in ("f16", "bf16", "i8") else 4
    res16 = dtype in ("f16", "i8") and not modern
    codes = H + 4 if dtype == "i8" else 0
    # The word row comes from HBM once a token; the position and type rows
    # are few and stay in L2 (counted once a run).
    rotary = shape.rope is not None
    ids = 4 if rotary else 8
    shared = 0 if rotary else (min(shape.seq, shape.positions) + shape.token_types) * 4 * H
    out = {"embed_ln": tokens * (4 * H + ids + (0 if res16 else 4 * H) + (0 if dtype == "f32" else act * H) + codes)
           + shared}
    L = shape.layers
    if modern:
        out["add_layer_norm"] = tokens * ((2 * L - 1) * (8 * H + ysz * H + act * H) + (8 * H + ysz * H))
    elif res16:
        out["add_layer_norm"] = tokens * (2 * L * (4 * H + ysz * H) + 4 * H + (2 * L - 1) * codes)
    else:
        out["add_layer_norm"] = tokens * 2 * L * (8 * H + ysz * H + (0 if dtype == "f32" else act * H))
    pooled = rows if shape.pooling in (S.TURBO_POOLING_CLS, S.TURBO_POOLING_LAST) and not shape.ranges_per_row \
        else tokens
    out["pool"] = pooled * 4 * H + rows * 4 * od
    return out


COPY_PROBE_BYTES = 256 << 20   # the traffic counters' reference copy: read and write this much


def traffic_file(workload):
    return os.path.join(ROOT, "profiles", f"traffic_{workload}.json")


def summarize_pmc(fetch_dir, write_dir, workload, command, bench_log=None):
    """HBM bytes per launch of the GEMM kernel from two rocprofv3 --pmc runs
    of this script with --copy-probe (FETCH_SIZE, then WRITE_SIZE, KiB per
    dispatch), each scaled by what the same counter read for the plain copy
    of COPY_PROBE_BYTES; written to profiles/traffic_<workload>.json and .md.
    With the profiled command's output (bench_log), the dispatches of the
    roofline's whole-batch run alone (the run at its timed_run_index; each
    run's first kernel is pack_rows_kernel), else every GEMM dispatch of the
    command. Also per product: a run launches each layer's products in the
    order QKV, out, FFN-in, FFN-out, so its GEMM dispatches, in dispatch
    order, take those names in turn; each product's algorithmic bytes
    (operands read once, output written once) are for launches over the
    whole batch (or over half of it, the default split, without bench_log)."""
    import csv
    import glob

    index = None
    if bench_log:
        for text in open(bench_log, errors="replace"):
            if text.startswith('{"metric"'):
                index = json.loads(text)["roofline"]["timed_run_index"]

    def per_dispatch(d, counter):
        rows = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        return sorted(rows)

    def run_only(v):
        return v if index is None else run_slice(v, index, lambda x: x[1]) or []

    shape = W.SHAPES[workload]
    H, I = shape.hidden, shape.intermediate
    gated = shape.family == S.TURBO_FAMILY_MODERNBERT
    el = 4 if shape.precision == S.TURBO_PRECISION_EXACT else 2
    # Whole-row batches of the embedding task only (every launch's rows known).
    M = shape.batch * shape.seq // (1 if index is not None else 2) \
        if shape.lengths is None and shape.task == S.TURBO_TASK_EMBED else None
    products = [("qkv", H, 3 * H), ("out", H, H), ("ffn_in", H, (2 if gated else 1) * I), ("ffn_out", I, H)]
    out = {"workload": workload, "command": command, "copy_probe_bytes": COPY_PROBE_BYTES}
    lines = [f"# HBM traffic per launch: {workload}", "", "Commands (from the repository root, one MI355X):", "",
             "```", *command, "```", "",
             "| counter | copy probe reads (KiB/dispatch) | expected KiB | factor | GEMM kernel KiB/dispatch (mean) "
             "| scaled bytes/launch | dispatches |", "|---|---|---|---|---|---|---|"]
    by_product = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        v = per_dispatch(d, counter)
        copy = [x for _, k, x in v if "copy_kernel" in k]
        gemm = [x for _, k, x in run_only(v) if "gemm_" in k and "splitk_reduce" not in k]
        expected = COPY_PROBE_BYTES / 1024.0
        factor = expected / (sum(copy) / len(copy))
        mean = sum(gemm) / len(gemm)
        out[counter] = {"copy_kib": sum(copy) / len(copy), "factor": factor, "gemm_kib": mean,
                        "gemm_bytes": mean * 1024.0 * factor, "dispatches": len(gemm)}
        lines.append(f"| {counter} | {sum(copy) / len(copy):.0f} | {expected:.0f} | {factor:.4f} | {mean:.0f} | "
                     f"{mean * 1024.0 * factor:.4g} | {len(gemm)} |")
        for i, x in enumerate(gemm):
            by_product.setdefault(products[i % 4][0], {}).setdefault(counter, []).append(x * 1024.0 * factor)
    out["traffic_bytes_per_launch"] = out["FETCH_SIZE"]["gemm_bytes"] + out["WRITE_SIZE"]["gemm_bytes"]
    lines += ["", f"Traffic per GEMM launch (fetch + write, scaled): {out['traffic_bytes_per_launch']:.4g} bytes.", ""]
    if M:
        lines += [f"Per product (launches over M = {M} rows; algorithmic: A = M·K and W = N·K read once, the "
                  f"M·N output written once, {el}-byte operands and outputs):", "",
                  "| product | N | K | fetched MB | algorithmic reads MB | ratio | written MB | algorithmic writes MB "
                  "| ratio |", "|---|---|---|---|---|---|---|---|---|"]
        out["products"] = {}
        alg_total = 0.0
        for name, K, N in products:
            f = by_product.get(name, {}).get("FETCH_SIZE", [0.0])
            w = by_product.get(name, {}).get("WRITE_SIZE", [0.0])
            fm, wm = sum(f) / len(f), sum(w) / len(w)
            nout = N // 2 if name == "ffn_in" and gated else N
            ar, aw = (M * K + N * K) * el, M * nout * el
            alg_total += ar + aw
            out["products"][name] = {"fetch_bytes": fm, "write_bytes": wm, "alg_read_bytes": ar, "alg_write_bytes": aw}
            lines.append(f"| {name} | {N} | {K} | {fm / 1e6:.1f} | {ar / 1e6:.1f} | {fm / ar:.2f} | {wm / 1e6:.1f} | "
                         f"{aw / 1e6:.1f} | {wm / aw:.2f} |")
        out["alg_bytes_per_launch"] = alg_total / 4
        lines += ["", f"Algorithmic bytes per launch (mean of the four): {alg_total / 4:.4g}; traffic / algorithmic: "
                  f"{out['traffic_bytes_per_launch'] / (alg_total / 4):.2f}."]
    with open(traffic_file(workload), "w") as f:
        json.dump(out, f, indent=1)
    with open(traffic_file(workload)[:-5] + ".md", "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(out))


def unsplit_rooflines(rows, workload):
    """Lines for a run of full-length rows whose launches each take the whole
    batch (TURBO_ROCM_SPLIT=1, one length, no tuner): each matrix-core
    kernel's achieved rate from its average launch, over the algorithmic
    FLOPs one launch does."""
    import re
    shape = W.SHAPES[workload]
    if (shape.lengths is not None or shape.family == S.TURBO_FAMILY_MODERNBERT or shape.task != S.TURBO_TASK_EMBED
            or shape.compute_dtype or shape.precision != S.TURBO_PRECISION_FASTEST):
        return []
    T, H, I, L = shape.batch * shape.seq, shape.hidden, shape.intermediate, shape.layers
    att = W.attention_flops(shape, [shape.seq] * shape.batch) / L
    # The products by epilogue: 1 Q/K/V, 2 GELU, 6 bias (the out and FFN-out
    # products, one launch each a layer).
    groups = [("Q/K/V product", r"EpiE1E", 2.0 * T * H * 3 * H), ("FFN-in product (GELU)", r"EpiE2E", 2.0 * T * H * I),
              ("attention", r"attention_mfma_kernel", att)]
    peak = PEAK["bf16" if shape.store == "bf16" else "f16"]
    out = ["", "Each launch over the whole batch (full-length rows, one launch a layer per kernel): the main "
           "instantiation of each kernel, its average launch against its algorithmic FLOPs.", "",
           "| kernel | instantiation | calls | average µs | GFLOP a launch | TFLOP/s | of peak |", "|---|---|---|---|---|---|---|"]

    def line(tag, name, calls, us, flops):
        rate = flops / (us * 1e-6)
        out.append(f"| {tag} | {name} | {calls} | {us:.1f} | {flops / 1e9:.1f} | {rate / 1e12:.0f} | "
                   f"{100 * rate / peak:.1f}% |")

    for tag, pat, flops in groups:
        sel = [r for r in rows if re.search(pat, r["Name"])]
        if sel:
            r = max(sel, key=lambda r: float(r["TotalDurationNs"]))
            line(tag, f"`{r['Name'][:60]}`", r["Calls"], float(r["AverageNs"]) / 1e3, flops)
    # A layer's out and FFN-out products together, whichever epilogue each
    # takes (the bias epilogue before a separate add + LayerNorm, or the
    # whole-row tile with the add + LayerNorm fused): their summed time a
    # layer against both products' FLOPs.
    sel = [r for r in rows if re.search(r"EpiE6E|gemm_ln_kernel", r["Name"])]
    calls = sum(int(r["Calls"]) for r in sel)
    if sel and calls % 2 == 0:
        ns = sum(float(r["TotalDurationNs"]) for r in sel)
        line("out + FFN-out products (a layer's pair)", "bias epilogue or fused add + LayerNorm", calls // 2,
             ns / (calls // 2) / 1e3, 2.0 * T * H * H + 2.0 * T * I * H)
    return out


def timed_run_from_trace(stats_dir, bench_log):
    """The bench's timed runs in the kernel trace of the profiled command:
    the roofline's whole-batch run and the split run (the runs at the JSON
    line's timed_run_index; each run's first kernel is pack_rows_kernel),
    their GEMM launches' average duration and busy time beside what the
    bench's HIP events gave for the same runs."""
    import csv
    import glob
    line = None
    for text in open(bench_log, errors="replace"):
        if text.startswith('{"metric"'):
            line = json.loads(text)
    traces = glob.glob(os.path.join(stats_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not line or "timed_run_index" not in line.get("roofline", {}) or not traces:
        return []
    rf = line["roofline"]
    rows = []
    for f in traces:
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    def run_of(k):
        run = run_slice(rows, k, lambda r: r["Kernel_Name"])
        if not run:
            return None
        spans = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in run
                       if "gemm_" in r["Kernel_Name"])
        busy = busy_union([("g", a, b) for a, b in spans], {"g"})
        length = (max(int(r["End_Timestamp"]) for r in run) - int(run[0]["Start_Timestamp"])) / 1e3
        return spans, busy / 1e3, length, sorted({r["Stream_Id"] for r in run})

    out = []
    w = run_of(rf["timed_run_index"])
    if w and w[0]:
        spans, busy, length, streams = w
        mean = sum(b - a for a, b in spans) / len(spans) / 1e3
        out += ["", f"The roofline's whole-batch run (run {rf['timed_run_index']} of the command, stream(s) "
                f"{', '.join(streams)}) in the kernel trace: {len(spans)} GEMM launches, average {mean:.1f} µs a "
                f"launch, {sum(b - a for a, b in spans) / 1e6:.2f} ms in all within the run's {length / 1e3:.2f} ms. "
                f"The bench's HIP events for the same run: {rf['launches_per_step']} launches, average "
                f"{rf['avg_launch_us']:.1f} µs, {rf['launch_ms_per_step']:.2f} ms in all within "
                f"{rf['timed_run_ms']:.2f} ms; roofline {rf['achieved']:.0f} {rf['unit']}, "
                f"{100 * rf['frac']:.1f}% of peak."]
    c = rf.get("concurrent")
    s = run_of(c["timed_run_index"]) if c else None
    if s and s[0]:
        spans, busy, length, streams = s
        mean = sum(b - a for a, b in spans) / len(spans) / 1e3
        out += ["", f"The headline session's timed run (run {c['timed_run_index']}, its parts side by side when it "
                f"splits; stream(s) "
                f"{', '.join(streams)}) in the kernel trace: {len(spans)} GEMM launches, average {mean:.1f} µs a "
                f"launch (overlapping), busy {busy:.0f} µs. The bench's events: {c['launches_per_step']} launches, "
                f"average {c['avg_launch_us']:.1f} µs, busy {c['busy_us_per_step']:.0f} µs; "
                f"{c['achieved']:.0f} {rf['unit']} over the busy time."]
    return out


def summarize_stats(stats_dir, workload, command, summary_tag="", bench_log=None):
    """profiles/kernels_<workload>.md from a rocprofv3 --kernel-trace --stats
    run of this script: each kernel's calls, total and average duration, and
    the GEMM kernel's launches over all its instantiations; with the
    profiled command's output (bench_log), the timed run's GEMM launches
    from the kernel trace beside the bench's HIP events for that run. With
    summary_tag "unsplit" (a run of whole-batch launches),
    kernels_<workload>_unsplit.md with each matrix-core kernel's achieved
    rate."""
    import csv
    import glob

    rows = []
    for f in glob.glob(os.path.join(stats_dir, "**", "*kernel_stats.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    lines = [f"# rocprofv3 kernel stats: {workload}", "", "Command (from the repository root, one MI355X):", "", "```",
             *command, "```", "", "| kernel (symbol) | calls | total ms | average µs | % |", "|---|---|---|---|---|"]
    for r in rows:
        ns = float(r["TotalDurationNs"])
        lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {ns / 1e6:.3f} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{100 * ns / total:.2f} |")
    for tag, pat in (("GEMM kernel (`gemm_lds_kernel` and `gemm_kernel`, every instantiation)", "gemm_"),
                     ("attention kernel", "attention"), ("add + LayerNorm kernel", "add_layer_norm")):
        sel = [r for r in rows if pat in r["Name"]]
        if sel:
            calls = sum(int(r["Calls"]) for r in sel)
            ns = sum(float(r["TotalDurationNs"]) for r in sel)
            lines.append(f"\nThe {tag}: {calls} launches, {ns / 1e6:.3f} ms, average {ns / calls / 1e3:.1f} µs a launch.")
            if pat == "gemm_":
                # The run's own products: the instantiations holding at least a
                # tenth of the GEMM time (the rest are the small bins' shapes).
                main = [r for r in sel if float(r["TotalDurationNs"]) >= 0.1 * ns]
                mc = sum(int(r["Calls"]) for r in main)
                mns = sum(float(r["TotalDurationNs"]) for r in main)
                lines.append(f"Its {len(main)} instantiations holding a tenth or more of that time (the run's own "
                             f"products): {mc} launches, average {mns / mc / 1e3:.1f} µs a launch.")
    if bench_log:
        lines += timed_run_from_trace(stats_dir, bench_log)
    if summary_tag == "unsplit":
        lines += unsplit_rooflines(rows, workload)
    out = os.path.join(ROOT, "profiles", f"kernels_{workload}{'_' + summary_tag if summary_tag else ''}.md")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(out)


PMC_PASSES = (
    # Matrix cores, vector unit, waves (one counter set a pass: 8 SQ and 1 GRBM counter).
    "GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_INSTS_VALU "
    "SQ_WAVE_CYCLES SQ_WAVES SQ_VALU_MFMA_COEXEC_CYCLES",
    # LDS and waits.
    "GRBM_GUI_ACTIVE SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS "
    "SQ_LDS_ADDR_CONFLICT SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY",
)


def summarize_counters(dirs, workload, command, bench_log=None):
    """profiles/counters_<workload>.md and .json from rocprofv3 --pmc runs of
    this script, one a counter set of PMC_PASSES (each dispatch counted on its
    own): per kernel instantiation, the matrix cores' busy share of the
    SIMD-cycles of its dispatches, the vector unit's active share, and the
    LDS's. The share's normalization (how the profiler sums GRBM_GUI_ACTIVE
    and the SQ counters over the chip's 8 XCDs) is read off the MFMA probe's
    dispatches, whose every wave keeps eight independent product chains in
    flight on every SIMD: their busy share is taken as full, and the factor
    that makes it so is applied to every kernel and printed. The algorithmic
    check beside it: SQ_INSTS_MFMA x the cycles one 32x32x16 product holds a
    SIMD's matrix core (32 on gfx950: 32768 FLOP at 1024 a cycle), over the
    same SIMD-cycles."""
    import csv
    import glob
    import re

    SIMDS = 256 * 4
    per = {}      # kernel -> counter -> summed value
    calls = {}    # kernel -> dispatches (of the first pass)
    for n, d in enumerate(dirs):
        seen = set()
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = r["Kernel_Name"]
                per.setdefault(k, {})
                c = r["Counter_Name"]
                per[k][c] = per[k].get(c, 0.0) + float(r["Counter_Value"])
                if n == 0 and c == "GRBM_GUI_ACTIVE" and (k, r["Dispatch_Id"]) not in seen:
                    seen.add((k, r["Dispatch_Id"]))
                    calls[k] = calls.get(k, 0) + 1
    # GRBM_GUI_ACTIVE appears in every pass: its per-pass sums add up, so
    # each kernel's cycles are their mean over the passes.
    for k, v in per.items():
        if "GRBM_GUI_ACTIVE" in v:
            v["GRBM_GUI_ACTIVE"] /= len(dirs)

    def short(k):
        m = re.match(r"_ZN4rocm\d+(\w+?)I", k)
        base = m.group(1) if m else k.split("(")[0]
        shape = re.findall(r"Li(\d+)E", k)
        return base + ("<" + ",".join(shape) + ">" if shape else "")

    def simd_cycles(v):
        return v.get("GRBM_GUI_ACTIVE", 0.0) * SIMDS

    probe = [k for k in per if "mfma_probe" in k]
    raw_probe = sum(per[k].get("SQ_VALU_MFMA_BUSY_CYCLES", 0) for k in probe) / max(
        1.0, sum(simd_cycles(per[k]) for k in probe))
    factor = 1.0 / raw_probe if raw_probe > 0 else 1.0
    rows = sorted(per.items(), key=lambda kv: -kv[1].get("GRBM_GUI_ACTIVE", 0.0))
    total = sum(v.get("GRBM_GUI_ACTIVE", 0.0) for _, v in rows)
    lines = [f"# Hardware counters per kernel: {workload}", "",
             "Commands (from the repository root, one MI355X; each pass counts every dispatch on its own):", "",
             "```", *command, "```", "",
             f"Matrix-core busy share = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x {SIMDS} SIMDs) x {factor:.4g}: "
             f"the factor makes the MFMA probe's dispatches (8 independent 32x32x16 chains a wave on every SIMD) read "
             f"as fully busy (raw {raw_probe:.4g}). \"by count\" = SQ_INSTS_MFMA x 32 cycles over the same SIMD-cycles "
             f"x the factor. VALU active = SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES (a wave's cycles issuing vector "
             f"instructions); LDS active = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE x 256 CUs) x the factor; bank "
             f"conflicts = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; waiting = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES.", "",
             "| kernel | dispatches | share of GPU cycles | matrix cores busy | by count | VALU active | LDS active "
             "| LDS bank conflicts | waiting on a dependency |", "|---|---|---|---|---|---|---|---|---|"]
    out = {"workload": workload, "command": command, "factor": factor, "probe_raw": raw_probe, "kernels": {}}
    for k, v in rows:
        sc = simd_cycles(v)
        if sc <= 0:
            continue
        g = v.get("GRBM_GUI_ACTIVE", 0.0)
        mf = v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / sc * factor
        cnt = v.get("SQ_INSTS_MFMA", 0.0) * 32 / sc * factor
        wc = v.get("SQ_WAVE_CYCLES", 0.0)
        valu = v.get("SQ_ACTIVE_INST_VALU", 0.0) / wc if wc else 0.0
        lds = v.get("SQ_LDS_IDX_ACTIVE", 0.0) / (g * 256) * factor if g else 0.0
        conf = v.get("SQ_LDS_BANK_CONFLICT", 0.0) / v["SQ_LDS_IDX_ACTIVE"] if v.get("SQ_LDS_IDX_ACTIVE") else 0.0
        wait = v.get("SQ_WAIT_INST_ANY", 0.0) / wc if wc else 0.0
        out["kernels"][k] = {"short": short(k), "dispatches": calls.get(k, 0), "gpu_cycles": g, "mfma_busy": mf,
                             "mfma_busy_by_count": cnt, "valu_active": valu, "lds_active": lds,
                             "lds_bank_conflicts": conf, "waiting": wait, "counters": v}
        if g / total < 0.005:
            continue
        lines.append(f"| `{short(k)}` | {calls.get(k, 0)} | {100 * g / total:.1f}% | {100 * mf:.1f}% | {100 * cnt:.1f}% "
                     f"| {100 * valu:.1f}% | {100 * lds:.1f}% | {100 * conf:.1f}% | {100 * wait:.1f}% |")
    # The command's runs as a whole (every kernel but the probe and the
    # copy): the matrix cores' busy share of all their dispatches'
    # SIMD-cycles, beside the bench line's algorithmic figure.
    run = [v for k, v in rows if "mfma_probe" not in k and "copy_kernel" not in k]
    sc = sum(simd_cycles(v) for v in run)
    if sc > 0:
        mf = sum(v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for v in run) / sc * factor
        gm = [v for k, v in rows if "gemm_" in k]
        at = [v for k, v in rows if "attention" in k]
        share = lambda vs: (sum(v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for v in vs) /  # noqa: E731
                            max(1.0, sum(simd_cycles(v) for v in vs)) * factor)
        out["run_mfma_busy"] = mf
        lines += ["", f"All the command's run kernels together (the probe and the copy left out): matrix cores busy "
                  f"{100 * mf:.1f}% of their dispatches' SIMD-cycles; the GEMM kernel's dispatches {100 * share(gm):.1f}%, "
                  f"attention's {100 * share(at):.1f}%. (The profiler runs each dispatch on its own, so these are "
                  f"shares of each kernel's own time, not of the step's.)"]
        if bench_log:
            for text in open(bench_log, errors="replace"):
                if text.startswith('{"metric"'):
                    d = json.loads(text)
                    out["bench_mfma_util_pct"] = d.get("mfma_util_pct")
                    lines.append(f"The same command run without the profiler (its bench line): mfma_util_pct "
                                 f"{d.get('mfma_util_pct'):.1f}% (the run's algorithmic FLOPs over its step time at "
                                 f"the dense peak: the step's share, where the busy shares above are the kernels' "
                                 f"own), roofline {d['roofline']['achieved']:.0f} {d['roofline']['unit']} for the "
                                 f"{d['roofline']['kernel']} kernel ({100 * d['roofline']['frac']:.1f}% of peak).")
    base = os.path.join(ROOT, "profiles", f"counters_{workload}")
    with open(base + ".md", "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(base + ".json", "w") as f:
        json.dump(out, f, indent=1)
    print("\n".join(lines))


def library_compare(workload, reps=20):
    """profiles/library_<workload>.md: the platform libraries on one layer's
    products and attention of a full-length batch, through torch (its F16 or
    BF16 linear, which calls hipBLASLt or rocBLAS, and its fused
    scaled-dot-product attention), with HIP events on torch's stream. No
    epilogue, no mask: the plain operations the session's kernels fuse more
    into. Measurement only; the session never calls these."""
    import torch
    import torch.nn.functional as F
    shape = W.SHAPES[workload]
    dt = torch.bfloat16 if shape.store == "bf16" else torch.float16
    B, L, H, I, nh = shape.batch, shape.seq, shape.hidden, shape.intermediate, shape.heads
    M, d = B * L, shape.hidden // shape.heads
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    peak = PEAK["bf16" if dt == torch.bfloat16 else "f16"]
    lines = [f"# Platform libraries on {workload}'s layer shapes", "", "Command (from the repository root, one MI355X):",
             "", "```", f"python3 bench.py --workload {workload} --library-compare", "```", "",
             f"torch {torch.__version__}, {torch.cuda.get_device_name(0)}; {str(dt).split('.')[-1]} operands, "
             f"random normal, {reps} launches a figure after 3 untimed.", "",
             "| operation | shape | average µs | TFLOP/s | of peak |", "|---|---|---|---|---|"]
    for tag, n, k in (("Q/K/V product", 3 * H, H), ("out product", H, H), ("FFN-in product", I, H),
                      ("FFN-out product", H, I)):
        a = torch.randn(M, k, device=dev, dtype=dt, generator=g)
        w = torch.randn(n, k, device=dev, dtype=dt, generator=g) * 0.05
        us = timed(lambda: F.linear(a, w))
        rate = 2.0 * M * n * k / (us * 1e-6)
        lines.append(f"| {tag} (linear) | M {M}, N {n}, K {k} | {us:.1f} | {rate / 1e12:.0f} | {100 * rate / peak:.1f}% |")
        del a, w
    q, k_, v = (torch.randn(B, nh, L, d, device=dev, dtype=dt, generator=g) for _ in range(3))
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("memory-efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(be):
                us = timed(lambda: F.scaled_dot_product_attention(q, k_, v))
        except RuntimeError as e:
            lines.append(f"| attention ({name}) | {B}×{nh} heads, {L} tokens, d {d} | not available: "
                         f"{str(e).splitlines()[0][:80]} | | |")
            continue
        rate = 4.0 * B * nh * L * L * d / (us * 1e-6)
        lines.append(f"| attention ({name}) | {B}×{nh} heads, {L} tokens, d {d} | {us:.1f} | {rate / 1e12:.0f} | "
                     f"{100 * rate / peak:.1f}% |")
    out = os.path.join(ROOT, "profiles", f"library_{workload}.md")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="bert-base", choices=sorted(W.SHAPES))
    ap.add_argument("--lengths", default="default", help="'default', 'full', or lo,hi")
    ap.add_argument("--cpu-rows", type=int, default=0,
                    help="rows of the CPU baseline's sample (0: as many as about 10 s of CPU work takes)")
    ap.add_argument("--also-lengths", default="auto",
                    help="lo,hi: also time the same session on rows of lengths uniform in [lo, hi] under the mask "
                         "('auto': 64,512 for bert-base, none otherwise)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--autotune", default="on", choices=["off", "on"],
                    help="the session's kernel choices: measured at session creation (on, the default) or the rule's")
    ap.add_argument("--budget-ms", type=int, default=750, help="the tuner's budget (the core's with a disk cache)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed steps, copy 256 MiB on the device (the traffic counters' reference)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic_<workload>.json from two rocprofv3 --pmc runs and exit")
    ap.add_argument("--pmc-command", action="append", default=[], help="the profiling commands, for the summary")
    ap.add_argument("--summarize-stats", metavar="STATS_DIR",
                    help="write profiles/kernels_<workload>.md from a rocprofv3 --kernel-trace --stats run and exit")
    ap.add_argument("--bench-log", metavar="FILE",
                    help="with --summarize-stats, --summarize-pmc or --summarize-counters: the profiled command's "
                         "output, whose JSON line names the timed runs")
    ap.add_argument("--summary-tag", default="", choices=["", "unsplit"],
                    help="with --summarize-stats: 'unsplit' for a run under TURBO_ROCM_SPLIT=1 of full-length rows "
                         "(per-kernel rates added; written to kernels_<workload>_unsplit.md)")
    ap.add_argument("--summarize-counters", nargs="+", metavar="PASS_DIR",
                    help="write profiles/counters_<workload>.md from rocprofv3 --pmc runs of PMC_PASSES and exit")
    ap.add_argument("--library-compare", action="store_true",
                    help="time torch's linear and fused attention on the workload's full-length layer shapes, write "
                         "profiles/library_<workload>.md and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not run (each row's encoder is "
              "independent, so more GPUs would shard rows with no exchange)", file=sys.stderr)
        sys.exit(2)

    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.workload, args.pmc_command, args.bench_log)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters, args.workload, args.pmc_command, args.bench_log)
        return
    if args.summarize_stats:
        summarize_stats(args.summarize_stats, args.workload, args.pmc_command, args.summary_tag, args.bench_log)
        return
    if args.library_compare:
        library_compare(args.workload)
        return
    shape = W.SHAPES[args.workload]
    lengths = {"default": "default", "full": None}.get(args.lengths)
    if lengths is None and args.lengths not in ("default", "full"):
        lengths = tuple(int(v) for v in args.lengths.split(","))
    t0 = time.time()
    desc = W.model(shape)
    if shape.task == S.TURBO_TASK_RERANK:
        # The cross-encoder's encoder: every pair's window ([CLS] query [SEP]
        # passage [SEP], types 0/1) as a row, CLS states unnormalized; the
        # head, applied on the host in F64, is outside the timed steps.
        from turboembed_amd.rerank import pair_windows
        qt = shape.extra["query_tokens"]
        wins = [pair_windows(q, p, shape.cls_id, shape.sep_id, query_tokens=qt, max_tokens=shape.seq)
                for q, p in W.rerank_pairs(shape)]
        ids = np.concatenate([w[0] for w in wins]).astype(np.int32)
        types = np.concatenate([w[1] for w in wins]).astype(np.int32)
        wl = np.concatenate([w[2] for w in wins])
        mask = (np.arange(shape.seq)[None, :] < wl[:, None]).astype(np.int32)
        assert ids.shape[0] == shape.batch, "one window a pair"
    else:
        ids, mask, types = W.rows(shape, lengths=lengths)
    print(f"# model and rows ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    rt = T.Runtime()
    assert rt.device_count() >= 1, "no gfx950 device"
    ctx = rt.context(0)
    model = ctx.load(desc)
    mode = S.TURBO_AUTOTUNE_ON if args.autotune == "on" else S.TURBO_AUTOTUNE_OFF
    # A range workload embeds once and mean-pools contiguous ranges of each
    # row's tokens (embed_write_ranges); the others pool each row.
    rngs = W.ranges(shape, mask) if shape.ranges_per_row else None
    sess = model.session(shape.batch, shape.seq, shape.precision, autotune=mode, budget_ms=args.budget_ms,
                         max_ranges=len(rngs) if rngs else 0)
    dtype = {S.TURBO_DTYPE_F16: "f16", S.TURBO_DTYPE_BF16: "bf16", S.TURBO_DTYPE_F32: "f32",
             S.TURBO_DTYPE_I8: "i8"}[sess.compute_dtype]
    if rngs:
        sess.write_ranges(ids, mask, rngs, types, normalize=shape.normalize)
    else:
        sess.write_tokens(ids, mask, types, pooling=shape.pooling, normalize=shape.normalize)
    sess.run()
    gpu_vecs = sess.read()
    print(f"# loaded, first run done in {time.time() - t0:.1f}s; choices {sess.choices()}", file=sys.stderr,
          flush=True)

    sess.replay(args.warmup)
    start = time.perf_counter()
    sess.replay(args.steps)
    elapsed = time.perf_counter() - start
    ms = elapsed / args.steps * 1e3
    lens = mask.sum(1)
    tokens = int(lens.sum())
    seq_per_s = shape.batch / (ms / 1e3)

    # The same rows written, run and read back each step (the reference's
    # p50 measures this, bench/src/measure/mod.rs:292-321): PCIe both ways
    # included, beside the device-resident figure.
    def write_run_read(batches, steps):
        for b in batches[:2]:
            put(*b)
            sess.run()
            sess.read()
        w0 = time.perf_counter()
        for i in range(steps):
            put(*batches[i % len(batches)])
            sess.run()
            sess.read()
        return (time.perf_counter() - w0) / steps * 1e3

    def put(i, m, t):
        if rngs:
            sess.write_ranges(i, m, rngs, t, normalize=shape.normalize)
        else:
            sess.write_tokens(i, m, t, pooling=shape.pooling, normalize=shape.normalize)

    wrr_ms = write_run_read([(ids, mask, types)], args.steps)

    # Per-kernel times from HIP events, one run launched directly as the
    # replayed run executes (a split run's two parts side by side, no marker
    # between launches): each launch's pair of events is bound to its
    # kernels' own dispatch packets (the start of the first, the end of the
    # last), the timestamps a kernel trace reads.
    def timed_run(s):
        s.set_timing(True)
        s.replay(1)
        out = s.times(), s.launches(), s.intervals()
        s.set_timing(False)
        return out

    times, counts, intervals = timed_run(sess)
    # The process's runs so far (each begins with pack_rows_kernel, so a
    # kernel trace finds them): the first run, the warm-up and timed steps,
    # the write-run-read steps with their one warm-up run, the timed run.
    runs_done = 1 + args.warmup + args.steps + 1 + args.steps + 1
    per = kernel_flops(shape, tokens, lens)
    total_flops = W.gemm_flops_per_token(shape) * tokens + W.attention_flops(shape, lens)

    def dominant(times, counts, intervals):
        """The dominant kernel of a timed run, the GEMM kernel (every linear
        layer's launches) or attention, whichever is busy longer: its name,
        summed launch time, FLOPs, launches and busy time (the union of its
        launches' intervals over every stream)."""
        def busy_ms(names):
            return busy_union(intervals, names)

        gemm_names = [k for k in times if k.startswith("gemm_")]
        gemm = ("gemm", sum(times[k] for k in gemm_names), sum(per[k] for k in gemm_names) * shape.layers,
                sum(counts[k] for k in gemm_names), busy_ms(set(gemm_names)))
        if "attention" in times and busy_ms({"attention"}) > gemm[4]:
            return ("attention", times["attention"], per["attention"] * shape.layers, counts["attention"],
                    busy_ms({"attention"}))
        return gemm

    # The split run's figures: its parts' launches overlap, so their own
    # durations sum past the time the kernel was running; the rate there is
    # over that busy time.
    c_dom, c_ms, c_flops, c_launches, c_busy = dominant(times, counts, intervals)
    concurrent = {"kernel": c_dom, "launches_per_step": c_launches, "avg_launch_us": c_ms / c_launches * 1e3,
                  "busy_us_per_step": c_busy * 1e3, "achieved": c_flops / (c_busy / 1e3) / 1e12,
                  "frac": c_flops / (c_busy / 1e3) / PEAK[dtype], "timed_run_ms": max(b for _, _, b in intervals),
                  "timed_run_index": runs_done - 1}

    # The roofline: the dominant kernel's launches over the whole batch (the
    # same rows in a session whose runs do not split: one launch a layer per
    # product, on one stream), so each launch's pair of events brackets that
    # launch alone and the launches' summed time lies inside the run.
    saved = os.environ.get("TURBO_ROCM_SPLIT")
    os.environ["TURBO_ROCM_SPLIT"] = "1"
    try:
        whole = model.session(shape.batch, shape.seq, shape.precision, autotune=mode, budget_ms=args.budget_ms,
                              max_ranges=len(rngs) if rngs else 0)
    finally:
        if saved is None:
            del os.environ["TURBO_ROCM_SPLIT"]
        else:
            os.environ["TURBO_ROCM_SPLIT"] = saved
    if rngs:
        whole.write_ranges(ids, mask, rngs, types, normalize=shape.normalize)
    else:
        whole.write_tokens(ids, mask, types, pooling=shape.pooling, normalize=shape.normalize)
    whole.run()
    whole.replay(2)
    w_times, w_counts, w_intervals = timed_run(whole)
    whole_index = runs_done + 3
    whole.close()
    dom, dom_ms, dom_flops, dom_launches, dom_busy = dominant(w_times, w_counts, w_intervals)
    achieved = dom_flops / (dom_ms / 1e3)
    traffic = None
    if dom == "gemm" and os.path.exists(traffic_file(args.workload)):
        with open(traffic_file(args.workload)) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")
    # The matrix cores' sustained F16 rate with random operands (as a GEMM's)
    # and with fixed ones, and the clock under that load: the ceiling the
    # chip's power lets a real GEMM reach, beside the published peak.
    ceiling = None
    if dtype in ("f16", "bf16"):
        rnd_tf, rnd_mhz = T.mfma_probe(random=True)
        fix_tf, fix_mhz = T.mfma_probe(random=False)
        ceiling = {"random_operands_tflops": round(rnd_tf, 1), "random_operands_mhz": round(rnd_mhz),
                   "fixed_operands_tflops": round(fix_tf, 1), "fixed_operands_mhz": round(fix_mhz),
                   "end_to_end_frac_of_random_ceiling": total_flops / (ms / 1e3) / (rnd_tf * 1e12)}
    if args.copy_probe:
        T.copy_probe(COPY_PROBE_BYTES, iters=3)
    roofline = {"kernel": dom, "bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK[dtype] / 1e12,
                "unit": "TOP/s" if dtype == "i8" else "TFLOP/s", "frac": achieved / PEAK[dtype], "traffic": traffic,
                "run": "whole batch: the same rows in a session whose runs do not split (one launch a layer per "
                       "product, one stream)",
                "launches_per_step": dom_launches, "avg_launch_us": dom_ms / dom_launches * 1e3,
                "flops_per_launch": dom_flops / dom_launches,
                "launch_ms_per_step": dom_ms, "timed_run_ms": max(b for _, _, b in w_intervals),
                # The timed run's place among the process's runs (0: the
                # first run), for finding it in a kernel trace.
                "timed_run_index": whole_index,
                "concurrent": concurrent}

    # The memory-bound kernels against HBM's published rate.
    n_out = len(rngs) if rngs else shape.batch
    tail = {}
    for k, b in tail_bytes(shape, dtype, tokens, n_out, shape.hidden).items():
        if times.get(k):
            gbps = b / (times[k] / 1e3) / 1e9
            tail[k] = {"launches": counts[k], "avg_launch_us": times[k] / counts[k] * 1e3,
                       "bytes_per_launch": b / counts[k], "achieved_GBps": gbps, "frac": gbps * 1e9 / HBM_PEAK}

    # The same session on variable-length rows under the mask (the second
    # run of the workload): one batch replayed on the device, then a fresh
    # batch every step written, run and read back (each replays its bin's
    # graph; none is captured in the run).
    extra_runs = {"write_run_read": {"ms_per_step": wrr_ms, "sequences_per_s": shape.batch / (wrr_ms / 1e3),
                                     "note": "the headline rows written, run and read back each step"}}
    also = ("64,512" if args.workload == "bert-base" else "") if args.also_lengths == "auto" else args.also_lengths
    if also and not rngs:
        lo, hi = (int(v) for v in also.split(","))
        vids, vmask, vtypes = W.rows(shape, lengths=(lo, hi), seed=1)
        sess.write_tokens(vids, vmask, vtypes, pooling=shape.pooling, normalize=shape.normalize)
        sess.replay(args.warmup)
        v0 = time.perf_counter()
        sess.replay(args.steps)
        vms = (time.perf_counter() - v0) / args.steps * 1e3
        vt = int(vmask.sum())
        vflops = W.gemm_flops_per_token(shape) * vt + W.attention_flops(shape, vmask.sum(1))
        fresh = [W.rows(shape, lengths=(lo, hi), seed=100 + k) for k in range(args.steps)]
        c0, _ = sess.graphs()
        fms = write_run_read(fresh, args.steps)
        c1, _ = sess.graphs()
        ft = sum(int(b[1].sum()) for b in fresh) / len(fresh)
        extra_runs[f"lengths_{lo}_{hi}"] = {"ms_per_step": vms, "sequences_per_s": shape.batch / (vms / 1e3),
                                            "tokens_per_s": vt / (vms / 1e3), "live_tokens": vt,
                                            "mfma_util_pct": 100.0 * vflops / (vms / 1e3) / PEAK[dtype],
                                            "fresh_write_run_read": {
                                                "ms_per_step": fms, "sequences_per_s": shape.batch / (fms / 1e3),
                                                "tokens_per_s": ft / (fms / 1e3), "batches": len(fresh),
                                                "captures_during_runs": c1 - c0}}

    cpu = None
    min_cos = None
    if not args.no_cpu:
        import oracle
        # A bounded sample, about 10 s of CPU work: the rows in order (on rows
        # over 1024 tokens the shortest first), as many as the one-row pass
        # before it says fit in 10 s (--cpu-rows fixes the count); its ranges
        # with it.
        order = np.argsort(lens, kind="stable") if shape.seq > 1024 else np.arange(shape.batch)
        # Every core this process may run on, one pinned thread each.
        threads = len(os.sched_getaffinity(0))
        oracle.set_pinning(True)
        model_name = oracle.cpu_model()
        # A one-row pass first pages the code and the model's tables in; a
        # second times a row (its pass alone: the oracle lays out the weights
        # on every call, outside the time it reports).
        for _ in range(2):
            oracle.encode(desc, ids[order[:1]], mask[order[:1]], types[order[:1]], pooling=shape.pooling,
                          normalize=shape.normalize, threads=threads)
            row_s = oracle.last_encode_seconds()
        # (A row's cost taken as growing with its length to the power 1.5:
        # the products go with the tokens, attention with their square.)
        if args.cpu_rows:
            n = min(args.cpu_rows, shape.batch)
        else:
            l0, spent, n = max(int(lens[order[0]]), 1), 0.0, 0
            while n < shape.batch:
                spent += max(row_s, 1e-3) * (max(int(lens[order[n]]), 1) / l0) ** 1.5
                if n > 0 and spent > 10.0:
                    break
                n += 1
        pick = order[:n]
        print(f"# timed; CPU baseline on rows {pick.tolist()} ({int(lens[pick].sum())} tokens) on {threads} threads "
              f"({model_name})", file=sys.stderr, flush=True)
        sample_ranges, got_idx = None, pick
        if rngs:
            where = {int(r): i for i, r in enumerate(pick)}
            got_idx = [k for k, r in enumerate(rngs) if r[0] in where]
            sample_ranges = [(where[rngs[k][0]], rngs[k][1], rngs[k][2]) for k in got_idx]
        want = oracle.encode(desc, ids[pick], mask[pick], types[pick], pooling=shape.pooling,
                             normalize=shape.normalize, ranges=sample_ranges, threads=threads)
        cpu_s = oracle.last_encode_seconds()
        got = gpu_vecs[got_idx]
        cos = (got * want).sum(1) / np.linalg.norm(got, axis=1) / np.linalg.norm(want, axis=1)
        min_cos = float(cos.min())
        what = f", {len(sample_ranges)} ranges" if sample_ranges else ""
        oracle.set_pinning(False)
        cpu = {"value": n / cpu_s, "unit": "sequences/s", "cores": threads, "kind": "port",
               "cpu_model": model_name,
               "sample": f"{n} of the {shape.batch} rows ({int(lens[pick].sum())} tokens{what}), all {shape.layers} "
                         f"layers, one pass after two one-row passes, {cpu_s:.1f} s on {threads} pinned threads (the rows' "
                         f"pass, not the oracle's weight layout before it) "
                         f"({model_name})"}

    eff_lengths = shape.lengths if lengths == "default" else lengths
    line = {
        "metric": f"sequences/s ({args.workload}, {dtype}, {shape.batch}x{shape.seq})",
        "value": seq_per_s, "unit": "sequences/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: {shape.layers} layers, hidden {shape.hidden}, {shape.heads} heads, "
                               f"FFN {shape.intermediate}, {shape.batch} rows x {shape.seq}, " +
                               (f"{shape.batch} query/passage pairs, query {shape.extra['query']} and passage "
                                f"{shape.extra['passage']} tokens, one [CLS] q [SEP] p [SEP] window each"
                                if shape.task == S.TURBO_TASK_RERANK else
                                ("all live" if eff_lengths is None else f"lengths uniform in {list(eff_lengths)}")),
                   "global_batch": shape.batch, "seq_len": shape.seq, "live_tokens": tokens, "parallelism": "none"},
        "tokens_per_s": tokens / (ms / 1e3),
        "mfma_util_pct": 100.0 * total_flops / (ms / 1e3) / PEAK[dtype],
        "algorithmic_tflop_per_step": total_flops / 1e12,
        "min_cosine_vs_cpu": min_cos,
        "kernel_ms": {k: round(v, 4) for k, v in times.items()},
        "kernel_choices": sess.choices(),
        "other_runs": extra_runs,
        "ranges": len(rngs) if rngs else 0,
        "tune_ms": sess.tuning.tune_ms,
        # The tuner's timings of the bins this workload's run takes (ms a
        # run through the first layer, parts overlapped as the run forks
        # them), <bin>/<knob>/<variant>.
        "tune_timings": {k: round(v, 4) for k, v in sess.timings.items()
                         if k.split("/")[0] in ("le16k", "gt16k") or shape.batch * shape.seq <= 16384},
        "roofline": roofline,
        "hbm_tail": tail,
        "cpu_baseline": cpu,
        "mfma_ceiling_measured": ceiling,
    }
    print(json.dumps(line), flush=True)
    sess.close()
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
