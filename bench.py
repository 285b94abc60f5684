"""Throughput of bert_embed on one MI355X, in the driver's JSON-line format.

Default workload: the synthetic varlen mix - 2000
sentences, lognormal lengths clipped to [5, 64], 32 consecutive batches of 64
in seeded order, each padded to round16(longest) (eff 32/48/64, 91,648 padded
rows).  One step = one bert_embed per batch at its padded length, as the
reference's corpus benchmark loops over its batches (bench/corpus.cu:120-132):
bbh_embed_each runs each batch as its own forward (nothing merged, every
padding row computed) and spreads the 32 forwards over EACH_STREAMS
concurrent HIP streams (the pool's and the caller's), one workspace each.  value = sentences/s over the K
timed steps, inputs pre-uploaded to HBM.

The roofline names the dominant kernel class of that pass: the same pass on a
one-slot pool with a pair of HIP events around every launch on the caller's
stream (so no other stream shares the GPU during a launch).  Its bound is the
roof that binds at the kernel's arithmetic intensity (FLOPs over the measured
L2-miss bytes of a counter run where one is committed, else over the
algorithmic bytes) against the ridge PEAK_FP16_DENSE / PEAK_HBM: MFMA above
it, HBM below; achieved = algorithmic FLOPs or bytes per launch / mean launch
time, in that roof's unit, and frac_of_mfma_peak is given either way.

Extra fields: the same pass on one stream; the reference corpus benchmark's
two modes on the same sentences (length-sorted dynamic batches, and every
batch at seq 128, bench/corpus.cu:64-132); the padding-free packed pass and
the equal-seq-merged padded pass; configs[1] / configs[2] (batch 64 x seq
16 / 128, 300 iterations as bench/bench.cu:32-51); the reference's batch
sweep (batch 1, 8, 32, 64 at seq 128 and 16, bench/bench.cu:86-96); configs[4] (batch 256 x
seq 512) with the fused GEMMs' fraction of the fp16 dense MFMA peak; the
tokenizer rate; and the CPU baseline (transformers' BertModel fp32 forward, the
library the reference's cpu_fp32 leg times, on this host's cores).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "bert-by-hand_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

EACH_STREAMS = 4  # concurrent per-batch forwards (pool slots): 3 pool streams and the caller's
#                  stream.  HIP maps streams onto GPU_MAX_HW_QUEUES = 4 hardware queues and
#                  the caller's stream holds one, so 4 slots keep every queue busy (per pass:
#                  3 pool streams beside an idle caller 5.07 ms, 4 slots 4.33 ms; earlier,
#                  4 pool streams beside the caller, two sharing a queue, 6.2-7.0 ms; with
#                  5-8 hardware queues every configuration above 3 busy queues took 11-22 ms)
POOL_BATCH = 1024  # workspace rows of the packed / merged pool = POOL_BATCH * 64
PEAK_FP16_DENSE = 2.5e15  # MI355X published dense fp16 MFMA, FLOP/s
PEAK_HBM = 8.0e12  # B/s
EPI_OF_OP = {"qkv": "0 (bias)", "ffn1_gelu": "1 (bias+GELU)"}
PROFILES = os.path.join(ROOT, "profiles")

# Algorithmic FLOPs of one Linear: 2*M*N*K.
LAYER_GEMMS = [  # (name, N, K, epilogue)
    ("qkv", 1152, 384, "bias"),
    ("o_proj_ln", 384, 384, "ln"),
    ("ffn1_gelu", 1536, 384, "gelu"),
    ("ffn2_ln", 384, 1536, "ln"),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(torch, fn, iters, warmup=3):
    """Average ms per call of fn() between events on the current stream."""
    for _ in range(warmup):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / iters


def gemm_runner(torch, engine, model_w, M, N, K, epi, buf):
    """Closure launching one encoder GEMM at (M, N, K) with synthetic data."""
    A = buf["A"][: M * K].view(M, K)
    W = buf["W"][: N * K].view(N, K)
    bias = buf["b"][:N]
    C = buf["C"][: M * N].view(M, N)
    if epi == "ln":
        res = buf["R"][: M * 384].view(M, 384)
        g, be = buf["g"], buf["be"]
        return lambda: engine.launch_linear_residual_layernorm(A, W, bias, res, g, be, C, M, K)
    return lambda: engine.launch_matmul(A, W, C, M, N, K, bias=bias, gelu=(epi == "gelu"))


def gemm_buffers(torch, max_m):
    g = torch.Generator(device="cuda").manual_seed(0)
    mk = lambda n, s=1.0: (torch.randn(n, device="cuda", generator=g) * s).half()  # noqa: E731
    return dict(A=mk(max_m * 1536), W=mk(1536 * 1536, 0.03), b=mk(1536, 0.02),
                C=torch.empty(max_m * 1536, dtype=torch.float16, device="cuda"),
                R=mk(max_m * 384), g=torch.ones(384, dtype=torch.float16, device="cuda"),
                be=torch.zeros(384, dtype=torch.float16, device="cuda"))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:  # pragma: no cover
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(batches, weights, budget_s=15.0):
    """The reference's torch CPU fp32 forward (transformers BertModel + mean
    pool + L2 normalize, the library its cpu_fp32 leg times,
    scripts/benchmark.py:64-86,110-111) on the same varlen batches and seeded
    weights, on this host's cores: 3 warmup forwards, then the batches in
    order, passes over the mix repeated until ~budget_s of CPU work (whole
    batches; the last pass may stop part-way)."""
    import torch

    from oracle import torch_forward as T

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(os.cpu_count() or 1, avail or 1, omp or (os.cpu_count() or 1)))
    torch.set_num_threads(threads)
    model = T.build(weights)
    for _ in range(3):
        T.embed(model, *batches[0][:3])
    n_sent, used, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 <= budget_s:
        for ids, types, mask, _ in batches:
            T.embed(model, ids, types, mask)
            n_sent += ids.shape[0]
            used += 1
            if time.perf_counter() - t0 > budget_s:
                break
    dt = time.perf_counter() - t0
    return {"value": round(n_sent / dt, 1), "unit": "sentences/s", "cores": int(torch.get_num_threads()),
            "kind": "port",
            "sample": f"transformers BertModel fp32 (sdpa) + mean pool + L2 normalize, torch "
                      f"{torch.__version__}, one forward per batch, {used} batches = {used / len(batches):.2f} "
                      f"passes over the {len(batches)} varlen batches ({n_sent} sentences, padded as on "
                      f"the GPU), {dt:.1f} s after 3 warmup forwards",
            "ms_per_sentence": round(dt / n_sent * 1e3, 4),
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "affinity_cpus": avail,
            "omp_num_threads": omp or None}


def tokenizer_rate(engine, synth, n=2000, seq=128, reps=5):
    """Host-side text -> ids throughput of the WordPiece tokenizer on seeded
    synthetic texts and vocabulary (one thread), beside transformers'
    BertTokenizerFast (the reference's tokenizer; Rust, batch-parallel) on
    the same texts when it is importable."""
    import tempfile

    vocab, texts = synth.text_vocab(), synth.texts(seed=3, n=n)
    out = {"texts": n, "seq": seq, "threads": 1, "vocab": f"seeded synthetic ({len(vocab)} entries)"}
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "vocab.txt"), "w", encoding="utf-8") as f:
            f.write("\n".join(vocab) + "\n")
        tok = engine.Tokenizer(os.path.join(d, "vocab.txt"))
        tok(texts[:100], seq)
        t0 = time.perf_counter()
        for _ in range(reps):
            tok(texts, seq)
        out["sentences_per_s"] = round(n * reps / (time.perf_counter() - t0), 1)
        tok.close()
        try:
            import transformers

            ref = transformers.BertTokenizerFast.from_pretrained(d, do_lower_case=True)
            kw = dict(padding="max_length", truncation=True, max_length=seq, return_tensors="np")
            ref(texts[:100], **kw)
            t0 = time.perf_counter()
            for _ in range(reps):
                ref(texts, **kw)
            out["hf_bert_tokenizer_fast_sentences_per_s"] = round(n * reps / (time.perf_counter() - t0), 1)
        except Exception as e:  # pragma: no cover
            out["hf_bert_tokenizer_fast_sentences_per_s"] = f"unavailable ({type(e).__name__})"
    return out


def pass_timer(torch, fn, steps, warmup):
    """(ms per pass between events on the current stream, wall ms per pass)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps, (time.perf_counter() - t0) / steps * 1e3


def launch_work(r):
    """Algorithmic (FLOPs, HBM bytes) of one recorded launch (bbh_launch_time)."""
    op, M, N, K = r["op"], r["m"], r["n"], r["k"]
    if op == "attention":  # (batch, seq, heads); padded keys count (the kernel visits them)
        B, S, H = M, N, K
        return 4.0 * B * H * 32 * S * S, B * S * (3 * 384 + 384) * 2.0 + 4.0 * B * S
    if op == "embed":  # rows: ids + types + word row in, hidden row out; pos/type rows from L2
        return 0.0, M * (8.0 + 768 + 768)
    if op == "pool":  # (batch, seq): hidden + mask in, embedding out
        return 0.0, M * N * (768.0 + 4) + M * 768.0
    if op == "layernorm":  # rows read and written in place, gamma/beta
        return 0.0, M * 1536.0 + 1536
    if op == "ffn":  # (M, 384, 1536): both Linears; X in (also the residual), out, weights
        return 4.0 * M * N * K, (2 * M * N + 2 * N * K + K + 3 * N) * 2.0
    if op == "qkv" and r.get("fused_ln") == 3:  # QKV Linear + attention, (M, batch, seq)
        B, S = N, K
        flops = 2.0 * M * 1152 * 384 + 4.0 * B * 12 * 32 * S * S
        return flops, (M * 384 * 2 + 1152 * 384 + M * 384) * 2.0 + B * S * 4.0 + M * 56.0
    flops = 2.0 * M * N * K
    byts = (M * K + N * K + M * N + N) * 2.0
    if op in ("o_proj_ln", "ffn2_ln"):
        byts += M * N * 2.0  # the residual
    if r.get("fused_ln") == 2:  # carried LayerNorm: (mean, rstd) a row, and up to 6 tile pairs
        byts += M * (8.0 + 48.0)
    return flops, byts


def qkv_attention_rows(seq):
    """Rows of a qkv_attention_kernel workgroup at this sentence length: 192 (six
    wavefronts) for seq 48, 80 and 96, whose sentences fill 192 rows exactly, else 128."""
    return 192 if seq in (48, 80, 96) else 128


def kernel_name(engine, op, tile, fused, seq=0):
    """(display name, class name as short_kernel() writes it) of a launch record;
    seq: the sentence length of a fused QKV + attention record (its k)."""
    row = {"attention": "attention_kernel", "embed": "embedding_ln_kernel",
           "pool": "pool_normalize_kernel", "layernorm": "ln384_kernel",
           "ffn": "ffn_fused_kernel"}
    if op in row:
        return row[op], row[op]
    if op == "qkv" and fused == 3:
        name = f"qkv_attention_kernel<{qkv_attention_rows(seq)}>"
        return name, name
    if fused == 2:  # the LayerNorm carried between the GEMMs as row statistics
        epi = {"qkv": "4 (carried LayerNorm in)", "ffn1_gelu": "5 (carried LayerNorm in+GELU)"}.get(
            op, "6 (bias+residual, row statistics out)")
    else:
        epi = EPI_OF_OP.get(op) or ("3 (bias+residual+LayerNorm)" if fused else "2 (bias+residual)")
    tname = engine.gemm_tile_name(tile)
    if tname.startswith("WRes"):
        return f"gemm_wres_kernel<{epi}>", f"gemm_wres_kernel<{epi[0]}>"
    return f"gemm_kernel<{tname}, {epi}>", f"gemm_kernel<{tname}, {epi[0]}>"


def gemm_grid_items(tile_name, M, N):
    """Work-items of a tiled-GEMM launch (the launcher's grid: N/BN column
    tiles x 8 XCDs x ceil(M-tiles / 8), 64*WM*WN threads), as rocprofv3
    reports Grid_Size; None for other kernels."""
    import re

    m = re.match(r"Cfg<(\d+),(\d+),(\d+),(\d+),", tile_name)
    if not m:
        return None
    bm, bn, wm, wn = (int(x) for x in m.groups())
    return (N // bn) * 8 * ((-(-M // bm) + 7) // 8) * 64 * wm * wn


def classify(engine, recs, steps):
    """Launch records -> classes keyed (op, tile, fused, M): summed ms, count,
    algorithmic FLOPs and bytes, sorted by summed time."""
    classes = {}
    for r in recs:
        key = (r["op"], r["tile"], r["fused_ln"], r["m"], r["k"] if r["fused_ln"] == 3 else 0)
        c = classes.setdefault(key, {"ms": 0.0, "n": 0, "flops": 0.0, "bytes": 0.0, "m": set()})
        f, b = launch_work(r)
        c["ms"] += r["ms"]
        c["n"] += 1
        c["m"].add(r["m"])
        c["flops"] += f
        c["bytes"] += b
    total = sum(c["ms"] for c in classes.values())
    rows = []
    for (op, tile, fused, m, seq), c in sorted(classes.items(), key=lambda kv: -kv[1]["ms"]):
        avg_s = c["ms"] / c["n"] / 1e3
        name, cls = kernel_name(engine, op, tile, fused, seq)
        n_out = {"qkv": 1152, "ffn1_gelu": 1536}.get(op, 384)
        grid = gemm_grid_items(engine.gemm_tile_name(tile), m, n_out) if tile >= 0 else None
        rows.append({"kernel": name, "class": cls, "op": op, "m": m, "grid_items": grid,
                     "launches_per_step": round(c["n"] / steps, 2),
                     "avg_launch_us": round(avg_s * 1e6, 2),
                     "tflops": round(c["flops"] / c["n"] / avg_s / 1e12, 1),
                     "gb_per_s": round(c["bytes"] / c["n"] / avg_s / 1e9, 1),
                     "algorithmic_flops_per_launch": round(c["flops"] / c["n"]),
                     "algorithmic_bytes_per_launch": round(c["bytes"] / c["n"]),
                     "share_of_op_time": round(c["ms"] / total, 3)})
    return rows


def short_kernel(name):
    """Readable kernel class of a rocprofv3 kernel name (mangled or demangled)."""
    import re

    n = name.replace("(anonymous namespace)::", "").replace("bbh::", "").replace(" ", "")
    m = (re.search(r"gemm_kernel<Cfg<([-\d,]+)>,(\d)>", n) or
         re.search(r"gemm_kernelINS0_3CfgILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(n?\d+)ELi(\d+)"
                   r"EEELi(\d)E", n))
    if m:
        g = [x.replace("n", "-") for x in m.groups()]  # Itanium mangling writes -2 as n2
        cfg, epi = (g[0], g[1]) if len(g) == 2 else (",".join(g[:7]), g[7])
        return f"gemm_kernel<Cfg<{cfg}>, {epi}>"
    m = re.search(r"gemm_wres_kernel(?:<|ILi)(\d)", n)
    if m:
        return f"gemm_wres_kernel<{m.group(1)}>"
    m = re.search(r"qkv_attention_kernel(?:<|ILi)(\d+)", n)
    if m:
        return f"qkv_attention_kernel<{m.group(1)}>"
    m = (re.search(r"attention_kernel<(\d+),(\d+),(\d+),(\w+)>", n) or
         re.search(r"attention_kernelILi(\d+)ELi(\d+)ELi(\d+)ELb(\d)E", n))
    if m:
        vl = {"0": "false", "1": "true"}.get(m.group(4), m.group(4))
        return f"attention_kernel<{m.group(1)},{m.group(2)},{m.group(3)},{vl}>"
    if "at6native" in n or n.startswith("at::") or "at::native" in n:
        return "torch kernel (" + ("copy" if "copy" in n else "fill/elementwise") + ")"
    m = re.search(r"GLOBAL__N_1\d+([A-Za-z_0-9]+?)E", n) or re.match(r"(?:void)?([A-Za-z_0-9]+)", n)
    return m.group(1) if m else n[:60]


def tile_id(kernel_class):
    """The GEMM tile configuration id of a short_kernel class (the id that
    bbh_gemm_tile_name names; 33 = the weight-resident kernel), else ""."""
    import re

    if kernel_class.startswith("gemm_wres_kernel"):
        return "33"
    m = re.search(r"(Cfg<[-\d,]+>)", kernel_class)
    if not m:
        return ""
    from bbh import capi

    for i in range(64):  # every id the table can hold
        if capi.lib().bbh_gemm_tile_name(i).decode() == m.group(1):
            return str(i)
    return "?"


def op_tags(rows, queue_col, grid):
    """Dispatch_Id -> " [o_proj]" / " [ffn2]" for the residual GEMMs of
    profiler rows.  O-proj and FFN2 can run the same kernel on the same grid
    (e.g. the 64x64 copy-ring tile at 2049-4096 rows), so kernel name and grid
    do not tell them apart; within one queue, an encoder layer runs O-proj
    right after attention and FFN2 right after the GELU Linear (FFN1)."""
    import re

    seen, order = set(), []
    for r in rows:  # counter CSVs hold one row per counter and dispatch
        if r["Dispatch_Id"] not in seen:
            seen.add(r["Dispatch_Id"])
            order.append(r)
    order.sort(key=lambda r: (r[queue_col], int(r["Dispatch_Id"])))
    tags, prev = {}, {}
    for r in order:
        q, k = r[queue_col], short_kernel(r["Kernel_Name"])
        p = prev.get(q)
        # residual epilogues 2, 3, 6 (row statistics out); GELU epilogues 1, 5
        if re.match(r"gemm_(kernel<.*, [236]>|wres_kernel<3>)$", k) and p:
            if p.startswith(("attention_kernel", "qkv_attention_kernel")):
                tags[r["Dispatch_Id"]] = " [o_proj]"
            elif re.match(r"gemm_(kernel<.*, [15]>|wres_kernel<1>)$", p):
                tags[r["Dispatch_Id"]] = " [ffn2]"
        prev[q] = k
    return tags


def pmc_summary(paths, trace=None, fetch_scale=1.0, write_scale=1.0, stream=None):
    """Per (kernel class, grid size) means over the dispatches of rocprofv3
    --pmc counter_collection CSVs, as a markdown table.  FETCH_SIZE and
    WRITE_SIZE (KiB) are turned into bytes with the copy-calibration scales:
    bytes that miss the L2 (what HBM and the memory-side cache serve, an upper
    bound on HBM traffic); with a --kernel-trace CSV, the mean duration
    (dispatches on `stream` only, if given) and the L2-miss rate
    (fetch + write) / duration are added."""
    import csv

    acc, counters = {}, []
    for p in paths:
        rows = list(csv.DictReader(open(p)))
        tags = op_tags(rows, "Queue_Id", lambda r: int(r["Grid_Size"]))
        for r in rows:
            key = (short_kernel(r["Kernel_Name"]) + tags.get(r["Dispatch_Id"], ""), int(r["Grid_Size"]))
            c = r["Counter_Name"]
            if c not in counters:
                counters.append(c)
            d = acc.setdefault(key, {}).setdefault(c, {})
            d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    dur = {}
    if trace:
        grid = lambda r: int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])  # noqa: E731
        rows = [r for r in csv.DictReader(open(trace))
                if stream is None or r["Stream_Id"] == str(stream)]
        tags = op_tags(rows, "Stream_Id", grid)
        for r in rows:
            dur.setdefault((short_kernel(r["Kernel_Name"]) + tags.get(r["Dispatch_Id"], ""), grid(r)),
                           []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    cols = [c for c in counters if c not in ("FETCH_SIZE", "WRITE_SIZE")]
    head = ["kernel", "tile", "grid (work-items)", "dispatches"]
    if trace:
        head += ["mean us (trace)"]
    head += ["L2-miss read MB", "L2-miss write MB"] + (["L2-miss GB/s"] if trace else []) + cols
    lines = ["| " + " | ".join(head) + " |", "|---|" + "---:|" * (len(head) - 1)]
    rows = []
    for (k, g), d in sorted(acc.items()):
        n = max(len(v) for v in d.values())
        rd = mean(d["FETCH_SIZE"].values()) * 1024 * fetch_scale if "FETCH_SIZE" in d else None
        wr = mean(d["WRITE_SIZE"].values()) * 1024 * write_scale if "WRITE_SIZE" in d else None
        us = mean(dur[(k, g)]) if (k, g) in dur else None
        cells = [f"`{k}`", tile_id(k), f"{g:,}", str(n)]
        if trace:
            cells.append(f"{us:.2f}" if us else "")
        cells += [f"{rd / 1e6:.2f}" if rd is not None else "", f"{wr / 1e6:.2f}" if wr is not None else ""]
        if trace:
            cells.append(f"{(rd + wr) / (us * 1e-6) / 1e9:,.0f}" if us and rd is not None and wr is not None
                         else "")
        cells += [f"{mean(d[c].values()):,.2f}" if c in d else "" for c in cols]
        lines.append("| " + " | ".join(cells) + " |")
        rows.append({"kernel": k, "grid": g, "dispatches": n, "us": us, "read": rd, "write": wr})
    return "\n".join(lines), rows


def trace_summary(trace, stream):
    """Per (kernel class, grid) of a rocprofv3 --kernel-trace CSV:
    dispatches, mean duration on Stream_Id `stream` and on the other
    streams, share of all kernel time; residual GEMMs tagged by op
    (op_tags).  A markdown table, largest share first."""
    import csv

    rows = list(csv.DictReader(open(trace)))
    grid = lambda r: int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])  # noqa: E731
    tags = op_tags(rows, "Stream_Id", grid)
    acc, total = {}, 0.0
    for r in rows:
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        total += us
        c = acc.setdefault((short_kernel(r["Kernel_Name"]) + tags.get(r["Dispatch_Id"], ""), grid(r)),
                           {"n": 0, "sum": 0.0, "own": [], "other": []})
        c["n"] += 1
        c["sum"] += us
        c["own" if r["Stream_Id"] == str(stream) else "other"].append(us)
    mean = lambda v: f"{sum(v) / len(v):.2f}" if v else ""  # noqa: E731
    lines = ["| kernel | grid (work-items) | dispatches | mean us, timing stream | "
             "mean us, concurrent streams | % of kernel time |", "|---|---:|---:|---:|---:|---:|"]
    for (k, g), c in sorted(acc.items(), key=lambda kv: -kv[1]["sum"]):
        lines.append(f"| `{k}` | {g:,} | {c['n']} | {mean(c['own'])} | {mean(c['other'])} | "
                     f"{100 * c['sum'] / total:.1f} |")
    return "\n".join(lines)


# (tile id, M, N, K, epilogue): a shape at which bbh_linear (epilogue "bias" /
# "gelu") or bbh_linear_residual_layernorm ("ln") launches that tile, for the
# tile configurations the forwards pick (1 is picked only beside other
# forwards: the per-batch pass on several slots).
TILE_SHAPES = [(0, 1024, 1536, 384, "gelu"), (26, 1024, 384, 384, "bias"),
               (34, 3072, 384, 1536, "bias"),
               (30, 1024, 1152, 384, "bias"), (31, 8192, 384, 1536, "bias"),
               (32, 16384, 384, 1536, "bias"), (19, 32768, 384, 1536, "bias"),
               (14, 16384, 384, 1536, "ln"),
               (28, 32768, 384, 384, "ln"), (18, 32768, 384, 1536, "ln"),
               (33, 32768, 1152, 384, "bias")]


def run_tiles(torch, engine, steps, warmup):
    """Each TILE_SHAPES launch, timed alone: {"tile M N K epi": us}."""
    gen = torch.Generator(device="cuda").manual_seed(3)
    h = lambda *shape: (torch.randn(*shape, device="cuda", generator=gen) * 0.5).half()  # noqa: E731
    out = {}
    for tile, M, N, K, epi in TILE_SHAPES:
        A, W, b = h(M, K), h(N, K), h(N)
        C = torch.empty((M, N), dtype=torch.float16, device="cuda")
        if epi == "ln":
            r, g, be = h(M, N), torch.ones(N, dtype=torch.float16, device="cuda"), h(N)
            fn = lambda: engine.launch_linear_residual_layernorm(A, W, b, r, g, be, C, M, K)  # noqa: E731,E501
        else:
            fn = lambda: engine.launch_matmul(A, W, C, M, N, K, bias=b, gelu=epi == "gelu")  # noqa: E731
        out[f"{tile} {M}x{N}x{K} {epi}"] = round(timed(torch, fn, steps, warmup) * 1e3, 2)
    return out


def run_cfg5(torch, engine, synth, model, ws):
    """batch 256 x seq 512 through bert_embed; the encoder layer's
    GEMM launches at M = 131072 as the forward makes them (QKV, O-proj +
    LayerNorm, and the FFN block, which from 65536 rows is one kernel for both
    of its Linears), each timed on its own: their FLOPs over their summed time
    is the fraction of the fp16 dense MFMA peak; the two FFN Linears as
    separate kernels are reported beside it.  Then the same batch through
    bbh_embed_packed (valid tokens only)."""
    M = 131072
    buf = gemm_buffers(torch, M)
    ids, types, mask = (torch.from_numpy(a).cuda() for a in synth.long_batch())
    emb5 = torch.empty((256, 384), dtype=torch.float16, device="cuda")
    ms = timed(torch, lambda: engine.bert_embed(ws, model, ids, types, mask, emb=emb5), 10,
               warmup=2)
    gem, sep = {}, {}
    for name, N, K, epi in LAYER_GEMMS:
        fn = gemm_runner(torch, engine, model, M, N, K, epi, buf)
        t = timed(torch, fn, 10, warmup=2)
        f = 2.0 * M * N * K
        sep[name] = (t, f)
        gem[name] = round(f / (t / 1e3) / PEAK_FP16_DENSE, 4)
    # the FFN block as the forward runs it (layer 0 of the model, synthetic input rows)
    hid = buf["R"][: M * 384].view(M, 384)
    out = buf["C"][: M * 384].view(M, 384)
    t_ffn = timed(torch, lambda: engine.ffn_block(ws, model, 0, hid, out, 256, 512), 10, warmup=2)
    f_ffn = sep["ffn1_gelu"][1] + sep["ffn2_ln"][1]
    gem["ffn_block"] = round(f_ffn / (t_ffn / 1e3) / PEAK_FP16_DENSE, 4)
    gemm_ms = sep["qkv"][0] + sep["o_proj_ln"][0] + t_ffn
    gemm_flops = sep["qkv"][1] + sep["o_proj_ln"][1] + f_ffn
    two = sum(t for t, _ in sep.values())
    del buf
    # lengths uniform in [256, 512]: about 3/4 of the padded rows are valid
    pk5 = engine.PackedBatches([synth.long_batch()])
    pool5 = engine.Pool(1, 256, 512)
    ms_p5 = timed(torch, lambda: engine.embed_packed(pool5, model, pk5, emb=emb5), 10, warmup=2)
    pool5.close()
    res = {
        "sentences_per_s": round(256 / (ms / 1e3), 1), "ms_per_forward": round(ms, 3),
        "packed_sentences_per_s": round(256 / (ms_p5 / 1e3), 1),
        "packed_valid_tokens": int(pk5.lengths.sum()),
        "tflops": round(synth.flops_per_forward(256, 512) / (ms / 1e3) / 1e12, 2),
        "fused_gemms_frac_of_fp16_peak": round(gemm_flops / (gemm_ms / 1e3) / PEAK_FP16_DENSE, 4),
        "fused_gemms_frac_ffn_as_two_kernels": round(gemm_flops / (two / 1e3) / PEAK_FP16_DENSE, 4),
        "layer_gemm_us": round(gemm_ms * 1e3, 1),
        "per_gemm_frac": gem}
    log("cfg5", res)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-extras", action="store_true", help="only the varlen workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only time a device-to-device copy of BYTES (the calibration kernel "
                         "for the L2-miss byte counters, and the practical copy bandwidth)")
    ap.add_argument("--only", choices=["varlen", "varlen1", "packed", "merged", "cfg2", "cfg3",
                                       "cfg5", "tiles"],
                    default=None,
                    help="only this workload, without the event-timed roofline pass (for "
                         "rocprofv3 counter runs); prints its dict")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV", default=None,
                    help="no GPU work: summarise rocprofv3 --pmc counter_collection CSVs per "
                         "kernel class and grid size as a markdown table")
    ap.add_argument("--trace", metavar="CSV", default=None,
                    help="with --pmc-summary: a rocprofv3 kernel_trace CSV for mean durations")
    ap.add_argument("--trace-summary", metavar="CSV", default=None,
                    help="print per-kernel-class times of a rocprofv3 kernel_trace CSV "
                         "(--trace-stream: the Stream_Id of the pass to single out) and exit")
    ap.add_argument("--trace-stream", default=None,
                    help="with --trace: only dispatches of this Stream_Id")
    ap.add_argument("--scales", nargs=2, type=float, default=(1.0, 1.0), metavar=("FETCH", "WRITE"),
                    help="with --pmc-summary: bytes per reported FETCH_SIZE / WRITE_SIZE byte, "
                         "from the same counters on the --copy-probe copy")
    ap.add_argument("--traffic-json", metavar="OUT", default=None,
                    help="with --pmc-summary: also write each kernel class's L2-miss bytes per "
                         "dispatch (fetch + write, dispatch-weighted over its grids) to OUT")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.trace_stream))
        return
    if args.pmc_summary:
        table, rows = pmc_summary(args.pmc_summary, args.trace, args.scales[0], args.scales[1],
                                  args.trace_stream)
        print(table)
        if args.traffic_json:
            cls = {}
            for r in rows:
                if r["read"] is None or r["write"] is None:
                    continue
                c = cls.setdefault(r["kernel"], {})
                c[str(r["grid"])] = round(r["read"] + r["write"])
            json.dump({"source": " ".join(sys.argv), "fetch_scale": args.scales[0],
                       "write_scale": args.scales[1],
                       "kernels": [{"class": k, "grid_bytes": v} for k, v in sorted(cls.items())]},
                      open(args.traffic_json, "w"), indent=1)
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; the embedding path is pure data "
              "parallel (whole batches per GPU, no collectives), so N>1 is not run.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from bbh import engine, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.copy_probe:
        n = args.copy_probe // 2
        src = torch.ones(n, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        ms = timed(torch, lambda: dst.copy_(src), 5, warmup=2)
        print(json.dumps({"copy_bytes": 2 * n, "ms": round(ms, 4),
                          "read_plus_write_GB_per_s": round(4 * n / (ms / 1e3) / 1e9, 1)}),
              flush=True)
        return
    weights = synth.make_weights(0)
    model = engine.Model.from_weights(weights)
    if args.only in ("varlen", "varlen1"):  # the default workload's pass alone (varlen1: the
        # one-slot pass whose launches the roofline times)
        slots = EACH_STREAMS if args.only == "varlen" else 1
        batches = synth.varlen_mix()
        pk = engine.PackedBatches([b[:3] for b in batches])
        emb_all = torch.empty((pk.rows, 384), dtype=torch.float16, device="cuda")
        pool = engine.Pool(slots, 64, 64)
        ms, _ = pass_timer(torch, lambda: engine.embed_each(pool, model, pk, emb=emb_all),
                           args.steps, args.warmup)
        pool.close()
        model.close()
        print(json.dumps({"workload": "varlen per-batch pass", "streams": slots,
                          "ms_per_pass": round(ms, 4), "sentences_per_s": round(2000 / (ms / 1e3), 1)}),
              flush=True)
        return
    if args.only == "tiles":  # one kernel-level launch per tile configuration the product picks
        print(json.dumps(run_tiles(torch, engine, args.steps, args.warmup)), flush=True)
        model.close()
        return
    if args.only in ("packed", "merged"):  # the varlen mix through bbh_embed_packed / _batches
        batches = synth.varlen_mix()
        pkg = engine.PackedBatches([b[:3] for b in batches], group_by_seq=True)
        emb_all = torch.empty((pkg.rows, 384), dtype=torch.float16, device="cuda")
        ppool = engine.Pool(1, POOL_BATCH, 64)
        run = engine.embed_packed if args.only == "packed" else engine.embed_batches
        ms, _ = pass_timer(torch, lambda: run(ppool, model, pkg, emb=emb_all), args.steps,
                           args.warmup)
        ppool.close()
        model.close()
        print(json.dumps({"workload": f"varlen mix, bbh_embed_{'packed' if args.only == 'packed' else 'batches'}",
                          "ms_per_pass": round(ms, 4), "sentences_per_s": round(2000 / (ms / 1e3), 1)}),
              flush=True)
        return
    if args.only in ("cfg2", "cfg3"):  # configs[1] / configs[2]: bert_embed, batch 64
        seq = 16 if args.only == "cfg2" else 128
        ws = engine.Workspace(64, seq)
        ids, types, mask = (torch.from_numpy(a).cuda() for a in synth.cfg_fixed(64, seq))
        emb = torch.empty((64, 384), dtype=torch.float16, device="cuda")
        ms = timed(torch, lambda: engine.bert_embed(ws, model, ids, types, mask, emb=emb),
                   args.steps, warmup=args.warmup)
        print(json.dumps({"workload": f"{args.only}: bert_embed batch 64 x seq {seq}",
                          "ms_per_forward": round(ms, 4),
                          "sentences_per_s": round(64 / (ms / 1e3), 1)}), flush=True)
        ws.close()
        model.close()
        return
    if args.only == "cfg5":
        ws = engine.Workspace(256, 512)
        print(json.dumps(run_cfg5(torch, engine, synth, model, ws)), flush=True)
        ws.close()
        model.close()
        return

    # ---- default workload: varlen mix, one bert_embed per batch ------------
    # The 32 consecutive batches of 64, each at its own padded round16 length,
    # pre-uploaded back to back; one step = bert_embed on every batch
    # (bbh_embed_each: one forward per batch, nothing merged, every padding
    # row computed), the batches spread over EACH_STREAMS pool slots (the last
    # one on the caller's stream).
    batches = synth.varlen_mix()
    n_sent = sum(b[0].shape[0] for b in batches)
    padded_rows = int(sum(b[0].size for b in batches))
    pk = engine.PackedBatches([b[:3] for b in batches])  # consecutive order, as given
    real_tokens = int(pk.lengths.sum())
    emb_all = torch.empty((pk.rows, 384), dtype=torch.float16, device="cuda")
    # Workspaces for seq up to 128, so the corpus modes below use the same
    # pools: HIP maps streams to hardware queues in creation order, and more
    # pools would put two busy streams on one queue.
    pool = engine.Pool(EACH_STREAMS, 64, 128)
    ms_step, wall = pass_timer(torch, lambda: engine.embed_each(pool, model, pk, emb=emb_all),
                               args.steps, args.warmup)
    sps = n_sent / (ms_step / 1e3)
    pad_flops = sum(synth.flops_per_forward(b[0].shape[0], b[3]) for b in batches)
    log(f"varlen per-batch bert_embed ({EACH_STREAMS} streams, {padded_rows} padded rows): "
        f"{ms_step:.3f} ms/pass ({wall:.3f} ms wall), {sps:,.0f} sent/s, "
        f"{pad_flops / (ms_step / 1e3) / 1e12:.1f} TFLOP/s executed")

    pool1 = engine.Pool(1, 64, 128)
    ms1, _ = pass_timer(torch, lambda: engine.embed_each(pool1, model, pk, emb=emb_all),
                        args.steps, args.warmup // 2)
    log(f"varlen per-batch bert_embed (1 stream): {ms1:.3f} ms/pass, {n_sent / (ms1 / 1e3):,.0f} sent/s")

    out = {
        "metric": "sentences/sec (batch 64, seq 16/128 + varlen mix); % of MFMA fp16 peak",
        "value": round(sps, 1), "unit": "sentences/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded random-init MiniLM-L6 weights N(0,0.02), synthetic token ids)",
        "config": {"workload": "varlen mix (BASELINE configs[3]): 2000 sentences, "
                               "lognormal(median 12, sigma 0.5) lengths clipped to [5,64], 32 "
                               "consecutive batches of 64 in seeded order, each padded to "
                               f"round16(max) (eff 32/48/64, {padded_rows} padded rows, "
                               f"{real_tokens} valid tokens); one step = one bert_embed per "
                               "batch at its padded length (bbh_embed_each: nothing merged, "
                               "every padding row computed), the 32 forwards spread over "
                               f"{EACH_STREAMS} concurrent HIP streams ({EACH_STREAMS - 1} pool "
                               "streams and the caller's) with one workspace each",
                   "streams": EACH_STREAMS,
                   "model": "MiniLM-L6 (6 layers, hidden 384, 12x32 heads, FFN 1536)",
                   "global_batch": 64,
                   "seq_len": f"5..64 valid ({real_tokens / n_sent:.1f} mean), padded 32/48/64",
                   "parallelism": "single GPU"},
        "ms_per_sentence": round(ms_step / n_sent, 6),
        "executed_tflops": round(pad_flops / (ms_step / 1e3) / 1e12, 2),
        "varlen_per_batch_1stream_sentences_per_s": round(n_sent / (ms1 / 1e3), 1),
        "varlen_per_batch_1stream_ms_per_pass": round(ms1, 4),
    }

    # ---- dominant kernel of the default workload ---------------------------
    # The same per-batch pass on a one-slot pool with per-launch timing: a
    # pair of HIP events on the caller's stream around every op launch, so each
    # pair brackets that kernel alone with no other stream sharing the GPU.
    n_ops = 32 * (2 + 6 * 7)
    pool1.timing(n_ops)
    engine.embed_each(pool1, model, pk, emb=emb_all)  # warm (records overwritten below)
    torch.cuda.synchronize()
    tsteps = max(5, args.steps // 5)
    pool1.timing(n_ops * tsteps)
    for _ in range(tsteps):
        engine.embed_each(pool1, model, pk, emb=emb_all)
    recs = pool1.timing_read()
    pool1.timing(0)
    classes = classify(engine, recs, tsteps)
    dom = classes[0]
    traffic = None
    tfile = os.path.join(PROFILES, "dominant_kernel_traffic.json")
    if os.path.exists(tfile):  # L2-miss bytes per dispatch of each class in a --pmc run of this pass
        # Residual GEMM rows carry the op (op_tags): O-proj and FFN2 may share
        # kernel and grid.
        tag = {"o_proj_ln": " [o_proj]", "ffn2_ln": " [ffn2]"}.get(dom["op"], "")
        g = str(dom["grid_items"])
        for name in (dom["class"] + tag, dom["class"]):
            for t in json.load(open(tfile)).get("kernels", []):
                if traffic is None and t.get("class") == name and g in t.get("grid_bytes", {}):
                    traffic = t["grid_bytes"][g]
    # The roof that binds: the kernel's arithmetic intensity (FLOPs over the
    # measured L2-miss bytes where a counter run gave them, else over the
    # algorithmic bytes) against the ridge point PEAK_FP16_DENSE / PEAK_HBM.
    flops, byts = dom["algorithmic_flops_per_launch"], dom["algorithmic_bytes_per_launch"]
    ai = flops / (traffic or byts)
    ridge = PEAK_FP16_DENSE / PEAK_HBM
    gemm = ai >= ridge
    ach = dom["tflops"] if gemm else dom["gb_per_s"]
    peak = PEAK_FP16_DENSE / 1e12 if gemm else PEAK_HBM / 1e9
    out["roofline"] = {
        "bound": "mfma" if gemm else "hbm", "achieved": ach, "peak": peak,
        "unit": "TFLOP/s" if gemm else "GB/s", "frac": round(ach / peak, 4), "traffic": traffic,
        "flop_per_byte": round(ai, 1), "ridge_flop_per_byte": round(ridge, 1),
        "attainable_tflops": round(min(PEAK_FP16_DENSE, ai * PEAK_HBM) / 1e12, 1),
        "frac_of_mfma_peak": round(dom["tflops"] / (PEAK_FP16_DENSE / 1e12), 4),
        "kernel": dom["kernel"], "op": dom["op"], "m": dom["m"], "grid_items": dom["grid_items"],
        "launches_per_step": dom["launches_per_step"], "avg_launch_us": dom["avg_launch_us"],
        "algorithmic_flops_per_launch": dom["algorithmic_flops_per_launch"],
        "algorithmic_bytes_per_launch": dom["algorithmic_bytes_per_launch"],
        "share_of_op_time": dom["share_of_op_time"],
        "timing": f"one-slot pool on the caller's stream, event pair per launch, {tsteps} passes"}
    out["kernel_classes"] = classes[:12]
    log("roofline", out["roofline"])
    for c in classes[:12]:
        log("  ", c)

    if not args.no_extras:
        # ---- the reference corpus benchmark's two modes on the same sentences
        sb, order = synth.varlen_sorted()
        pb = synth.varlen_padded()
        for tag, bl, desc in (
                ("corpus_sorted_dynamic", sb, "sentences stable-sorted by length, batches of 64 "
                 "at max(16, round16(longest)) (bench/corpus.cu:79-132)"),
                ("corpus_padded_128", pb, "consecutive batches of 64 at seq 128 "
                 "(bench/corpus.cu:64-77)")):
            pkc = engine.PackedBatches([b[:3] for b in bl])
            cp, cp1 = pool, pool1
            msc, _ = pass_timer(torch, lambda: engine.embed_each(cp, model, pkc, emb=emb_all),
                                args.steps, args.warmup // 2)
            msc1, _ = pass_timer(torch, lambda: engine.embed_each(cp1, model, pkc, emb=emb_all),
                                 max(10, args.steps // 2), 10)
            fl = sum(synth.flops_per_forward(b[0].shape[0], b[3]) for b in bl)
            out[tag] = {"sentences_per_s": round(n_sent / (msc / 1e3), 1), "streams": EACH_STREAMS,
                        "ms_per_pass": round(msc, 4),
                        "sentences_per_s_1stream": round(n_sent / (msc1 / 1e3), 1),
                        "padded_rows": int(sum(b[0].size for b in bl)),
                        "executed_tflops": round(fl / (msc / 1e3) / 1e12, 2), "batching": desc}
            log(tag, out[tag])

        # ---- the same sentences without padding, and with equal-seq batches merged
        pkg = engine.PackedBatches([b[:3] for b in batches], group_by_seq=True)
        ppool = engine.Pool(1, POOL_BATCH, 64)
        ms_p, _ = pass_timer(torch, lambda: engine.embed_packed(ppool, model, pkg, emb=emb_all),
                             args.steps, args.warmup)
        ms_m, _ = pass_timer(torch, lambda: engine.embed_batches(ppool, model, pkg, emb=emb_all),
                             args.steps, args.warmup // 2)
        ppool.close()
        valid_flops = sum(synth.flops_per_forward(1, int(L)) for L in pkg.lengths)
        out["varlen_packed"] = {
            "sentences_per_s": round(n_sent / (ms_p / 1e3), 1), "ms_per_pass": round(ms_p, 4),
            "executed_tflops": round(valid_flops / (ms_p / 1e3) / 1e12, 2),
            "what": f"bbh_embed_packed: only the {real_tokens} valid tokens enter one forward "
                    "(no padding rows), same embeddings as the padded batches"}
        out["varlen_merged_padded"] = {
            "sentences_per_s": round(n_sent / (ms_m / 1e3), 1), "ms_per_pass": round(ms_m, 4),
            "what": "bbh_embed_batches: runs of equal-seq batches merged into one forward per "
                    "run (one stream), every padding row computed"}
        log("packed", out["varlen_packed"], "merged", out["varlen_merged_padded"])

        ws = engine.Workspace(256, 512)
        emb = torch.empty((64, 384), dtype=torch.float16, device="cuda")
        # ---- batch 64 x seq 16 / 128 ----------------
        for tag, seq in (("cfg2_b64_s16", 16), ("cfg3_b64_s128", 128)):
            ids, types, mask = (torch.from_numpy(a).cuda() for a in synth.cfg_fixed(64, seq))
            ms = timed(torch, lambda: engine.bert_embed(ws, model, ids, types, mask, emb=emb), 300,
                       warmup=20)
            # the same forward captured once as a HIP graph and replayed
            graph = engine.EmbedGraph(ws, model, ids, types, mask, emb)
            ms_g = timed(torch, graph.launch, 300, warmup=20)
            graph.close()
            out[tag] = {"sentences_per_s": round(64 / (ms / 1e3), 1),
                        "ms_per_sentence": round(ms / 64, 6),
                        "tflops": round(synth.flops_per_forward(64, seq) / (ms / 1e3) / 1e12, 2),
                        "graph_sentences_per_s": round(64 / (ms_g / 1e3), 1),
                        "graph_ms_per_sentence": round(ms_g / 64, 6)}
            log(tag, out[tag])
        # ---- the reference's batch sweep (bench/bench.cu:86-96): one 9-token
        # sentence tiled over batch 1, 8, 32, 64 at seq 128 (padded) and at
        # its effective length 16, bert_embed 300 times after 20 warmups
        sweep = {}
        for seq in (128, 16):
            for bsz in (1, 8, 32, 64):
                ids, types, mask = (torch.from_numpy(a).cuda() for a in synth.cfg_fixed(bsz, seq))
                ms = timed(torch, lambda: engine.bert_embed(ws, model, ids, types, mask,
                                                            emb=emb[:bsz]), 300, warmup=20)
                # the same forward captured once as a HIP graph and replayed
                graph = engine.EmbedGraph(ws, model, ids, types, mask, emb[:bsz])
                ms_g = timed(torch, graph.launch, 300, warmup=20)
                graph.close()
                sweep[f"seq{seq}_b{bsz}"] = {"ms_per_sentence": round(ms / bsz, 6),
                                             "sentences_per_s": round(bsz / (ms / 1e3), 1),
                                             "graph_ms_per_sentence": round(ms_g / bsz, 6)}
        out["batch_sweep"] = sweep
        log("batch sweep", sweep)
        out["cfg5_b256_s512"] = run_cfg5(torch, engine, synth, model, ws)
        ws.close()
        out["tokenizer"] = tokenizer_rate(engine, synth)
        log("tokenizer", out["tokenizer"])

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(batches, weights)
        log("cpu baseline", out["cpu_baseline"])
    else:
        out["cpu_baseline"] = None

    pool.close()
    pool1.close()
    model.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
