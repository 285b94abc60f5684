"""Throughput of bert_embed on one MI355X, in the driver's JSON-line format.

Default workload: the synthetic varlen mix - 2000
sentences, lognormal lengths clipped to [5, 64], consecutive batches of 64 in
seeded order, each padded to round16(longest) (32 batches, eff 32/48/64).
One step = one pass of bert_embed over all 32 pre-uploaded batches (the
reference times passes over its corpus the same way, bench/corpus.cu:120-132),
through bbh_embed_packed: only each sentence's valid tokens enter the forward
(26,857 of the 91,648 padded rows), as one forward on N_STREAMS stream(s).
The embeddings are those of the padded computation (bbh_embed_batches, which
runs every padded row) bit for bit; that path is timed too and reported as
varlen_padded_sentences_per_s.  value = sentences/s over the K timed steps.

Defaults: W = 200 untimed warmup steps, K = 100 timed steps (~0.4 s of GPU
work together).  The MI355X reaches its sustained clock only after some
100 ms of continuous load: from a fresh process, 3 warmup steps measured
1.50M sent/s and 200 measured 1.75M on the same box, in either order.

The same line also carries, as extra fields: configs[1] (batch 64 x seq 16)
and configs[2] (batch 64 x seq 128) sent/s (300 timed iterations as
bench/bench.cu:32-51), configs[4] (batch 256 x seq 512) sent/s with the
fused GEMMs' fraction of the fp16 dense MFMA peak, the roofline of the
dominant kernel of the default workload (the same packed runs through a
one-stream pool, timed live with an event pair around each launch on that
stream, so no other stream's kernels share the GPU during a launch), and the
CPU baseline (the fp32 numpy oracle on a bounded sample, on this host's
cores).
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

N_STREAMS = 1  # forwards of the packed varlen pass (one workspace per stream)
PAD_STREAMS = 2  # concurrent forwards of the padded varlen pass
POOL_BATCH = 1024  # workspace rows per stream = POOL_BATCH * 64: the 21 batches of
#                    padded length 48 (64,512 rows) run as one padded forward
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


def cpu_baseline(batches, weights, budget_s=12.0):
    """The fp32 numpy oracle (the reference's fp32 torch forward restated) on
    the first batches of the same workload, until ~budget_s of CPU work."""
    from oracle import bert_oracle as O

    try:
        from threadpoolctl import threadpool_info

        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        cores = os.cpu_count() or 1
    O.bert_embed(weights, *batches[0][:3])  # warm
    n_sent, t0, used = 0, time.perf_counter(), 0
    for ids, types, mask, _ in batches:
        O.bert_embed(weights, ids, types, mask)
        n_sent += ids.shape[0]
        used += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": round(n_sent / dt, 1), "unit": "sentences/s", "cores": int(cores),
            "kind": "port",
            "sample": f"fp32 numpy oracle bert_embed over the first {used} batches "
                      f"({n_sent} sentences) of the varlen mix, {dt:.1f} s"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-extras", action="store_true", help="only the varlen workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only time a device-to-device copy of BYTES (the calibration kernel "
                         "for the HBM byte counters, and the practical copy bandwidth)")
    args = ap.parse_args()

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
    ws = engine.Workspace(256, 512)

    # ---- default workload: varlen mix ------------------------------------
    # All 32 batches pre-uploaded; bert_embed on every batch through
    # bbh_embed_packed (valid tokens only) on a pool of N_STREAMS streams.
    batches = synth.varlen_mix()
    n_sent = sum(b[0].shape[0] for b in batches)
    packed = engine.PackedBatches([b[:3] for b in batches], group_by_seq=True)
    real_tokens = int(packed.lengths.sum())
    padded_rows = int(sum(b[0].size for b in batches))
    pool = engine.Pool(N_STREAMS, POOL_BATCH, 64)
    emb_all = torch.empty((packed.rows, 384), dtype=torch.float16, device="cuda")

    def step():
        engine.embed_packed(pool, model, packed, emb=emb_all)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s_ev.record()
    for _ in range(args.steps):
        step()
    e_ev.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = s_ev.elapsed_time(e_ev) / args.steps
    sps = n_sent / (ms_step / 1e3)
    # algorithmic FLOPs over the valid tokens (what the packed pass executes)
    total_flops = sum(synth.flops_per_forward(1, int(L)) for L in packed.lengths)
    log(f"varlen packed ({N_STREAMS} stream(s), {real_tokens} of {padded_rows} rows): "
        f"{ms_step:.3f} ms/pass ({wall / args.steps * 1e3:.3f} ms wall), {sps:,.0f} sent/s, "
        f"{total_flops / (ms_step / 1e3) / 1e12:.1f} TFLOP/s executed")

    # the padded computation (every padded row) through bbh_embed_batches
    ppool = engine.Pool(PAD_STREAMS, POOL_BATCH, 64)
    ms_pad = timed(torch, lambda: engine.embed_batches(ppool, model, packed, emb=emb_all),
                   args.steps, warmup=args.warmup)
    ppool.close()
    pad_flops = sum(synth.flops_per_forward(b[0].shape[0], b[3]) for b in batches)
    log(f"varlen padded ({PAD_STREAMS} streams, {padded_rows} rows): {ms_pad:.3f} ms/pass, "
        f"{n_sent / (ms_pad / 1e3):,.0f} sent/s, "
        f"{pad_flops / (ms_pad / 1e3) / 1e12:.1f} TFLOP/s executed")

    # the same workload as one bert_embed per batch on a single stream
    dev = [(torch.from_numpy(i).cuda(), torch.from_numpy(t).cuda(), torch.from_numpy(m).cuda())
           for i, t, m, _ in batches]
    emb = torch.empty((64, 384), dtype=torch.float16, device="cuda")

    def step1():
        for i, t, m in dev:
            engine.bert_embed(ws, model, i, t, m, emb=emb[: i.shape[0]])

    ms1 = timed(torch, step1, args.steps, warmup=args.warmup)
    log(f"varlen (1 stream): {ms1:.3f} ms/pass, {n_sent / (ms1 / 1e3):,.0f} sent/s")

    out = {
        "metric": "sentences/sec (batch 64, seq 16/128 + varlen mix); % of MFMA fp16 peak",
        "value": round(sps, 1), "unit": "sentences/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded random-init MiniLM-L6 weights N(0,0.02), synthetic token ids)",
        "config": {"workload": "varlen mix: 2000 sentences, lognormal(median 12, sigma 0.5) "
                               "lengths clipped to [5,64], consecutive batches of 64 padded to "
                               f"round16(max) ({padded_rows} padded rows, {real_tokens} valid "
                               "tokens); one step = bert_embed over all 32 batches via "
                               "bbh_embed_packed: only valid tokens enter the forward (one "
                               f"forward of {real_tokens} rows on {N_STREAMS} stream(s)); the "
                               "embeddings equal the padded computation's (bbh_embed_batches) "
                               "bit for bit",
                   "streams": N_STREAMS, "pool_rows_per_stream": POOL_BATCH * 64,
                   "model": "MiniLM-L6 (6 layers, hidden 384, 12x32 heads, FFN 1536)",
                   "global_batch": 64,
                   "seq_len": f"5..64 valid ({real_tokens / n_sent:.1f} mean), padded 32/48/64",
                   "parallelism": "single GPU"},
        "ms_per_sentence": round(ms_step / n_sent, 6),
        "varlen_padded_sentences_per_s": round(n_sent / (ms_pad / 1e3), 1),
        "varlen_padded_streams": PAD_STREAMS,
        "varlen_single_stream_sentences_per_s": round(n_sent / (ms1 / 1e3), 1),
        "executed_tflops": round(total_flops / (ms_step / 1e3) / 1e12, 2),
    }

    # ---- dominant kernel of the default workload ---------------------------
    # The same packed pass again, through a one-stream pool with per-launch
    # timing on: a pair of HIP events on the pool stream around every op
    # launch, so each event pair brackets that kernel alone.  The dominant
    # kernel is the (op, tile) class with the largest summed time per pass.
    tpool = engine.Pool(1, POOL_BATCH, 64)
    n_ops = 6 * (4 + 16)  # 4 GEMMs and up to 16 attention length classes per layer
    tpool.timing(n_ops * args.steps)
    engine.embed_packed(tpool, model, packed, emb=emb_all)  # warm (records overwritten below)
    torch.cuda.synchronize()
    tpool.timing(n_ops * args.steps)
    for _ in range(args.steps):
        engine.embed_packed(tpool, model, packed, emb=emb_all)
    recs = tpool.timing_read()
    tpool.timing(0)
    tpool.close()
    classes = {}
    for r in recs:
        key = (r["op"], r["tile"], r["fused_ln"])
        c = classes.setdefault(key, {"ms": 0.0, "n": 0, "flops": 0.0, "bytes": 0.0, "m": set()})
        c["ms"] += r["ms"]
        c["n"] += 1
        c["m"].add(r["m"])
        if r["op"] == "attention":
            pass  # packed: per sentence at its own length, set below per pass
        else:
            M, N, K = r["m"], r["n"], r["k"]
            c["flops"] += 2.0 * M * N * K
            extra = M * N * 2.0 if r["op"] in ("o_proj_ln", "ffn2_ln") else 0.0  # residual
            c["bytes"] += (M * K + N * K + M * N + N) * 2.0 + extra
    # attention launches once per 32-token length class; its work per pass is
    # 6 layers x the sum over sentences at their own lengths
    lens = packed.lengths.astype(np.float64)
    for (op, tile, fused), c in classes.items():
        if op == "attention":
            c["flops"] = args.steps * 6 * 4.0 * 12 * 32 * float((lens * lens).sum())
            c["bytes"] = args.steps * 6 * float(lens.sum()) * (3 * 384 + 384) * 2.0
    per_op = {}
    for (op, tile, fused), c in classes.items():
        per_op[op] = per_op.get(op, 0.0) + c["ms"] / args.steps

    def kernel_name(op, tile, fused):
        if op == "attention":
            return "attention_kernel"
        epi = EPI_OF_OP.get(op) or ("3 (bias+residual+LayerNorm)" if fused else
                                    "2 (bias+residual), then ln384_kernel")
        tname = engine.gemm_tile_name(tile)
        return (f"gemm_wres_kernel<{epi}>" if tname.startswith("WRes") else
                f"gemm_kernel<{tname}, {epi}>")

    key = max(classes, key=lambda k: classes[k]["ms"])
    op, tile, fused = key
    c = classes[key]
    avg_s = c["ms"] / c["n"] / 1e3
    ach = c["flops"] / c["n"] / avg_s
    kname = kernel_name(op, tile, fused)
    # HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE summary
    # (one entry per leading kernel class of the profiled run)
    traffic = None
    tfile = os.path.join(PROFILES, "dominant_kernel_traffic.json")
    if os.path.exists(tfile):
        for t in json.load(open(tfile)).get("kernels", []):
            if t.get("kernel") == kname and t.get("op") == op and t.get("m") == sorted(c["m"]):
                traffic = t["traffic_bytes_per_launch"]
    out["roofline"] = {
        "bound": "mfma", "achieved": round(ach / 1e12, 2), "peak": PEAK_FP16_DENSE / 1e12,
        "unit": "TFLOP/s", "frac": round(ach / PEAK_FP16_DENSE, 4), "traffic": traffic,
        "kernel": kname, "op": op, "m": sorted(c["m"]),
        "launches_per_step": c["n"] // args.steps,
        "avg_launch_us": round(avg_s * 1e6, 2),
        "algorithmic_flops_per_launch": round(c["flops"] / c["n"]),
        "algorithmic_bytes_per_launch": round(c["bytes"] / c["n"]),
        "share_of_op_time": round(c["ms"] / sum(v["ms"] for v in classes.values()), 3)}
    out["op_ms_per_step"] = {k: round(v, 4) for k, v in sorted(per_op.items())}

    top = sorted(classes, key=lambda k: -classes[k]["ms"])[:3]
    out["top_kernel_classes"] = [
        {"kernel": kernel_name(*k), "op": k[0], "m": sorted(classes[k]["m"]),
         "avg_launch_us": round(classes[k]["ms"] / classes[k]["n"] * 1e3, 2),
         "algorithmic_bytes_per_launch": round(classes[k]["bytes"] / classes[k]["n"]),
         "share_of_op_time": round(classes[k]["ms"] / sum(v["ms"] for v in classes.values()), 3)}
        for k in top]
    by_m = {}
    for r in recs:
        d = by_m.setdefault(r["op"], {}).setdefault(r["m"], [0.0, 0])
        d[0] += r["ms"]
        d[1] += 1
    out["op_us_per_launch_by_m"] = {op: {m: round(t / n * 1e3, 2) for m, (t, n) in sorted(d.items())}
                                    for op, d in sorted(by_m.items())}
    log("roofline", out["roofline"])
    log("op ms per step", out["op_ms_per_step"])
    log("op us per launch by M", out["op_us_per_launch_by_m"])

    buf = gemm_buffers(torch, 131072)
    if not args.no_extras:
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
        # ---- batch 256 x seq 512 ---------------------------------
        ids, types, mask = (torch.from_numpy(a).cuda() for a in synth.long_batch())
        emb5 = torch.empty((256, 384), dtype=torch.float16, device="cuda")
        ms = timed(torch, lambda: engine.bert_embed(ws, model, ids, types, mask, emb=emb5), 10,
                   warmup=2)
        gemm_ms, gemm_flops = 0.0, 0.0
        gem = {}
        for name, N, K, epi in LAYER_GEMMS:
            fn = gemm_runner(torch, engine, model, 131072, N, K, epi, buf)
            t = timed(torch, fn, 10, warmup=2)
            f = 2.0 * 131072 * N * K
            gem[name] = round(f / (t / 1e3) / PEAK_FP16_DENSE, 4)
            gemm_ms += t
            gemm_flops += f
        # the same batch through bbh_embed_packed (valid tokens only: lengths
        # uniform in [256, 512], so about 3/4 of the padded rows)
        pk5 = engine.PackedBatches([synth.long_batch()])
        pool5 = engine.Pool(1, 256, 512)
        ms_p5 = timed(torch, lambda: engine.embed_packed(pool5, model, pk5, emb=emb5), 10,
                      warmup=2)
        pool5.close()
        out["cfg5_b256_s512"] = {
            "sentences_per_s": round(256 / (ms / 1e3), 1), "ms_per_forward": round(ms, 3),
            "packed_sentences_per_s": round(256 / (ms_p5 / 1e3), 1),
            "packed_valid_tokens": int(pk5.lengths.sum()),
            "tflops": round(synth.flops_per_forward(256, 512) / (ms / 1e3) / 1e12, 2),
            "fused_gemms_frac_of_fp16_peak": round(gemm_flops / (gemm_ms / 1e3) / PEAK_FP16_DENSE, 4),
            "per_gemm_frac": gem}
        log("cfg5", out["cfg5_b256_s512"])

    if not args.no_extras:
        out["tokenizer"] = tokenizer_rate(engine, synth)
        log("tokenizer", out["tokenizer"])

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(batches, weights)
        log("cpu baseline", out["cpu_baseline"])
    else:
        out["cpu_baseline"] = None

    pool.close()
    ws.close()
    model.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
