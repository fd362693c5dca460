"""Benchmark: batch-1 decode tok/s of the 8B-shape Q4_K Llama (BASELINE config
5) and the Q4_K GEMV's achieved HBM bandwidth against MI355X's 8 TB/s.

One "step" is one decode token through the whole model (embedding, 32
layers, final norm, Q6_K output head, greedy argmax), replayed from a HIP
graph with the position on the device.  The timed region starts with the
weights resident in HBM and the 4096-token prompt already in the KV cache:
its first 4095 tokens go through ifr_llama2_prefill (MFMA GEMMs and causal
attention, in passes of up to 4096 tokens), which is timed on its own and
reported as config.prefill, the last through the first decode step.  The
prefill GEMMs dequantize the GGUF weight tiles inside the kernel (no f16
copy of the weights); config.prefill.ms_tile128 times the same prompt with
every product forced onto the 128 x 128-tile kernel.

Prints one JSON line.  Besides the decode rate it carries each decode
stage's time and HBM rate (config.stages), the exact-GEMV-path decode rate,
the sampled decode rate and the prefill.  Extra modes: --sweep (BASELINE
config 2 GEMV sweep, GB/s per format and shape), --attn (config 3 attention
GB/s), --pmc-sample / --pf-sample (workloads for rocprofv3 counter passes).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import inferi_amd as I  # noqa: E402

HBM_PEAK_GBS = 8000.0
ROT_BYTES = 640 << 20  # rotate over > 512 MB of distinct buffers: defeats the 256 MB MALL

CFG_8B = dict(n_layers=32, hidden=4096, ffn=14336, n_heads=32, n_kv_heads=8, vocab=128256, rope_theta=500000.0,
              rms_eps=1e-5)
CFG_C4 = dict(n_layers=22, hidden=2048, ffn=5632, n_heads=32, n_kv_heads=4, vocab=32000, rope_theta=10000.0,
              rms_eps=1e-5)


def make_ctx(args):
    """The library context with the options given by --opt KEY=VALUE."""
    ctx = I.LlmContext(0, args.code_object)
    for kv in args.opt:
        k, v = kv.split("=", 1)
        ctx.set_option(k, int(v))
    return ctx


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(dtype: int, rows: int, cols: int) -> int:
    """Algorithmic bytes of one GEMV: the weight blocks, x and y."""
    return rows * I.row_bytes(dtype, cols) + 4 * cols + 4 * rows


def decode_token_bytes(cfg: I.Llama2Config, ctx_len: float, mat=I.Q4_K, head=I.Q6_K) -> float:
    """Algorithmic HBM bytes of one decode token: every weight once, the f16
    KV cache up to the position, and the embedding row."""
    h, kv, f = cfg.hidden, cfg.kv_dim, cfg.ffn
    per_layer = (I.row_bytes(mat, h) * (h + 2 * kv + h + 2 * f) + I.row_bytes(mat, f) * h + 2 * 4 * h)
    weights = cfg.n_layers * per_layer + I.row_bytes(head, h) * cfg.vocab + 4 * h + I.row_bytes(mat, h)
    kv_bytes = cfg.n_layers * 2 * kv * 2 * ctx_len
    return weights + kv_bytes


def time_gemv(ctx: I.LlmContext, dtype: int, rows: int, cols: int, iters: int, seed: int = 0,
              keep_host: bool = False) -> dict:
    """Average launch time of the GEMV kernel the decode step uses
    (ifr_matmul_quant_xq on a pre-quantized x) over `iters` back-to-back
    launches, rotating through enough weight copies to defeat the MALL; and
    of ifr_matmul_quant as a caller sees it (x in f32, its quantization
    inside the call) over the same rotation.  keep_host: also return the
    first copy's bytes and x on the host (for the CPU baseline)."""
    n = rows * cols
    wbytes = rows * I.row_bytes(dtype, cols)
    copies = max(2, -(-ROT_BYTES // wbytes))
    tmp = ctx.alloc(n * 4)
    ctx.fill_normal(tmp, n, seed, 1, 0.0, 0.02)
    ws = []
    for _ in range(copies):
        b = ctx.alloc(wbytes)
        ctx.quantize(b, tmp, dtype, n)
        ws.append(b)
    tmp.free()
    xh = np.random.default_rng(seed).standard_normal(cols).astype(np.float32)
    x = ctx.upload(xh)
    xq = ctx.alloc(I.LlmContext.activation_bytes(cols))
    ctx.quantize_activation(xq, x, cols)  # once: the decode step's GEMVs get x quantized by its producer
    y = ctx.alloc(rows * 4)
    for i in range(copies):  # warm-up
        ctx.matmul_quant_xq(y, ws[i], dtype, rows, cols, xq)
        ctx.matmul_quant_assign(y, ws[i], dtype, rows, cols, x)
    ctx.sync()
    ctx.event_record(2)
    for i in range(iters):
        ctx.matmul_quant_xq(y, ws[i % copies], dtype, rows, cols, xq)
    ctx.event_record(3)
    ms = ctx.event_elapsed(2, 3)
    ctx.event_record(2)
    for i in range(iters):
        ctx.matmul_quant_assign(y, ws[i % copies], dtype, rows, cols, x)
    ctx.event_record(3)
    ms_f32 = ctx.event_elapsed(2, 3)
    host_w = ws[0].download(np.uint8, wbytes) if keep_host else None
    for b in ws:
        b.free()
    x.free()
    xq.free()
    y.free()
    us, us_f32 = ms * 1000.0 / iters, ms_f32 * 1000.0 / iters
    nbytes = gemv_bytes(dtype, rows, cols)
    return {"us": us, "bytes": nbytes, "gbs": nbytes / (us * 1e-6) / 1e9, "us_f32x": us_f32,
            "gbs_f32x": nbytes / (us_f32 * 1e-6) / 1e9, "host_w": host_w, "host_x": xh}


def cpu_threads(args) -> int:
    """Threads of the CPU baselines: --cpu-threads, else the cores this
    process may run on (at most 16, the GPU box's CPU share)."""
    if args.cpu_threads:
        return args.cpu_threads
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_median_ms(fn, runs: int) -> float:
    """One warm-up, then the median wall time of `runs` calls (ms)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1000.0)
    return float(np.median(ts))


MFMA_F16_PEAK = 2.5e15  # MI355X dense f16 matrix-core FLOP/s


SAMPLE_WARMUP = 4
EXACT_WARMUP = 3


def time_sampler(ctx: I.LlmContext, n: int, iters: int = 50) -> float:
    """Microseconds per ifr_sample call (T 0.7, top-p 0.95) on n logits of
    an N(0, 4^2) draw."""
    x = (np.random.default_rng(3).standard_normal(n) * 4).astype(np.float32)
    dl, dp = ctx.upload(x), ctx.alloc(n * 4)
    dc, di = ctx.upload(np.array([0.37], np.float32)), ctx.alloc(4)
    ctx.sample(dl, dp, n, 0.7, 0.95, dc, di)
    ctx.sync()
    ctx.event_record(6)
    for _ in range(iters):
        ctx.sample(dl, dp, n, 0.7, 0.95, dc, di)
    ctx.event_record(7)
    us = ctx.event_elapsed(6, 7) * 1000.0 / iters
    for b in (dl, dp, dc, di):
        b.free()
    return us


def prefill_flops(cfg: I.Llama2Config, n: int) -> float:
    """Algorithmic FLOPs of a prompt of n tokens: 2 per weight per token for
    the layer matrices, plus causal attention (q.k and p.v: 2 x 2 x hs per
    key per head, sum over t of t+1 keys); of the last layer only the Q/K/V
    product, since the prefill's product is the KV rows (its attention and
    FFN outputs feed nothing)."""
    hs = cfg.hidden // cfg.n_heads
    kv = cfg.n_kv_heads * hs
    qkv = cfg.hidden * (cfg.hidden + 2 * kv)
    mats = qkv + cfg.hidden * cfg.hidden + 3 * cfg.hidden * cfg.ffn
    attn = 4.0 * hs * cfg.n_heads * (n * (n + 1) / 2)
    return (cfg.n_layers - 1) * (2.0 * n * mats + attn) + 2.0 * n * qkv


STAGES = ("qkv", "attention", "attn_output", "ffn_gate_up", "ffn_down")
# the decode step's kernel behind each stage (Q4_K matrices, f16 cache, head size 128, 4 query heads per KV
# head; the library's default GEMV forms)
STAGE_KERNELS = {"qkv": "gemv_q4_k_qkv_one", "attention": "attn_f16_h128_g4 + attn_merge",
                 "attn_output": "gemv_q4_k_resid_r2w8k1", "ffn_gate_up": "gemv_q4_k_gateup_one4",
                 "ffn_down": "gemv_q4_k_resid_xf"}
ROOFLINE_STAGE = "ffn_gate_up"  # the decode step's dominant kernel


def stage_bytes(cfg: I.Llama2Config, stage: str, ctx_len: float, mat=I.Q4_K) -> int:
    """Algorithmic HBM bytes of one layer's decode stage: its weight blocks
    once, the vectors it reads and writes once (quantized activations at
    3.5 bytes per value, f32 vectors at 4), and for attention the f16 K and V
    rows of ctx_len positions."""
    h, kv, f = cfg.hidden, cfg.kv_dim, cfg.ffn
    xq = lambda n: 3.5 * n  # noqa: E731  (XQ layout: three digit planes, a scale and a sum per 16)
    if stage == "qkv":
        return int(I.row_bytes(mat, h) * (h + 2 * kv) + xq(h) + 4 * h + 2 * 2 * kv)
    if stage == "attention":
        return int(2 * kv * 2 * ctx_len + 4 * h + 4 * h + xq(h))
    if stage == "attn_output":
        return int(I.row_bytes(mat, h) * h + xq(h) + 2 * 4 * h + xq(h))
    if stage == "ffn_gate_up":
        return int(I.row_bytes(mat, h) * 2 * f + xq(h) + 4 * f)
    if stage == "ffn_down":
        return int(I.row_bytes(mat, f) * h + 4 * f + 2 * 4 * h + xq(h))
    raise ValueError(stage)


def measured_traffic(kernel: str):
    """HBM bytes per launch of a decode kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (calibrated on add_k), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_8b_q4k_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["kernels"][kernel]["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def cpu_baseline(cfg: I.Llama2Config, weights: I.Llama2Weights, n_tokens: int, threads: int, pos0: int) -> dict:
    """The CPU oracle (a C restatement of the reference's forward) timed on
    the host cores on a bounded sample: n_tokens decode steps of the same
    model bytes at the GPU leg's positions pos0.. (the oracle's cache rows
    below pos0 are zeros, which cost the same attention work), with its
    matrix products accumulated left to right in f32 as the reference's CPU
    forward does (crates/inferi/src/models/llama2/cpu.rs:375-381)."""
    import oracle as O

    if not os.path.exists(O.LIB_PATH):
        O.build()
    host = {}
    for name in cfg.shapes():
        dt, arr, rows, cols = weights.download(name)
        vector = name.endswith(("norm.weight", ".bias"))
        host[name] = arr if vector else (dt, np.ascontiguousarray(arr).view(np.uint8), rows, cols)
    c = dict(hidden=cfg.hidden, ffn=cfg.ffn, n_layers=cfg.n_layers, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
             vocab=cfg.vocab, max_pos=pos0 + n_tokens + 1, rope_theta=cfg.rope_theta, rms_eps=cfg.rms_eps,
             kv_f16=1)
    m = O.Model(c, host)
    with O.f32_accumulation():
        m.forward(1, pos0, threads)  # warm the pages
        t0 = time.perf_counter()
        for p in range(pos0 + 1, pos0 + n_tokens + 1):
            m.forward(p % cfg.vocab, p, threads)
        dt = time.perf_counter() - t0
    try:
        host_cores = len(os.sched_getaffinity(0))
    except AttributeError:
        host_cores = os.cpu_count()
    return {"value": n_tokens / dt, "unit": "tok/s", "cores": threads, "host_cores": host_cores,
            "host_cpu_count": os.cpu_count(), "kind": "port",
            "sample": f"{n_tokens} decode tokens of the same 8B-shape model bytes at positions {pos0 + 1}-"
                      f"{pos0 + n_tokens} (the GPU leg's context) through oracle/oracle.c ifo_forward with f32 "
                      f"left-to-right GEMV accumulation (the reference CPU forward's arithmetic), "
                      f"{threads} threads on {host_cores} available cores"}


def run_decode(args) -> None:
    ctx = make_ctx(args)
    ctx.set_option("gemv_max_grid", args.gemv_grid)
    ctx.set_option("gemv_waves", args.gemv_waves)
    if args.gemv_grp >= 0:
        ctx.set_option("gemv_grp", args.gemv_grp)
    dev_name, n_cu = ctx.device_info()
    base = CFG_8B if args.model == "8b" else CFG_C4
    prompt_len = args.prompt
    n_exact = args.exact_steps + (EXACT_WARMUP if args.exact_steps else 0)
    max_pos = prompt_len + args.warmup + args.steps + SAMPLE_WARMUP + args.sample_steps + n_exact + 1
    cfg = I.Llama2Config(max_pos=max_pos, kv_dtype=I.F16, **base)
    t0 = time.perf_counter()
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=args.seed)
    log(f"bench: {dev_name}, {n_cu} CUs; synthetic weights in {time.perf_counter() - t0:.1f}s")
    s = I.Llama2State(ctx, cfg)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, prompt_len).astype(np.uint32)
    s.reset(prompt, 0)
    # prompt: the first prompt_len - 1 tokens through the matrix-core prefill
    # (the last one goes through the first decode step); timed on its own
    n_pf = prompt_len - 1
    pf = None
    if n_pf > 0:
        I.Llama2.prefill(ctx, s, w, n_pf)  # warm-up: kernels loaded, scratch allocated
        s.reset(prompt, 0)
        ctx.sync()
        ctx.event_record(4)
        I.Llama2.prefill(ctx, s, w, n_pf)
        ctx.event_record(5)
        pf_ms = ctx.event_elapsed(4, 5)
        flops = prefill_flops(cfg, n_pf)
        pf = {"tokens": n_pf, "ms": round(pf_ms, 3), "tok_s": round(n_pf / pf_ms * 1000.0, 1),
              "tflops": round(flops / (pf_ms * 1e-3) / 1e12, 2), "flops": int(flops),
              "mfma_frac": round(flops / (pf_ms * 1e-3) / MFMA_F16_PEAK, 4),
              "weights": "GGUF blocks dequantized to f16 inside the GEMM tiles (no f16 copy)"}
        log(f"bench: prefill {n_pf} tokens in {pf_ms:.2f} ms ({pf['tok_s']:.0f} tok/s, {pf['tflops']:.1f} TFLOP/s, "
            f"{pf['mfma_frac'] * 100:.1f}% of the f16 dense peak)")
        # the same prompt on 128 x 128 GEMM tiles (the same results bit for bit)
        ctx.set_option("pf_tile", 128)
        s.reset(prompt, 0)
        ctx.sync()
        ctx.event_record(4)
        I.Llama2.prefill(ctx, s, w, n_pf)
        ctx.event_record(5)
        pf["ms_tile128"] = round(ctx.event_elapsed(4, 5), 3)
        ctx.set_option("pf_tile", 0)
        log(f"bench: prefill on 128 x 128 GEMM tiles {pf['ms_tile128']:.2f} ms")
        # and with the Q4_K products in the eight-wave form (no warp
        # specialization; the same results bit for bit)
        ctx.set_option("pf_ws", 0)
        s.reset(prompt, 0)
        ctx.sync()
        ctx.event_record(4)
        I.Llama2.prefill(ctx, s, w, n_pf)
        ctx.event_record(5)
        pf["ms_eight_wave"] = round(ctx.event_elapsed(4, 5), 3)
        ctx.set_option("pf_ws", 1)
        log(f"bench: prefill with the eight-wave Q4_K GEMM {pf['ms_eight_wave']:.2f} ms")
    I.Llama2.generate(ctx, s, w, args.warmup, use_graph=not args.no_graph)
    ctx.sync()
    pos0 = int(s.read("pos", np.uint32)[0])
    ctx.event_record(0)
    I.Llama2.generate(ctx, s, w, args.steps, use_graph=not args.no_graph)
    ctx.event_record(1)
    ms = ctx.event_elapsed(0, 1)
    ctx.sync()
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    mean_ctx = pos0 + (args.steps + 1) / 2.0
    tok_bytes = decode_token_bytes(cfg, mean_ctx)
    log(f"bench: decode {args.steps} tokens at pos {pos0}..{pos0 + args.steps - 1}: {ms_per_step:.4f} ms/token, "
        f"{tok_s:.1f} tok/s, {tok_bytes / (ms_per_step * 1e-3) / 1e9:.0f} GB/s of {HBM_PEAK_GBS:.0f}")
    toks = s.tokens(pos0, args.steps + 1)
    assert np.all(toks < cfg.vocab)

    # the same loop sampling as the reference's chat loop does
    # (Sampler::new(vocab, 0.7, 0.95), crates/inferi-chat/src/sampler.rs:109)
    sampled = None
    if args.sample_steps > 0:
        s.set_sampler(0.7, 0.95, args.seed)
        I.Llama2.generate(ctx, s, w, SAMPLE_WARMUP, use_graph=not args.no_graph)
        ctx.sync()
        ctx.event_record(2)
        I.Llama2.generate(ctx, s, w, args.sample_steps, use_graph=not args.no_graph)
        ctx.event_record(3)
        sms = ctx.event_elapsed(2, 3) / args.sample_steps
        s.set_sampler(0.0)
        sampled = {"temperature": 0.7, "topp": 0.95, "steps": args.sample_steps, "ms_per_step": round(sms, 5),
                   "tok_s": round(1000.0 / sms, 2), "sampler_us": round(time_sampler(ctx, cfg.vocab), 2)}
        log(f"bench: sampled decode (T 0.7, top-p 0.95): {sms:.4f} ms/token, {1000.0 / sms:.1f} tok/s; "
            f"sampler alone {sampled['sampler_us']:.1f} us")

    # the same loop on the exact GEMV path (x kept in f32, fp32 FMAs)
    exact = None
    if args.exact_steps > 0:
        ctx.set_option("gemv_exact", 1)
        I.Llama2.generate(ctx, s, w, EXACT_WARMUP, use_graph=not args.no_graph)
        ctx.sync()
        ctx.event_record(2)
        I.Llama2.generate(ctx, s, w, args.exact_steps, use_graph=not args.no_graph)
        ctx.event_record(3)
        ems = ctx.event_elapsed(2, 3) / args.exact_steps
        ctx.set_option("gemv_exact", 0)
        exact = {"steps": args.exact_steps, "ms_per_step": round(ems, 5), "tok_s": round(1000.0 / ems, 2)}
        log(f"bench: exact-path decode (gemv_exact): {ems:.4f} ms/token, {1000.0 / ems:.1f} tok/s")

    # every stage of the step on its own (the step's own launches, each layer
    # in turn, so no weights are reused from the caches), at this context
    ctx_now = int(s.read("pos", np.uint32)[0]) + 1
    stages = {}
    for st in STAGES:
        us = I.Llama2.time_stage(ctx, s, w, st, args.stage_iters)
        nb = stage_bytes(cfg, st, ctx_now)
        stages[st] = {"kernel": STAGE_KERNELS[st], "us": round(us, 3), "bytes": nb,
                      "gbs": round(nb / (us * 1e-6) / 1e9, 1), "frac": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "us_per_token": round(us * cfg.n_layers, 1)}
        log(f"bench: stage {st} ({STAGE_KERNELS[st]}): {us:.2f} us/layer, {stages[st]['gbs']:.0f} GB/s")
    dom = stages[ROOFLINE_STAGE]

    # the op-level Q4_K GEMV (ifr_matmul_quant_xq) at the 14336x4096 FFN shape
    g = time_gemv(ctx, I.Q4_K, 14336, 4096, iters=args.gemv_iters)
    log(f"bench: gemv_q4_k_plain_one 14336x4096: {g['us']:.2f} us/launch, {g['gbs']:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        t0 = time.perf_counter()
        cpu = cpu_baseline(cfg, w, args.cpu_tokens, threads, pos0)
        log(f"bench: cpu baseline {cpu['value']:.3f} tok/s ({time.perf_counter() - t0:.1f}s)")

    out = {
        "metric": "decode tok/s batch 1 (8B-shape Q4_K); Q4_K GEMV achieved HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x int8 (v_dot4) + f32",
        "data": "synthetic (random-init N(0,0.02) weights quantized on device; uniform random prompt ids)",
        "config": {
            "workload": ("8B-shape Llama decode: 32 layers, hidden 4096, 32 q / 8 kv heads, FFN 14336, vocab 128256, "
                         "Q4_K matmuls + Q6_K head, f16 KV cache" if args.model == "8b" else
                         "22-layer Llama decode: hidden 2048, 32 q / 4 kv heads, FFN 5632, vocab 32000, Q4_K + Q6_K"),
            "prompt_tokens": prompt_len,
            "positions": [pos0, pos0 + args.steps - 1],
            "batch": 1,
            "decode_bytes_per_token": int(tok_bytes),
            "decode_hbm_frac": round(tok_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "device": dev_name,
            "prefill": pf,
            "sampled_decode": sampled,
            "exact_path_decode": exact,
            "stages": stages,
            "op_gemv_q4_k_14336x4096": {"kernel": "gemv_q4_k_plain_one", "us": round(g["us"], 3), "bytes": g["bytes"],
                                        "gbs": round(g["gbs"], 1), "frac": round(g["gbs"] / HBM_PEAK_GBS, 4)},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": (f"{dom['kernel']} (the decode step's FFN gate/up GEMV, 2 x {cfg.ffn} x {cfg.hidden} Q4_K; "
                       f"{dom['bytes']:,} algorithmic bytes per launch)"),
            "achieved": dom["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["frac"],
            "traffic": measured_traffic(dom["kernel"]),
            "avg_launch_us": dom["us"],
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    s.close()
    w.close()
    ctx.close()


def run_sweep(args) -> None:
    ctx = make_ctx(args)
    ctx.set_option("gemv_max_grid", args.gemv_grid)
    ctx.set_option("gemv_waves", args.gemv_waves)
    if args.gemv_grp >= 0:
        ctx.set_option("gemv_grp", args.gemv_grp)
    rows_out = []
    cpu = not args.no_cpu
    if cpu:
        import oracle as O  # the CPU baseline only: the reference shaders' decomposition on host threads

        nthr = cpu_threads(args)
    for name, dt in (("Q4_K", I.Q4_K), ("Q5_K", I.Q5_K), ("Q6_K", I.Q6_K), ("Q8_0", I.Q8_0)):
        for rows, cols in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
            g = time_gemv(ctx, dt, rows, cols, iters=args.gemv_iters, keep_host=cpu)
            rec = {"format": name, "rows": rows, "cols": cols, "us": round(g["us"], 3), "bytes": g["bytes"],
                   "gbs": round(g["gbs"], 1), "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
                   "us_f32x": round(g["us_f32x"], 3), "gbs_f32x": round(g["gbs_f32x"], 1),
                   "frac_f32x": round(g["gbs_f32x"] / HBM_PEAK_GBS, 4)}
            if cpu:
                w, x = g["host_w"], g["host_x"]
                cms = cpu_median_ms(lambda: O.ref_gemv(dt, w, rows, cols, x, nthr), 5)
                rec["cpu"] = {"ms": round(cms, 3), "gbs": round(g["bytes"] / (cms * 1e-3) / 1e9, 2), "threads": nthr}
            rows_out.append(rec)
            log(f"sweep: {name} {rows}x{cols}: {g['us']:.2f} us, {g['gbs']:.0f} GB/s ({rec['frac'] * 100:.1f}%); "
                f"f32 x {g['us_f32x']:.2f} us ({rec['frac_f32x'] * 100:.1f}%)"
                + (f"; cpu {rec['cpu']['ms']:.2f} ms, {rec['cpu']['gbs']:.2f} GB/s" if cpu else ""))
    print(json.dumps({"sweep": rows_out}), flush=True)
    ctx.close()


def run_pmc_sample(args) -> None:
    """Workload for the rocprofv3 --pmc passes behind roofline.traffic: the
    element-wise add kernel (add_k) over 64 Mi floats, whose HBM traffic is
    known (reads 2 x 256 MiB, writes 256 MiB), calibrates FETCH_SIZE and
    WRITE_SIZE; then the op-level GEMV (gemv_q4_k_plain_one 14336x4096) on
    weight copies rotated past the Infinity Cache; then each stage of the
    8B decode step at position 4100, twice over the 32 layers."""
    ctx = make_ctx(args)
    n = 64 << 20
    a, b = ctx.alloc(n * 4), ctx.alloc(n * 4)
    ctx.fill_normal(a, n, 1, 0, 0.0, 1.0)
    ctx.fill_normal(b, n, 2, 0, 0.0, 1.0)
    for _ in range(3):
        ctx.add_assign(a, b, n)
    ctx.sync()
    a.free()
    b.free()
    g = time_gemv(ctx, I.Q4_K, 14336, 4096, iters=args.gemv_iters)
    log(f"pmc sample: add_k {3} x {n} floats; gemv_q4_k_plain_one 14336x4096 {g['us']:.2f} us")
    cfg = I.Llama2Config(max_pos=4608, kv_dtype=I.F16, **CFG_8B)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=args.seed)
    s = I.Llama2State(ctx, cfg)
    s.reset(np.zeros(4102, np.uint32), 4100)
    for st in STAGES:
        us = I.Llama2.time_stage(ctx, s, w, st, 1)
        log(f"pmc sample: stage {st} ({STAGE_KERNELS[st]}) {us:.2f} us/layer")
    s.close()
    w.close()
    ctx.close()


def run_pf_sample(args) -> None:
    """Workload for the rocprofv3 --pmc passes on the prefill kernels: the
    8B model's 4095-token prompt through ifr_llama2_prefill, twice."""
    ctx = make_ctx(args)
    cfg = I.Llama2Config(max_pos=args.prompt + 8, kv_dtype=I.F16, **CFG_8B)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=args.seed)
    s = I.Llama2State(ctx, cfg)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, args.prompt).astype(np.uint32)
    for _ in range(2):
        s.reset(prompt, 0)
        ctx.sync()
        ctx.event_record(4)
        I.Llama2.prefill(ctx, s, w, args.prompt - 1)
        ctx.event_record(5)
        log(f"pf sample: prefill {args.prompt - 1} tokens in {ctx.event_elapsed(4, 5):.2f} ms")
    s.close()
    w.close()
    ctx.close()


def run_attn(args) -> None:
    ctx = make_ctx(args)
    ctx.set_option("gemv_max_grid", args.gemv_grid)
    ctx.set_option("gemv_waves", args.gemv_waves)
    if args.gemv_grp >= 0:
        ctx.set_option("gemv_grp", args.gemv_grp)
    out = []
    nh, nkv, hs = 32, 8, 128
    kv_dim = nkv * hs
    for L in (512, 2048, 4352, 8192, 16384, 32768):
        copies = max(2, -(-ROT_BYTES // (2 * L * kv_dim * 2)))
        caches = []
        for i in range(copies):
            kc = ctx.alloc(2 * L * kv_dim * 4)
            ctx.fill_normal(kc, 2 * L * kv_dim, 3, i, 0.0, 1.0)
            k16 = ctx.alloc(L * kv_dim * 2)
            v16 = ctx.alloc(L * kv_dim * 2)
            ctx.quantize(k16, kc, I.F16, L * kv_dim)
            ctx.quantize(v16, kc.at(L * kv_dim * 4), I.F16, L * kv_dim)
            kc.free()
            caches.append((k16, v16))
        q = ctx.upload(np.random.default_rng(5).standard_normal(nh * hs).astype(np.float32))
        o = ctx.alloc(nh * hs * 4)
        p = I.AttentionParams(L, kv_dim, nh // nkv, nh, hs, L - 1)
        dp = ctx.upload(np.frombuffer(bytes(p), np.uint8))
        for k16, v16 in caches:
            I.BatchedMultiqueryAttention.launch(ctx, p, dp, q, k16, v16, I.F16, o)
        ctx.sync()
        iters = args.gemv_iters
        ctx.event_record(2)
        for i in range(iters):
            k16, v16 = caches[i % copies]
            I.BatchedMultiqueryAttention.launch(ctx, p, dp, q, k16, v16, I.F16, o)
        ctx.event_record(3)
        us = ctx.event_elapsed(2, 3) * 1000.0 / iters
        nbytes = 2 * L * kv_dim * 2 + 2 * nh * hs * 4
        rec = {"L": L, "us": round(us, 3), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
        if not args.no_cpu:
            import oracle as O  # the CPU baseline only: the reference shaders' decomposition on host threads

            k16, v16 = caches[0]
            kh, vh = k16.download(np.uint16, L * kv_dim), v16.download(np.uint16, L * kv_dim)
            qh = np.random.default_rng(5).standard_normal(nh * hs).astype(np.float32)
            nthr = cpu_threads(args)
            cms = cpu_median_ms(lambda: O.ref_attention(qh, kh, vh, nh, nkv, hs, L - 1, nthr), 3)
            rec["cpu"] = {"ms": round(cms, 3), "gbs": round(nbytes / (cms * 1e-3) / 1e9, 2), "threads": nthr}
        out.append(rec)
        log(f"attn: L={L}: {us:.2f} us, {rec['gbs']:.0f} GB/s"
            + (f"; cpu {rec['cpu']['ms']:.2f} ms, {rec['cpu']['gbs']:.2f} GB/s" if "cpu" in rec else ""))
        for k16, v16 in caches:
            k16.free()
            v16.free()
        q.free()
        o.free()
        dp.free()
    print(json.dumps({"attention": out}), flush=True)
    ctx.close()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--model", choices=["8b", "c4"], default="8b")
    ap.add_argument("--seed", type=int, default=2000)
    ap.add_argument("--gemv-iters", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="launch the decode step's kernels directly")
    ap.add_argument("--cpu-tokens", type=int, default=8)
    ap.add_argument("--sample-steps", type=int, default=64,
                    help="decode steps timed with the reference chat loop's sampler (T 0.7, top-p 0.95)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--exact-steps", type=int, default=32, help="decode steps timed on the exact GEMV path")
    ap.add_argument("--stage-iters", type=int, default=10, help="passes over the layers per stage timing")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--attn", action="store_true")
    ap.add_argument("--pmc-sample", action="store_true", help="workload for the rocprofv3 --pmc traffic passes")
    ap.add_argument("--pf-sample", action="store_true", help="workload for the rocprofv3 --pmc prefill passes")
    ap.add_argument("--code-object", default=None, help="another build of the kernels' code object")
    ap.add_argument("--opt", action="append", default=[], help="library option KEY=VALUE (repeatable)")
    ap.add_argument("--gemv-grid", type=int, default=0, help="GEMV workgroups (0: chosen by shape)")
    ap.add_argument("--gemv-waves", type=int, default=0, help="waves per GEMV workgroup (0: chosen by shape)")
    ap.add_argument("--gemv-grp", type=int, default=-1, help="GEMV form mask (option gemv_grp; -1: the library default, whose kernels the stage lines name)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU; the multi-GPU sharding of the decode path is designed "
              "but not built. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.pmc_sample:
        run_pmc_sample(args)
    elif args.pf_sample:
        run_pf_sample(args)
    elif args.sweep:
        run_sweep(args)
    elif args.attn:
        run_attn(args)
    else:
        run_decode(args)


if __name__ == "__main__":
    main()
