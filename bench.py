#!/usr/bin/env python3
"""Benchmark of libsimp_hip.so on one MI355X.

Headline (the JSON line's ``value``): exact int8 GEMM throughput, u8 x s8 -> i32
(vpdpbusd semantics), at the largest square shape of BASELINE configs[1]
(8192^3), inputs resident in HBM.  One step = one C = A x B over the
synthetic batch (A u8 uniform [0,255], B s8 uniform [-128,127], seed 42).

``value`` and ``ms_per_step`` cover the whole call (column sums + GEMM).
``roofline`` is the dominant kernel alone: its launches are bracketed with HIP
events on the stream they run on (simp_rt_timing), so ``achieved`` is 2*M*N*K
over that kernel's average launch time.

Clock settling: under this kernel's sustained load the chip's clocks dip and
recover over its first ~60 calls (per-call times on one box: 546, 601, 652,
740, 733, 714, 669, ... 559 us average over calls 21-40, 532 over 41-60, then
523-526 us), so SETTLE_CALLS untimed calls run before the W warmup calls and
the K timed ones; the line reports the count as ``settle_calls``.  Without
them, 5 warmup + 20 timed calls average 613 us on the same box.

Also reported on the same line: the configs[1] sweep (TOPS per shape), the W4
GEMV (with its CPU baseline per shape), rmsnorm / softmax / silu, fp32 GEMM and
decode sections, and the CPU baseline -- the oracle's restatement of the
reference's VNNI kernel timed on the host cores one GPU gets (and on one core)
on a bounded row-block sample of the same 8192^3 problem, with the host's CPU
model, nproc and AVX-512 VNNI flag.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-sweep] [--no-cpu]
                    [--only gemm|w4|f32|decode|norm|copy]

``--only copy`` times a plain 256 MiB device copy (the calibration run for the
rocprofv3 FETCH_SIZE / WRITE_SIZE counters) and prints its own JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int8 GEMM TOPS (% MFMA peak); W4 decode tokens/s + HBM GB/s (1 GPU)"
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
FP32_PEAK_TFS = 157.3    # MI355X dense fp32 MFMA
HBM_PEAK_GBS = 8000.0
SETTLE_CALLS = 60        # untimed headline calls before the warmup (clock settling)


def gemm_events(fn, a, b, c, steps, warmup, stream):
    """Average ms per call over `steps` back-to-back launches (HIP events)."""
    import torch
    for _ in range(warmup):
        fn(a, b, c)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn(a, b, c)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def make_inputs(M, N, K, dev, seed=42):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=g)
    b = torch.randint(-128, 128, (K, N), dtype=torch.int8, device=dev, generator=g)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    return a, b, c


# One MI355X's share of its box's host CPUs: the GPU boxes give each GPU 16
# cores whatever nproc reports, so "all cores" means at most 16 there.
CPU_SHARE = 16


def host_info():
    """nproc, the CPU model (as lscpu prints it) and the AVX-512 VNNI flag."""
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "model": None, "avx512_vnni": False}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and info["model"] is None:
                    info["model"] = line.split(":", 1)[1].strip()
                elif line.startswith("flags"):
                    info["avx512_vnni"] = "avx512_vnni" in line.split()
                    break
    except OSError:
        pass
    info["cores_used"] = min(info["affinity"], CPU_SHARE)
    return info


def cpu_baseline(n, threads, budget_s):
    """Oracle VNNI restatement on `threads` host cores, 64-row blocks of the n^3
    problem, repeated until about budget_s of CPU work."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    rng = np.random.default_rng(42)
    rows = 64
    a = rng.integers(0, 256, (rows, n)).astype(np.uint8)
    b = rng.integers(-128, 128, (n, n)).astype(np.int8)
    bt = np.ascontiguousarray(b.T)
    oracle.matmul_i8_vnni(a[:8], bt, a_unsigned=True, b_nk=True, nthreads=threads)  # warm
    done, t0, hw = 0, time.perf_counter(), False
    while True:
        _, hw = oracle.matmul_i8_vnni(a, bt, a_unsigned=True, b_nk=True, nthreads=threads)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    tops = 2.0 * done * rows * n * n / el / 1e12
    return {"value": round(tops, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": (f"{done} blocks of {rows} rows x {n} x {n} ({done * rows / n:.2f} passes "
                       f"over the {n}^3 problem; u8xs8->i32, B pre-transposed as the "
                       f"reference's B_T) in {el:.1f}s on {threads} thread(s); "
                       f"{'AVX-512 VNNI' if hw else 'scalar (host lacks AVX-512 VNNI)'}")}


def cpu_baselines(n):
    """The headline's CPU baseline on all the cores one GPU gets (value) and on
    one core, with the host's identity."""
    host = host_info()
    line = cpu_baseline(n, host["cores_used"], 10.0)
    one = cpu_baseline(n, 1, 5.0)
    line["single_thread"] = {"value": one["value"], "unit": "TOPS", "cores": 1,
                             "sample": one["sample"]}
    line["host"] = host
    return line


def graph_time_ms(calls, stream, replays=5, warm_ms=30.0):
    """GPU time per call of a sequence of library calls, captured once in a HIP
    graph and replayed (removes the Python/ctypes enqueue cost, which exceeds the
    runtime of the small kernels).  About `warm_ms` of untimed replays come
    first: the clocks ramp over the first tens of milliseconds of GPU work
    (measured: 48.7 us per call over the first 5 replays of a 43 us fp32 GEMM,
    43.0 us after 50)."""
    import torch
    import simplang_amd as sa
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        sa.set_stream(side)
        for f in calls:
            f()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):    # same stream as the warm-up: workspaces exist
        sa.set_stream(side)
        for f in calls:
            f()
    sa.set_stream(stream)
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    for _ in range(min(1000, int(warm_ms / max(t0.elapsed_time(t1), 1e-3)))):
        g.replay()
    t0.record(stream)
    for _ in range(replays):
        g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (replays * len(calls))


def w4_cpu_us(w, s, x, threads, budget_s=0.4):
    """The W4 product through the reference lowering's loop structure
    (oracle orc_matmul_w4s_lowering, ConvertSimpToMemRef.cpp:3906-4011) on the
    host: microseconds per call."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    oracle.matmul_w4s_lowering(w, s, x, 32, threads)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        oracle.matmul_w4s_lowering(w, s, x, 32, threads)
        n += 1
    return (time.perf_counter() - t0) / n * 1e6


def w4_bench(dev, stream, with_cpu=True):
    """W4 GEMV/skinny GEMM, BASELINE configs[2].  Weight copies are rotated so
    that more than 512 MB is touched per pass: every launch streams its weights
    from HBM (the 256 MB Infinity Cache cannot hold them), as in a decode step.
    Timed by HIP-graph replay of one launch per copy.  Each row also carries the
    CPU baseline on the cores one GPU gets."""
    import torch
    import simplang_amd as sa
    out = []
    threads = host_info()["cores_used"]
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    for (K, N) in ((3200, 8640), (8640, 3200), (3200, 32000)):
        wbytes = N * K // 2 + 4 * N * K // 32
        copies = max(2, -(-512 * 2**20 // wbytes))
        ws = [torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=g)
              for _ in range(copies)]
        ss = [(torch.rand((N, K // 32), device=dev, generator=g) * 0.02 / 7) for _ in range(copies)]
        wh, sh = (ws[0].cpu().numpy(), ss[0].cpu().numpy()) if with_cpu else (None, None)
        for M in (1, 4, 16):
            x = torch.randn((M, K), device=dev, generator=g)
            o = torch.empty((M, N), device=dev)
            calls = [(lambda i=i: sa.matmul_w4s(ws[i], ss[i], x, o, 32)) for i in range(copies)]
            ms = graph_time_ms(calls, stream)
            byts = N * K / 2 + 4 * N * K / 32 + 4 * M * K + 4 * M * N
            row = {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                   "GBs": round(byts / (ms * 1e-3) / 1e9, 1),
                   "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
            if with_cpu:
                cus = w4_cpu_us(wh, sh, x.cpu().numpy(), threads)
                row["cpu_baseline"] = {"us": round(cus, 1), "GBs": round(byts / cus / 1e3, 2),
                                       "cores": threads, "kind": "port"}
            out.append(row)
        del ws, ss
        torch.cuda.empty_cache()
    return out


def norm_bench(dev, stream, with_cpu=True):
    """rmsnorm / softmax / silu (rows a9-a11) as standalone launches at the model
    sizes (768 and 3200 dims, 2048 and 8640 FFN widths, 288 and 512 attention
    rows), where a launch's latency is the cost, and at 2^24 elements (64 MB
    vectors, the two-pass multi-block forms), where HBM is: GPU time by HIP-graph
    replay of back-to-back launches, GB/s over the algorithmic bytes of the
    reference loops (12n; 16n for softmax's read, write, re-read and write;
    8n), and the oracle's restatement of the reference loop on one host core.
    The kernels move 12n, 8n and 8n up to 32767 elements and 16n, 12n and 8n
    in the two-pass forms beyond (x read twice)."""
    import numpy as np
    import torch
    import simplang_amd as sa
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    out = []
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    big = 1 << 24
    cases = [("rmsnorm", n) for n in (768, 3200, 8640, big)] + \
            [("softmax", n) for n in (288, 512, 768, 3200, 8640, big)] + \
            [("silu", n) for n in (768, 2048, 3200, 8640, big)]
    for op, n in cases:
        # the 2^24 cases rotate through 4 sets of vectors (768 MB for rmsnorm),
        # more than the 256 MB Infinity Cache, so every launch streams from HBM
        sets = 4 if n == big else 1
        xs = [torch.randn(n, device=dev, generator=g) for _ in range(sets)]
        ws = [torch.randn(n, device=dev, generator=g) for _ in range(sets)]
        os_ = [torch.empty(n, device=dev) for _ in range(sets)]
        x, w = xs[0], ws[0]
        if op == "rmsnorm":
            calls = [lambda i=i: sa.rmsnorm(xs[i], ws[i], os_[i], n) for i in range(sets)]
            byts = 12 * n
            cpu = lambda xh=x.cpu().numpy(), wh=w.cpu().numpy(): oracle.rmsnorm(xh, wh)
        elif op == "softmax":
            calls = [lambda i=i: sa.softmax(xs[i], os_[i], n) for i in range(sets)]
            byts = 16 * n
            cpu = lambda xh=x.cpu().numpy(): oracle.softmax(xh)
        else:
            calls = [lambda i=i: sa.silu(xs[i], os_[i], n) for i in range(sets)]
            byts = 8 * n
            cpu = lambda xh=x.cpu().numpy(): oracle.silu(xh)
        ms = graph_time_ms(calls * (20 if n == big else 50), stream)
        row = {"op": op, "n": n, "us": round(ms * 1e3, 2),
               "GBs": round(byts / (ms * 1e-3) / 1e9, 2)}
        if with_cpu:
            cpu()
            k, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 0.1:
                cpu()
                k += 1
            row["cpu_baseline"] = {"us": round((time.perf_counter() - t0) / k * 1e6, 2),
                                   "cores": 1, "kind": "port"}
        out.append(row)
        del xs, ws, os_
    torch.cuda.empty_cache()
    return out


def f32_bench(dev, stream):
    """fp32 tensor_matmul (row a5) on prefill-shaped and square problems, and the
    rank-3 batched product; inputs N(0,1) resident in HBM, HIP-graph replay."""
    import torch
    import simplang_amd as sa
    out = []
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    for (bt, M, K, N) in ((1, 8, 2048, 2048), (1, 128, 2048, 8192), (1, 512, 2048, 2048),
                          (1, 4096, 4096, 4096), (32, 512, 128, 512)):
        shape = (bt, M, K) if bt > 1 else (M, K)
        a = torch.randn(shape, device=dev, generator=g)
        b = torch.randn((bt, K, N) if bt > 1 else (K, N), device=dev, generator=g)
        c = torch.empty((bt, M, N) if bt > 1 else (M, N), device=dev)
        fn = sa.tensor_batch_matmul if bt > 1 else sa.tensor_matmul_f32
        reps = 5 if M * N * K * bt >= 2**34 else 20
        t = graph_time_ms([lambda: fn(a, b, c)] * reps, stream)
        tfs = 2.0 * bt * M * N * K / (t * 1e-3) / 1e12
        out.append({"batch": bt, "M": M, "K": K, "N": N, "us": round(t * 1e3, 2),
                    "TFs": round(tfs, 1), "frac_fp32_peak": round(tfs / FP32_PEAK_TFS, 3)})
        del a, b, c
    torch.cuda.empty_cache()
    return out


def decode_bench(dev, stream, with_cpu=True):
    """Greedy decode tok/s, BASELINE configs[3] (110M fp32) and configs[4]
    (3B W4): random-init weights, random prompt of 32 tokens, then 256 / 128
    greedy tokens, every step one replay of the captured step graph.  tok/s =
    steps / wall time of the generation (one token per step, prompt steps
    included, as bench_llama_quant.cpp:255-292 times every forward call)."""
    import numpy as np
    import torch
    import simplang_amd as sa
    from simplang_amd.llama_synth import CFG_110M, CFG_3B_W4, make_model, weight_bytes, kv_bytes
    out = []
    for name, cfg, n_new in (("llama-110M f32", CFG_110M, 256), ("llama-3B W4 g32", CFG_3B_W4, 128)):
        w = make_model(cfg, dev, seed=42)
        prompt = np.random.default_rng(42).integers(0, cfg["vocab_size"], 32).astype(np.int32)
        m = sa.Llama(cfg, w)
        # capture + warm: the same positions as the timed run, so every step
        # graph (one per attention form and chunk count) exists before timing
        m.generate(prompt, n_new, use_graph=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = m.generate(prompt, n_new, use_graph=True)
        el = time.perf_counter() - t0
        steps = len(prompt) + n_new - 1
        m.close()
        byts = np.mean([weight_bytes(cfg) + kv_bytes(cfg, p) for p in range(steps)])
        rec = {"model": name, "prompt": 32, "generated": n_new, "tok_s": round(steps / el, 1),
               "ms_per_token": round(el / steps * 1e3, 3),
               "GBs": round(byts * steps / el / 1e9, 1),
               "frac_hbm": round(byts * steps / el / 1e9 / HBM_PEAK_GBS, 3),
               "tokens_head": [int(t) for t in toks[32:40]]}
        if with_cpu:
            rec["cpu_baseline"] = decode_cpu(cfg, w, prompt, steps)
        out.append(rec)
        del w
        torch.cuda.empty_cache()
    return out


def llama32_bench(dev, with_cpu=True):
    """llama32_forward (examples/llama2/llama32_1b_int8_tensor.sl) at the
    LLaMA-3.2-1B shape of bench_llama32_1b_int8.cpp:17-25 with its init (int8
    uniform [-64,63], fp32 uniform +-0.01), arrays resident on the device: ms per
    call at the reference bench's positions and a 64-token loop from pos 128
    (bench_llama32_1b_int8.cpp:240-315).  Every call is a full token (16 layers
    of int8 GEMVs over 0.97 GB plus the 1.05 GB fp32 classifier)."""
    import numpy as np
    import torch
    import simplang_amd as sa
    D, H, L, NH, NKV, V, S, HD = 2048, 8192, 16, 32, 8, 128256, 4096, 64
    kv = NKV * HD
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    i8 = lambda n: torch.randint(-64, 64, (n,), dtype=torch.int8, device=dev, generator=g)
    f32 = lambda n: (torch.rand((n,), device=dev, generator=g) * 0.02 - 0.01)
    a = {"x_i8": i8(D), "rms_att_w": f32(L * D), "rms_ffn_w": f32(L * D), "rms_final_w": f32(D),
         "wq_t": i8(L * D * D), "wk_t": i8(L * kv * D), "wv_t": i8(L * kv * D),
         "wo_t": i8(L * D * D), "w1_t": i8(L * H * D), "w2_t": i8(L * D * H),
         "w3_t": i8(L * H * D), "wcls": f32(V * D),
         "x_fp32": torch.zeros(D, device=dev), "xb_fp32": torch.zeros(D, device=dev),
         "logits": torch.zeros(V, device=dev), "xb_i8": torch.zeros(D, dtype=torch.int8, device=dev),
         "k_cache": torch.zeros(L * S * kv, dtype=torch.int8, device=dev),
         "v_cache": torch.zeros(L * S * kv, dtype=torch.int8, device=dev),
         "att_scores": torch.zeros(NH * S, device=dev), "att_probs": torch.zeros(NH * S, device=dev),
         "attn_out": torch.zeros(D, dtype=torch.int32, device=dev),
         "ffn_hb": torch.zeros(H, dtype=torch.int8, device=dev)}
    dims = (D, H, L, NH, NKV, V, S, HD)
    wbytes = L * (2 * D * D + 2 * kv * D + 3 * H * D) + 4 * V * D
    # descriptors built once, as the reference's C++ bench passes its vectors
    fwd = sa.Llama32Program(a, *dims)
    for _ in range(2):
        fwd(0)
    per_pos = []
    for pos in (0, 127, 511, 1023, 2047, 4095):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(5):
            fwd(pos)
        ms = (time.perf_counter() - t0) / 5 * 1e3
        byts = wbytes + 2 * L * (pos + 1) * kv
        per_pos.append({"pos": pos, "ms": round(ms, 3), "GBs": round(byts / ms / 1e6, 1)})
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(64):
        fwd(128 + i)
    el = time.perf_counter() - t0
    rec = {"model": "llama32-1B int8 (llama32_forward)", "positions": per_pos,
           "loop_64_from_128": {"tok_s": round(64 / el, 1), "ms_per_token": round(el / 64 * 1e3, 3),
                                "GBs": round((wbytes + 2 * L * 160 * kv) * 64 / el / 1e9, 1)}}
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        host = {k: v.cpu().numpy() for k, v in a.items()}
        n_cpu = 20
        t0 = time.perf_counter()
        for i in range(n_cpu):
            oracle.llama32_int8_forward(host, 128 + i, *dims)
        el = time.perf_counter() - t0
        rec["cpu_baseline"] = {"tok_s": round(n_cpu / el, 3), "cores": 1, "kind": "port",
                               "sample": f"{n_cpu} calls at positions 128..{127 + n_cpu} (the "
                                         "first of the GPU loop's 64) of the oracle's "
                                         "restatement, one core"}
        del host
    sa.forward_cache_clear()
    del a
    torch.cuda.empty_cache()
    return rec


def llama2_quant_bench(dev, with_cpu=True):
    """llama2_quant_forward (examples/llama2/llama2_quant.sl) at the "LLaMA 1B"
    shape of bench_llama_quant.cpp:324 (dim 1536, 24 layers, 16 heads, hidden
    6144, vocab 32000, seq_len 512, groups of 128): every array uniform +-0.01
    (bench_llama_quant.cpp:42-47, drawn on the GPU), the seven matrices quantized
    one after another into one flat array with the reference quantizer
    (simp_rt_quantize_w4u, bit-identical to bench_llama_quant.cpp:51-93), then
    the reference's loop: two warm-up calls, caches zeroed, 10 calls at pos
    0..9 with token 50 + 10 pos (bench_llama_quant.cpp:232-292), timed three
    times (median).  Once with host arrays as the reference host passes them
    (per call: one fingerprint chunk per weight array checked, logits and the
    new K/V rows copied back) and once with device-resident arrays."""
    import numpy as np
    import torch
    import simplang_amd as sa
    D, H, L, NH, NKV, V, S, GS = 1536, 6144, 24, 16, 16, 32000, 512, 128
    kv = D * NKV // NH
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    u = lambda n: torch.rand((n,), device=dev, generator=g) * 0.02 - 0.01
    per = [D * D, D * kv, D * kv, D * D, H * D, D * H, H * D]
    total = L * sum(per)
    q = torch.empty(total // 2, dtype=torch.uint8, device=dev)
    sc = torch.empty(total // GS, device=dev)
    ze = torch.empty(total // GS, device=dev)
    offs, at = [], 0
    for p in per:
        w = u(L * p)
        sa.quantize_w4u(w, GS, q[at // 2:], sc[at // GS:], ze[at // GS:])
        offs.append(at)
        at += L * p
        del w
    dv = {"token_emb": u(V * D), "rms_att_w": u(L * D), "rms_ffn_w": u(L * D), "rms_final_w": u(D),
          "wcls": u(V * D), "qweights": q.view(torch.int8), "scales": sc, "zeros": ze}
    for k, n in (("x", D), ("xb", D), ("xb2", D), ("q", D), ("k", kv), ("v", kv), ("att", NH * S),
                 ("att_soft", NH * S), ("hb", H), ("hb_silu", H), ("hb2", H), ("logits", V),
                 ("key_cache", L * S * kv), ("value_cache", L * S * kv)):
        dv[k] = torch.zeros(n, device=dev)
    torch.cuda.synchronize()
    dims = (D, H, L, NH, NKV, V, S, GS)
    wbytes = total // 2 + 8 * (total // GS) + 4 * V * D
    out = {"model": "llama2_quant_forward LLaMA-1B W4 g128 (bench_llama_quant.cpp config 1)",
           "weight_bytes": wbytes}

    def run(arrays, label, zero):
        for _ in range(2):
            sa.llama2_quant_forward(arrays, 100, 0, *dims[:-1], GS, offs)
        times = []
        for _ in range(3):
            zero(arrays)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for pos in range(10):
                r = sa.llama2_quant_forward(arrays, 50 + pos * 10, pos, *dims[:-1], GS, offs)
            times.append(time.perf_counter() - t0)
            if not np.isfinite(r):
                raise RuntimeError("llama2_quant_forward: non-finite logits[0]")
        ms = float(np.median(times)) / 10 * 1e3
        out[label] = {"ms_per_token": round(ms, 3), "tok_s": round(1e3 / ms, 1),
                      "GBs": round(wbytes / ms / 1e6, 1)}

    def zero_dev(a):
        a["key_cache"].zero_()
        a["value_cache"].zero_()

    def zero_host(a):
        a["key_cache"][:] = 0
        a["value_cache"][:] = 0

    run(dv, "device_arrays", zero_dev)
    host = {k: v.cpu().numpy() for k, v in dv.items()}
    sa.forward_cache_clear()
    run(host, "host_arrays", zero_host)
    sa.forward_cache_clear()
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        cfg = dict(dim=D, hidden_dim=H, n_layers=L, n_heads=NH, n_kv_heads=NKV, vocab_size=V,
                   seq_len=S)
        o = oracle.LlamaQuantOracle(cfg, {k: host[k] for k in ("token_emb", "rms_att_w", "rms_ffn_w",
                                                              "rms_final_w", "wcls", "scales",
                                                              "zeros")} |
                                    {"qweights": host["qweights"].view(np.uint8)}, GS, offs)
        # the reference bench's loop (bench_llama_quant.cpp:255-292): 10 calls from pos 0
        t0 = time.perf_counter()
        for pos in range(10):
            o.forward(50 + pos * 10, pos)
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"tok_s": round(10 / el, 3), "cores": host_info()["cores_used"],
                               "kind": "port",
                               "sample": "the reference bench's 10-call loop from pos 0, the "
                                         "oracle's llama2_quant_forward"}
    del dv, host
    torch.cuda.empty_cache()
    return out


def decode_cpu(cfg, w, prompt, n_steps, sample_steps=20):
    """The decode CPU baseline (oracle/cpu_decode.c: the step restated in fp32,
    OpenMP GEMVs over output rows in 16 fp32 lanes, the host cores one GPU gets)
    on a bounded sample of the same generation: `sample_steps` consecutive
    steps centred on the mean position of the GPU run's `n_steps`, the cache
    rows below the first one filled with random values (the work of a step does
    not depend on what the rows hold).  tok/s = steps / wall time of that loop
    (bench_llama_quant.cpp:255-292)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    wn = {k: v.detach().cpu().numpy() for k, v in w.items()}
    o = oracle.CpuLlama(cfg, wn)
    p0 = max(0, (n_steps - 1) // 2 - sample_steps // 2)
    kv = cfg["dim"] * cfg["n_kv_heads"] // cfg["n_heads"]
    rng = np.random.default_rng(5)
    for c in (o.kc, o.vc):
        c.reshape(cfg["n_layers"], cfg["seq_len"], kv)[:, :p0] = \
            rng.standard_normal((cfg["n_layers"], p0, kv), dtype=np.float32) * 0.1
    o.forward(int(prompt[0]), p0)     # warm (the step at p0 is timed again below)
    t0 = time.perf_counter()
    for i in range(sample_steps):
        o.forward(int(prompt[i % len(prompt)]), p0 + i)
    el = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or os.cpu_count() or 1
    return {"tok_s": round(sample_steps / el, 3), "ms_per_token": round(el / sample_steps * 1e3, 2),
            "cores": threads, "kind": "port",
            "sample": (f"{sample_steps} decode steps at positions {p0}..{p0 + sample_steps - 1} "
                       f"(centred on the mean position of the GPU run) of the fp32 restatement "
                       f"(oracle/cpu_decode.c) on {threads} OpenMP threads")}


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (committed summary)."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        return json.load(open(p)).get(name)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=40,
                    help="untimed calls right before the timed ones (after SETTLE_CALLS)")
    ap.add_argument("--size", type=int, default=8192)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--only", choices=["gemm", "w4", "f32", "decode", "norm", "copy"], default=None,
                    help="run one section (for profiling); the JSON line is still printed")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: every configuration of this path fits one "
              "MI355X and no multi-GPU run is part of this build (use --gpus 1).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import simplang_amd as sa

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    sa.set_stream(stream)

    if args.only is not None:
        args.no_sweep = args.only != "gemm" or args.no_sweep
        args.no_decode = args.only != "decode"
    n = args.size
    ms = tops = 0.0
    kern, kern_ms = None, 0.0
    if args.only == "copy":
        # calibration for the --pmc FETCH_SIZE / WRITE_SIZE counters: one plain
        # device copy of a known size per launch
        nbytes = 256 << 20
        src = torch.randint(-128, 127, (nbytes,), dtype=torch.int8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / args.steps
        print(json.dumps({"calibration": "device copy", "bytes_read": nbytes,
                          "bytes_written": nbytes, "us": round(t * 1e3, 2),
                          "GBs": round(2 * nbytes / (t * 1e-3) / 1e9, 1)}), flush=True)
        return
    if args.only in (None, "gemm"):
        a, b, c = make_inputs(n, n, n, dev)
        torch.cuda.synchronize()
        for _ in range(SETTLE_CALLS):  # clocks settle under the sustained load
            sa.matmul_u8s8_i32(a, b, c)
        ms = gemm_events(sa.matmul_u8s8_i32, a, b, c, args.steps, args.warmup, stream)
        tops = 2.0 * n * n * n / (ms * 1e-3) / 1e12
        # the dominant kernel alone: HIP events around its launches, on its stream
        sa.timing(True)
        for _ in range(args.steps):
            sa.matmul_u8s8_i32(a, b, c)
        torch.cuda.synchronize()
        for k in ("gemm_i8_dma", "gemm_i8_nt16", "gemm_i8_mfma"):
            kms, kn = sa.timing_query(k)
            if kn:
                kern, kern_ms = k, kms / kn
                break
        sa.timing(False)
        del a, b, c
        torch.cuda.empty_cache()

    sweep = []
    if not args.no_sweep:
        shapes = [(s, s, s) for s in (256, 512, 768, 1024, 2048, 4096)]
        shapes += [(m, nn, k) for m in (1, 8, 64) for (k, nn) in ((768, 2048), (2048, 768),
                                                                   (3200, 8640))]
        for (M, N, K) in shapes:
            a, b, c = make_inputs(M, N, K, dev)
            reps = 20 if M * N * K < 2**33 else 5
            t = graph_time_ms([lambda: sa.matmul_u8s8_i32(a, b, c)] * reps, stream)
            byts = M * K + K * N + 4 * M * N
            sweep.append({"M": M, "N": N, "K": K, "us": round(t * 1e3, 2),
                          "TOPS": round(2.0 * M * N * K / (t * 1e-3) / 1e12, 2),
                          "GBs": round(byts / (t * 1e-3) / 1e9, 1)})
            del a, b, c
        torch.cuda.empty_cache()

    w4 = (w4_bench(dev, stream, with_cpu=not args.no_cpu)
          if args.only == "w4" or (args.only is None and not args.no_sweep) else [])
    norms = (norm_bench(dev, stream, with_cpu=not args.no_cpu)
             if args.only == "norm" or (args.only is None and not args.no_sweep) else [])
    f32 = f32_bench(dev, stream) if args.only == "f32" or (args.only is None and not args.no_sweep) else []
    decode = [] if args.no_decode else decode_bench(dev, stream, with_cpu=not args.no_cpu)
    if not args.no_decode:
        decode.append(llama32_bench(dev, with_cpu=not args.no_cpu))
        decode.append(llama2_quant_bench(dev, with_cpu=not args.no_cpu))

    cpu = None if (args.no_cpu or args.only not in (None, "gemm")) else cpu_baselines(n)

    ktops = 2.0 * n * n * n / (kern_ms * 1e-3) / 1e12 if kern_ms > 0 else 0.0
    line = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "settle_calls": SETTLE_CALLS if args.only in (None, "gemm") else 0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 (u8 x s8 -> i32)",
        "data": "synthetic: A u8 uniform [0,255], B s8 uniform [-128,127], seed 42",
        "config": {"workload": f"int8 GEMM u8xs8->i32 {n}^3 (BASELINE configs[1], largest square)",
                   "M": n, "N": n, "K": n, "layout": "A[M,K], B[K,N] row-major, C[M,N] i32"},
        "roofline": {"bound": "mfma", "achieved": round(ktops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(ktops / INT8_PEAK_TOPS, 4),
                     "traffic": load_traffic(f"{kern}_{n}"),
                     "traffic_source": "profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE of this kernel at this size, copy-calibrated "
                                       "(a committed measurement, not this run's counters)",
                     "kernel": kern,
                     "launch_us": round(kern_ms * 1e3, 2)},
        "cpu_baseline": cpu,
        "sweep": sweep,
        "w4_gemv": w4,
        "norms": norms,
        "f32_gemm": f32,
        "decode": decode,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
