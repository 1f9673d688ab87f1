#!/usr/bin/env python3
"""Benchmark of the hip backend's hot path on one MI355X.

Headline: the near-exact INT16 group-64 decode GEMV,
W[4096 x 1024] int16 codes uniform over [-32768, 32767], one FP32 scale per 64
inputs ~ U(1e-6, 4e-6), X[1 x 1024] ~ N(0, 1). A step is one GEMV over one
matrix; steps rotate through a pool of distinct device copies (> 512 MB, twice
the 256 MB Infinity Cache) so every step streams its weights from HBM. The K
timed steps are replayed from a HIP graph (captured launches of the C ABI),
and `value` is algorithmic bytes / wall time over those K steps.

`roofline` describes the GEMV kernel: algorithmic bytes per launch divided by
the average launch duration, i.e. the HIP-event time of the K replayed launches
(events recorded on the stream the kernels run on) divided by K, from a second
flushed replay whose events bracket the kernels rather than the host's
submission of the replay (the stream sleeps while the host submits it); the
first replay's event window, which includes that submission, is reported as
`per_op.gemv_i16_m1.timed_window_us_per_step`. `per_op` reports the other BASELINE configurations on the
same box (FP32 prefill GEMM, INT16-activation x INT8 prefill GEMM, INT8 GEMV,
attention prefill). `cpu_baseline` times the C oracle (a restatement of the
reference's CPU operator) on the host cores for a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--ops a,b] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "falcon-ocr-cpu_amd", ROOT / "tests", ROOT / "oracle"):
    sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
# HBM bytes per launch of the headline kernel, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE runs scaled by the same counters on a copy of known size (the
# file records the commands and the scaling).
TRAFFIC_FILE = ROOT / "profiles" / "gemv_decode_traffic.md"
FP32_MFMA_PEAK = 157.3  # TFLOP/s dense
# FP32 vector peak (TFLOP/s) for the exact-order chain kernels. They issue
# plain (non-packed) v_fmac_f32, which gfx950 runs faster than 16 lanes per
# clock per SIMD: a register-only FMA loop reaches 114 TFLOP/s, above the
# 78.6 that 16 lanes x 2.4 GHz would allow, so the vector peak bounds them.
FP32_VECTOR_PEAK = 157.3
INT8_MFMA_PEAK = 5000.0  # TOP/s dense
F16_MFMA_PEAK = 2500.0  # TFLOP/s dense, FP16 and BF16
POOL_BYTES = 600 << 20  # > 2 x 256 MB Infinity Cache
# Device clock cycles the stream sleeps (torch.cuda._sleep: a spin on the
# clock, no memory traffic) while the host submits the timed replay whose
# launches the events then bracket: well over a replay's submission time.
SUBMIT_COVER_CYCLES = 2_000_000


def gemv_bytes(n, k, rows, code_bytes, group=64):
    """Algorithmic bytes of one decode GEMV: codes + scales + inputs + outputs."""
    return n * k * code_bytes + 4 * n * (k // group) + 4 * rows * k + 4 * rows * n


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """Per-launch HIP event pairs on torch's current stream (the stream the
    library's context launches on)."""

    def __init__(self, torch):
        self.torch = torch

    def per_launch_ms(self, fn, reps):
        torch = self.torch
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        for i in range(reps):
            starts[i].record()
            fn(i)
            ends[i].record()
        torch.cuda.synchronize()
        times = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
        return sum(times) / len(times), times[len(times) // 2]


def make_pool(fh, gen, np, bits, n, k, count_bytes, seed):
    code_bytes = {8: 1, 16: 2}[bits]
    lo, hi, dt = (-32768, 32767, np.int16) if bits == 16 else (-127, 127, np.int8)
    codes = gen.codes_uniform((n, k), lo, hi, dt, seed)
    scales = gen.uniform((n, k // 64), 1e-6, 4e-6, seed + 1) if bits == 16 else gen.uniform((n, k // 64), 1e-4, 4e-4, seed + 1)
    per = n * k * code_bytes
    copies = max(2, -(-count_bytes // per))
    return codes, scales, [fh.QuantLinear(bits, codes, scales, 64) for _ in range(copies)]


def bench_gemv(torch, fh, gen, np, bits, rows, steps, warmup, graph=True, n=4096, k=1024):
    """Decode GEMV over a rotating pool; returns whole-job and per-launch numbers."""
    # A 512 MiB buffer (twice the 256 MB Infinity Cache), written before the
    # pool's uploads push its lines out of the cache, read before the timed
    # replay (below).
    flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    codes, scales, pool = make_pool(fh, gen, np, bits, n, k, POOL_BYTES, 1 if bits == 16 else 4)
    x = torch.from_numpy(gen.normal((rows, k), 1.0, 3)).cuda()
    out = torch.empty((rows, n), device="cuda")
    nbytes = gemv_bytes(n, k, rows, 2 if bits == 16 else 1)
    step = lambda i: pool[i % len(pool)].linear(x, rows, out)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    # Whole job: K steps replayed from a HIP graph (or launched directly).
    ctx = fh.default_context()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            ctx.use_stream(s)
            with torch.cuda.graph(g, stream=s):
                ctx.use_stream(torch.cuda.current_stream())
                for i in range(steps):
                    step(i)
        stream.wait_stream(s)
        ctx.use_stream(stream)
        g.replay()
        torch.cuda.synchronize()
        run = g.replay
    else:
        def run():
            for i in range(steps):
                step(i)
    # The warm-up replay just touched the first K copies of the pool; reading
    # the flush buffer evicts them, so that the timed steps read their weights
    # from HBM whatever K is. A read, not a write: a decode step's other
    # matrices and caches pass through the cache as reads, and a freshly
    # written buffer would leave dirty lines whose write-back the timed reads
    # would pay for.
    float(flush.sum())
    # Timed region: barrier, events on the launch stream around the K steps.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    window_ms = ev0.elapsed_time(ev1) / steps
    # The launches' own duration: the same K steps once more after another
    # flush, with the stream held by a bounded sleep (no memory traffic)
    # while the host submits them, so the events bracket the K kernels and
    # not the host's submission of the replay (which the window above, and
    # the whole-job wall clock, include).
    float(flush.sum())
    del flush
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SUBMIT_COVER_CYCLES)
    k0.record(stream)
    run()
    k1.record(stream)
    torch.cuda.synchronize()
    avg_ms = k0.elapsed_time(k1) / steps
    return {"bytes": nbytes, "wall_s": wall, "steps": steps, "avg_launch_ms": avg_ms, "window_ms": window_ms,
            "pool_copies": len(pool), "codes": codes, "scales": scales, "x": x, "cache_flushed": True}


def bench_gemv_sustained(torch, fh, gen, np, graph=True, k=1024, ns=(4096, 16384, 65536, 131072, 262144)):
    """The INT8 g64 GEMV (M = 1) at growing output widths, each launch on a
    cold copy: per-launch time t(B) over algorithmic bytes B, and the
    least-squares line t = t0 + B / R over the points from 16,384 channels
    up. R is the rate the kernel streams at once its launch is long enough to
    hide t0, the fixed cost of a launch (dispatch, first-byte latency, drain)."""
    points = []
    for n in ns:
        r = bench_gemv(torch, fh, gen, np, 8, 1, 200 if n <= 65536 else 60, 5, graph=graph, n=n, k=k)
        us = r["avg_launch_ms"] * 1e3
        points.append({"n": n, "bytes": r["bytes"], "launch_us": round(us, 3), "gbs": round(r["bytes"] / us / 1e3, 1),
                       "frac_hbm": round(r["bytes"] / us / 1e3 / HBM_PEAK_GBS, 3), "pool_copies": r["pool_copies"]})
    fit = [p for p in points if p["n"] >= 16384]
    slope, t0 = np.polyfit(np.array([p["bytes"] for p in fit], float), np.array([p["launch_us"] for p in fit], float), 1)
    rate = 1e-3 / slope  # GB/s
    return {"k": k, "points": points,
            "fit": {"over_n": [p["n"] for p in fit], "t0_us": round(float(t0), 3), "streaming_gbs": round(float(rate), 1),
                    "streaming_frac_hbm": round(float(rate) / HBM_PEAK_GBS, 3)}}


def bench_gemm(torch, fh, gen, np, reps, bits=32):
    """BASELINE config 1 (FP32, m = 6544) on the checkpoint shapes and the
    literal shape; with bits=16 the same projections on a near-exact body
    (INT16 g64 codes, scales U(1e-6, 4e-6), dequantized fl(code * scale) as
    the kernels stage them: the FP32 panels' exact chain is near-exact
    mode's prefill projection)."""
    m = 6544
    shapes = [("qkv", 768, 2048, fh.Epilogue.STORE), ("wo", 1024, 768, fh.Epilogue.ADD),
              ("w13", 768, 4608, fh.Epilogue.GLU), ("w2", 2304, 768, fh.Epilogue.ADD),
              ("literal", 1024, 4096, fh.Epilogue.STORE)]
    timer = Timer(torch)
    res = {}
    for name, k, n, epi in shapes:
        a = torch.from_numpy(gen.normal((m, k), 1.0, 10)).cuda()
        if bits == 32:
            lin = fh.Linear.from_f32(gen.normal((n, k), 0.02, 11))
        else:
            lin = fh.QuantLinear(16, gen.codes_uniform((n, k), -32767, 32767, np.int16, 11),
                                 gen.uniform((n, k // 64), 1e-6, 4e-6, 12), 64)
        width = n // 2 if epi == fh.Epilogue.GLU else n
        out = torch.zeros((m, width), device="cuda")
        kernels = [fh.PrefillProjection.F32_MFMA, fh.PrefillProjection.F32_CHAIN]
        if bits == 32:
            kernels.append(fh.PrefillProjection.F32_SPLIT)
        for kern in kernels:
            fn = lambda i: lin.prefill(a, m, epilogue=epi, out=out, kernel=kern)
            for i in range(2):
                fn(i)
            avg, med = timer.per_launch_ms(fn, reps)
            flops = 2.0 * m * k * n
            tag = {fh.PrefillProjection.F32_MFMA: "mfma", fh.PrefillProjection.F32_CHAIN: "chain",
                   fh.PrefillProjection.F32_SPLIT: "split"}[kern]
            tflops = flops / (avg * 1e-3) / 1e12
            peak = FP32_VECTOR_PEAK if tag == "chain" else FP32_MFMA_PEAK
            res[f"{name}_{tag}"] = {"ms": round(avg, 4), "tflops": round(tflops, 2), "frac": round(tflops / peak, 3)}
            if tag == "split":
                # Three FP16 pair products per FP32 product: the FP16 matrix-
                # core work done, against the 2.5 PFLOP/s dense FP16 peak.
                res[f"{name}_{tag}"]["f16_frac"] = round(3 * tflops / F16_MFMA_PEAK, 3)
        lin.free()
    return res


def bench_i16(torch, fh, gen, np, reps):
    """BASELINE config 3 prefill: X[6544 x k] FP32 -> INT16 activations x INT8 codes."""
    m = 6544
    shapes = [("literal", 1024, 4096, fh.Epilogue.STORE), ("qkv", 768, 2048, fh.Epilogue.STORE),
              ("wo", 1024, 768, fh.Epilogue.ADD), ("w13", 768, 4608, fh.Epilogue.GLU),
              ("w2", 2304, 768, fh.Epilogue.ADD)]
    timer = Timer(torch)
    res = {}
    for name, k, n, epi in shapes:
        a = torch.from_numpy(gen.normal((m, k), 1.0, 7)).cuda()
        codes = gen.codes_uniform((n, k), -127, 127, np.int8, 8)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 9)
        lin = fh.QuantLinear(8, codes, scales, 64)
        width = n // 2 if epi == fh.Epilogue.GLU else n
        out = torch.zeros((m, width), device="cuda")
        fn = lambda i: lin.prefill(a, m, epilogue=epi, out=out, kernel=fh.PrefillProjection.I16)
        for i in range(2):
            fn(i)
        avg, med = timer.per_launch_ms(fn, reps)
        ops = 2.0 * m * k * n
        res[name] = {"ms": round(avg, 4), "tops": round(ops / (avg * 1e-3) / 1e12, 2)}
        lin.free()
    return res


def bench_attention(torch, fh, gen, np, reps):
    """6,544 tokens, 16 heads x 64 (8 KV heads), image prefix 4,096."""
    L, img = 6544, 4096
    q = torch.from_numpy(gen.normal(L * 16 * 64, 1.0, 20)).cuda()
    k = torch.from_numpy(gen.normal(L * 16 * 64, 1.0, 21)).cuda()
    v = torch.from_numpy(gen.normal(L * 8 * 64, 1.0, 22)).cuda()
    sinks = torch.from_numpy(gen.uniform(16, -2.0, 2.0, 23)).cuda()
    out = torch.empty_like(q)
    kv = fh.CompactKv.prefill(k, v, L, 16, 8)
    visible = img * img + sum(qq + 1 for qq in range(img, L))
    flops = 4.0 * 64 * visible * 16
    res = {"visible_pairs_per_head": visible, "gflop": round(flops / 1e9, 2)}
    timer = Timer(torch)
    # FP32 products from scaled FP16 pairs (the default on a pure prefill),
    # then on the FP32 matrix cores (split_products=False).
    for name, opts in (("online_fast", fh.PrefillOptions()), ("static", fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC)),
                       ("online_fast_fp32_mfma", fh.PrefillOptions(split_products=False)),
                       ("static_fp32_mfma", fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC, split_products=False))):
        fn = lambda i: fh.attention_with(q, kv, L, fh.Geometry(0, 0, img), sinks, opts, output=out)
        for i in range(2):
            fn(i)
        avg, med = timer.per_launch_ms(fn, reps)
        res[name] = {"ms": round(avg, 4), "tflops": round(flops / (avg * 1e-3) / 1e12, 2)}
    # A8: the BF16 kernels (K/V conversion included in the timed launch).
    for name, sm in (("bf16_online", fh.Softmax.ONLINE), ("bf16_static", fh.Softmax.STATIC)):
        opts = fh.PrefillOptions(softmax=sm)
        fn = lambda i: fh.attention_prefill_bf16(q, kv, L, fh.Geometry(0, 0, img), sinks, out, opts)
        for i in range(2):
            fn(i)
        avg, med = timer.per_launch_ms(fn, reps)
        res[name] = {"ms": round(avg, 4), "tflops": round(flops / (avg * 1e-3) / 1e12, 2)}
    return res


def bench_layer(torch, fh, gen, np, steps=64):
    """one GPTQ INT8 g64 decoder layer (checkpoint shapes:
    dim 768, QKV 768->2048, WO 1024->768, W13 768->4608 + GLU, W2 2304->768;
    16 query / 8 KV heads of 64) prefilled over P = 16,320 rows (image
    [0, 4096)), then `steps` greedy decode steps growing the cache to 16,384,
    first over the compact FP32 cache (Kv::Compact), then over the sealed Q8
    records (Kv::Q8: the prefill seals the prefix after its attention; fast
    mode's decode exp for Q8, default_fast_exp), then
    with fast mode's BF16 prefill attention as well (`fast_plan`).
    Prefill stages are timed with HIP events (the layer's phase marks); the
    decode steps are captured into one HIP graph and replayed."""
    P, img, dim, heads, kv = 16384 - steps, 4096, 768, 16, 8
    qd, kd, ffn = heads * 64, kv * 64, 2304
    shapes = {"qkv": (qd + 2 * kd, dim), "wo": (dim, qd), "w13": (2 * ffn, dim), "w2": (dim, ffn)}
    lins = {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        codes = gen.codes_uniform((n, k), -127, 127, np.int8, 30 + 2 * i)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 31 + 2 * i)
        lins[name] = fh.QuantLinear(8, codes, scales, 64)
    sinks = torch.from_numpy(gen.uniform(heads, -2.0, 2.0, 40)).cuda()
    ang = gen.uniform((P + steps, heads, 32), -3.14159, 3.14159, 41)
    ang[:, 1::2, :16] = ang[:, 0::2, :16]  # 2D RoPE: a GQA pair shares the temporal pairs
    rope = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)).cuda()
    h0 = torch.from_numpy(gen.normal((P, dim), 1.0, 42)).cuda()
    xs = torch.from_numpy(gen.normal((steps, 1, dim), 1.0, 43)).cuda()
    stream = torch.cuda.current_stream()
    ctx = fh.default_context()
    proj_flop = 2.0 * P * sum(n * k for n, k in shapes.values())
    visible = img * img + sum(q + 1 for q in range(img, P))
    attn_flop = 4.0 * 64 * visible * heads
    # Bytes per decode step: the four matrices' GEMV tiles and scales plus
    # the visible cache at the average length.
    w_bytes = sum(n * k + 4 * n * (k // 64) for n, k in shapes.values())
    avg_total = P + (steps + 1) / 2.0

    def run(kv_bits, bf16=False):
        layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], sinks, capacity=P + steps,
                                kv_bits=kv_bits, bf16_attention=bf16)
        # Prefill: one untimed pass (allocates the workspace), then a timed one.
        marks = []
        clock = lambda stage: marks.append((stage, torch.cuda.Event(enable_timing=True))) or \
            marks[-1][1].record(stream)
        layer.prefill(h0.clone(), rope[:P], 0, img)
        h = h0.clone()
        layer.len = 0
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        layer.prefill(h, rope[:P], 0, img, clock=clock)
        torch.cuda.synchronize()
        stage_ms, prev = {}, start
        for stage, ev in marks:
            stage_ms[stage] = round(prev.elapsed_time(ev), 4)
            prev = ev
        prefill_ms = start.elapsed_time(marks[-1][1])
        # Decode: a warm step allocates the decode workspace; the cache is
        # then truncated back to the prompt and the `steps` steps are
        # captured and replayed once.
        layer.decode(xs[0].clone(), rope[P:P + 1])
        layer.truncate(P)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                ctx.use_stream(torch.cuda.current_stream())
                for t in range(steps):
                    layer.decode(xs[t], rope[P + t:P + t + 1])
        stream.wait_stream(cap)
        ctx.use_stream(stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        decode_ms = e0.elapsed_time(e1)
        if kv_bits == 32:
            # Prefix keys per query head, generated keys per KV head, values.
            kv_bytes = 4 * 64 * (P * heads + (avg_total - P) * kv + avg_total * kv)
            cache_bytes = 4 * 64 * (P + steps) * (heads + 2 * kv)
        else:
            # Stored records: 176 bytes per prefix position and group (160
            # codes, five BF16 steps, padded to 16 bytes), 144 per tail one.
            _, _, _, _, cache_bytes = layer.split.info()
            kv_bytes = kv * (P * 176 + (avg_total - P) * 144)
        step_bytes = w_bytes + kv_bytes
        fast_exp = layer.decode_fast_exp
        del g
        layer.free()
        return {"prefill_ms": round(prefill_ms, 3), "prefill_stage_ms": stage_ms,
                "prefill_tflops": round((proj_flop + attn_flop) / (prefill_ms * 1e-3) / 1e12, 2),
                "decode_us_per_step": round(decode_ms * 1e3 / steps, 2), "decode_bytes_per_step": int(step_bytes),
                "decode_gbs": round(step_bytes / (decode_ms * 1e-3 / steps) / 1e9, 1),
                "decode_frac_hbm": round(step_bytes / (decode_ms * 1e-3 / steps) / 1e9 / HBM_PEAK_GBS, 3),
                "cache_bytes": int(cache_bytes), "decode_fast_exp": fast_exp}

    res = {"prefill_rows": P, "decode_steps": steps, "prefill_gflop": round((proj_flop + attn_flop) / 1e9, 2)}
    res.update(run(32))
    res["q8"] = run(8)
    # Fast mode's whole plan (w8-body-kv-q8 with hip-i16 + hip-bf16-static):
    # BF16 static-softmax prefill attention, then decode over Q8 records.
    res["fast_plan"] = run(8, bf16=True)
    for lin in lins.values():
        lin.free()
    return res


def bench_kv(torch, fh, gen, np, reps=30):
    """Decode attention of one query row over one layer's cache, cold (a
    512 MiB read before every call evicts the Infinity Cache, as the other
    layers' weights and caches do between a layer's steps; a read, so no
    dirty lines are left for the timed call to write back): sealed Q8 records
    (focr_kv_attention_decode) against the FP32 compact cache
    (focr_attention_decode), at 4,096 / 16,320 / 65,472 prefix positions plus
    64 generated ones; the Q8 records with the exact exp and with the fast
    exp (q8_fast_us: the reference runner's default for Q8 caches in fast
    mode, default_fast_exp). Bytes = the records (176 B per group and prefix
    position, 144 per generated one) or the compact keys and values."""
    heads, kvh, T = 16, 8, 64
    flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    res = {}

    def cold_us(fn):
        for _ in range(3):
            fn()
        ts = []
        for _ in range(reps):
            flush.sum()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        ts.sort()
        return ts[len(ts) // 2]

    for P in (4096, 16320, 65472):
        k = gen.normal((P, 2 * kvh, 64), 1.0, 60)
        k[:, 1::2, :32] = k[:, 0::2, :32]  # the pair's shared temporal half
        v = gen.normal((P, kvh, 64), 1.0, 61)
        gk = torch.from_numpy(gen.normal((T, kvh, 64), 1.0, 62)).cuda()
        gv = torch.from_numpy(gen.normal((T, kvh, 64), 1.0, 63)).cuda()
        q = torch.from_numpy(gen.normal((1, heads, 64), 1.0, 64)).cuda()
        sinks = torch.from_numpy(gen.uniform(heads, -2.0, 2.0, 65)).cuda()
        out = torch.empty((1, heads, 64), device="cuda")
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
        split = fh.KvSplit.seal(8, kd, vd, P, P + T, heads, kvh)
        split.append(gk, gv, T)
        q8_us = cold_us(lambda: split.attention_decode(q, 1, sinks, out=out))
        split.set_fast_exp(True)
        q8_fast_us = cold_us(lambda: split.attention_decode(q, 1, sinks, out=out))
        split.free()
        vals = torch.cat([vd, gv])
        kv = fh.CompactKv(kd, gk, vals, P, P + T, heads, kvh, 64)
        geo = fh.Geometry(P + T - 1, 0, 4096)
        f32_us = cold_us(lambda: fh.attention_decode(q, kv, 1, geo, sinks, output=out))
        q8_bytes = kvh * (P * 176 + T * 144)
        f32_bytes = 4 * 64 * (P * heads + T * kvh + (P + T) * kvh)
        res[f"prefix_{P}"] = {"q8_us": round(q8_us, 2), "q8_bytes": q8_bytes,
                              "q8_gbs": round(q8_bytes / (q8_us * 1e-6) / 1e9, 1),
                              "q8_fast_us": round(q8_fast_us, 2),
                              "q8_fast_gbs": round(q8_bytes / (q8_fast_us * 1e-6) / 1e9, 1),
                              "compact_us": round(f32_us, 2), "compact_bytes": f32_bytes,
                              "compact_gbs": round(f32_bytes / (f32_us * 1e-6) / 1e9, 1),
                              "speedup": round(f32_us / q8_us, 2)}
        del kd, vd, vals
    del flush
    return res


def bench_screen(torch, fh, gen, np, reps=40):
    """The INT8 screened vocabulary head (65,536 x 768, FP32 head N(0, 0.02)):
    one exact greedy selection per call (rows 1 and 5, synchronous, host wall
    time) against the full FP32 head GEMV + argmax. "warm": back-to-back
    calls (the 201 MB FP32 head stays in the 256 MB Infinity Cache); "cold":
    a 512 MiB read between calls evicts it first, as the other layers'
    weights and caches do in a decode step."""
    vocab, dim = 65536, 768
    head = gen.normal((vocab, dim), 0.02, 40)
    screen = fh.ScreenedHead.build(head)
    lin = fh.Linear.from_f32(head)
    flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    screen_bytes = vocab * (dim + 4 * (dim // 64))
    res = {"vocab": vocab, "dim": dim, "screen_bytes": screen_bytes, "fp32_head_bytes": vocab * dim * 4}

    def timed(fn, cold):
        t = []
        for _ in range(reps):
            if cold:
                flush.sum()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        t.sort()
        return t[len(t) // 2]

    for rows in (1, 5):
        x = torch.from_numpy(gen.normal((rows, dim), 1.0, 41)).cuda()
        out = torch.empty((rows, vocab), device="cuda")
        sel = screen.select(x, rows, lin)
        select = lambda: screen.select(x, rows, lin)
        full = lambda: (lin.linear(x, rows, out), fh.argmax(out, rows, vocab))
        for _ in range(3):
            select()
            full()
        entry = {"candidates": [c for _, c in sel]}
        for cold in (False, True):
            s_med, f_med = timed(select, cold), timed(full, cold)
            tag = "cold" if cold else "warm"
            entry[tag] = {"select_us": round(s_med * 1e6, 1), "full_head_us": round(f_med * 1e6, 1),
                          "speedup": round(f_med / s_med, 2)}
        res[f"rows{rows}"] = entry
    screen.free()
    lin.free()
    del flush
    return res


def bench_copy(torch, reps):
    """A plain device copy of known size (calibrates rocprofv3 FETCH/WRITE_SIZE)."""
    n = 256 << 20
    src = torch.empty(n // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    fn = lambda i: dst.copy_(src)
    avg, med = Timer(torch).per_launch_ms(fn, reps)
    return {"bytes_read": n, "bytes_written": n, "ms": round(avg, 4), "gbs": round(2 * n / (avg * 1e-3) / 1e9, 1)}


def bench_launch_floor(torch, steps=2000):
    """What a launch costs in the headline's own setup (K launches replayed
    from one HIP graph, HIP events around the replay): a one-workgroup fill
    (4 bytes: the dispatch floor), and a plain device copy moving the headline
    GEMV's 8,671,232 bytes (4,335,616 read from a rotating 520 MB pool of
    sources, so they come from HBM, and as many written)."""
    res = {}
    tiny = torch.zeros(1, device="cuda")
    n = 8671232 // 2 // 4
    pool = [torch.ones(n, device="cuda") for _ in range(120)]
    dst = torch.empty(n, device="cuda")
    for name, fn in (("fill_4B", lambda i: tiny.fill_(1.0)),
                     ("copy_8.67MB_from_pool", lambda i: dst.copy_(pool[i % len(pool)]))):
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                for i in range(steps):
                    fn(i)
        torch.cuda.current_stream().wait_stream(cap)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_us"] = round(e0.elapsed_time(e1) * 1e3 / steps, 3)
        del g
    del pool
    return res


def host_facts():
    """The host CPU the baselines run on: logical CPUs, the CPUs this job may
    use (affinity, capped by OMP_NUM_THREADS, the one-GPU job's host share),
    the physical cores among them, model, clock and the ISA flags the
    reference's kernels select on (avx2/fma: the AVX2 panels and tiles;
    avx512f/vl: the 16-lane attention tiles; avx512_vnni / avx512_bf16: the
    VNNI INT16 panels and the BF16 attention)."""
    import oracle

    facts = {"nproc": os.cpu_count()}
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = list(range(os.cpu_count() or 1))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    share = len(allowed)
    if omp.isdigit() and int(omp) > 0:
        share = min(share, int(omp))
    facts["affinity"] = len(allowed)
    facts["omp_num_threads"] = omp or None
    facts["share"] = share
    cores = set()
    for cpu in allowed[:share]:
        base = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology")
        try:
            cores.add(((base / "physical_package_id").read_text().strip(), (base / "core_id").read_text().strip()))
        except OSError:
            cores.add(("?", str(cpu)))
    facts["physical_cores_in_share"] = len(cores)
    try:
        count = 0
        for part in Path("/sys/devices/system/cpu/cpu0/topology/thread_siblings_list").read_text().strip().split(","):
            lo, _, hi = part.partition("-")
            count += int(hi) - int(lo) + 1 if hi else 1
        facts["threads_per_core"] = count
    except (OSError, ValueError):
        facts["threads_per_core"] = None
    model, mhz = None, []
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and model is None:
                model = line.split(":", 1)[1].strip()
            elif line.startswith("cpu MHz"):
                mhz.append(float(line.split(":", 1)[1]))
    except OSError:
        pass
    facts["model"] = model
    try:
        facts["max_mhz"] = int(Path("/sys/devices/system/cpu/cpu0/cpufreq/cpuinfo_max_freq").read_text()) // 1000
    except (OSError, ValueError):
        facts["max_mhz"] = None
    facts["mean_mhz"] = round(sum(mhz) / len(mhz)) if mhz else None
    flags = oracle.cpu_flags()
    facts["isa"] = [f for f in ("avx2", "fma", "avx512f", "avx512vl", "avx512bw", "avx512_vnni", "avx512_bf16",
                                "amx_tile") if f in flags]
    facts["oracle_build"] = oracle.variant()
    return facts


def cpu_baseline(np, gen, facts, seconds=10.0):
    """The reference's AVX2 INT16 GEMV (dot_q restated in oracle/focr_cpu_gemv.c,
    bitwise the oracle) on the host cores, on the headline matrix. Like the GPU side, calls rotate through a pool of copies
    (1 GiB, above any host last-level cache) so weights stream from DRAM."""
    import oracle

    # The reference's decode team: one thread per physical core (docs/PERFORMANCE.md:48).
    threads = max(1, facts["physical_cores_in_share"])
    oracle.set_threads(threads)
    n, k = 4096, 1024
    codes = gen.codes_uniform((n, k), -32768, 32767, np.int16, 1)
    scales = gen.uniform((n, k // 64), 1e-6, 4e-6, 2)
    x = gen.normal((1, k), 1.0, 3)
    pool = [(codes.copy(), scales.copy()) for _ in range(max(2, (1 << 30) // codes.nbytes))]
    oracle.linear_decode(16, codes, scales, n, k, 64, x, 1, fast=True)
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < 5:
        c, sc = pool[i % len(pool)]
        t0 = time.perf_counter()
        oracle.linear_decode(16, c, sc, n, k, 64, x, 1, fast=True)
        times.append(time.perf_counter() - t0)
        i += 1
    times.sort()
    med = times[len(times) // 2]
    oracle.set_threads(1)
    return {"value": round(gemv_bytes(n, k, 1, 2) / med / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"INT16 g64 GEMV W[4096x1024] M=1 over a {len(pool)}-copy pool (1 GiB), median of {len(times)} "
                      f"calls in ~{seconds:.0f} s (oracle/focr_cpu_gemv.c: the reference's AVX2 dot_q, OpenMP, one thread per physical core of the "
                      f"job's {facts['share']}-CPU host share; host {facts['nproc']} logical CPUs, {facts['model']})",
            "host": facts}


def cpu_prefill_page(np, gen, gpu_gemm, gpu_attention, facts, reps=2):
    """The FP32 prefill of one 6,544-token page on the host cores against the
    GPU's: the literal projection X[6544x1024] x W[1024x4096] and the four
    checkpoint projections, each plus the config-4 attention (16 heads, image
    prefix 4,096). The CPU side runs the reference's AVX2 panel micro-kernel
    and the attention tile vectorized over the query lanes (bitwise the
    oracle's results), over the whole page; best of `reps` calls each."""
    import oracle

    # The reference's prefill pool: every logical CPU it may use (threads = 0,
    # src/config.rs:391-395) -- here the job's host share.
    threads = max(1, facts["share"])
    oracle.set_threads(threads)
    m = 6544

    def best(fn):
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return min(t) * 1e3

    cpu = {}
    for name, k, n, epi in (("literal", 1024, 4096, oracle.STORE), ("qkv", 768, 2048, oracle.STORE),
                            ("wo", 1024, 768, oracle.ADD), ("w13", 768, 4608, oracle.GLU),
                            ("w2", 2304, 768, oracle.ADD)):
        a = gen.normal((m, k), 1.0, 10)
        w = gen.normal((n, k), 0.02, 11)
        cpu[name] = best(lambda: oracle.panel_gemm_fast(a, m, k, w, n, epilogue=epi))
        log(f"cpu {name} GEMM: {cpu[name]:.1f} ms")
    L, img = 6544, 4096
    q, k = gen.normal(L * 16 * 64, 1.0, 20), gen.normal(L * 16 * 64, 1.0, 21)
    v, sinks = gen.normal(L * 8 * 64, 1.0, 22), gen.uniform(16, -2.0, 2.0, 23)
    cpu["attention"] = best(lambda: oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, 0, img, sinks))
    log(f"cpu attention: {cpu['attention']:.1f} ms")
    # Thread scaling of the literal GEMM and the attention (half the share).
    half = max(1, threads // 2)
    oracle.set_threads(half)
    a = gen.normal((m, 1024), 1.0, 10)
    w = gen.normal((4096, 1024), 0.02, 11)
    half_ms = {"literal": round(best(lambda: oracle.panel_gemm_fast(a, m, 1024, w, 4096)), 2),
               "attention": round(best(lambda: oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, 0, img,
                                                                            sinks)), 2)}
    oracle.set_threads(1)
    # MACs per cycle per core of the FP32 panels (the reference's 7700X: about
    # 14.3 of a 16-MAC ceiling, docs/PERFORMANCE.md:544-558), at the clock the
    # host reports (its maximum if known, else the mean current clock).
    ghz = (facts.get("max_mhz") or facts.get("mean_mhz") or 0) / 1000.0
    cores = max(1, facts["physical_cores_in_share"])
    macs_cycle_core = None
    if ghz:
        macs_cycle_core = round(m * 1024 * 4096 / (cpu["literal"] * 1e-3) / (cores * ghz * 1e9), 2)
    layer = ("qkv", "wo", "w13", "w2")
    # The GPU side runs exact mode's plan: the FP32 projections from FP16
    # pairs (hip-f32-split) and the online FP32 attention on FP16 pairs.
    gpu_literal = gpu_gemm["literal_split"]["ms"] + gpu_attention["online_fast"]["ms"]
    gpu_layer = sum(gpu_gemm[f"{s}_split"]["ms"] for s in layer) + gpu_attention["online_fast"]["ms"]
    cpu_literal = cpu["literal"] + cpu["attention"]
    cpu_layer = sum(cpu[s] for s in layer) + cpu["attention"]
    return {"cores": threads, "kind": "port", "physical_cores": cores, "ghz_assumed": ghz or None,
            "gemm_macs_per_cycle_per_core": macs_cycle_core, "reference_macs_per_cycle_per_core": 14.3,
            "cpu_ms": {s: round(t, 2) for s, t in cpu.items()},
            "cpu_ms_half_threads": {"threads": half, **half_ms},
            "literal_page": {"gpu_ms": round(gpu_literal, 4), "cpu_ms": round(cpu_literal, 1),
                             "speedup": round(cpu_literal / gpu_literal, 1)},
            "layer_page": {"gpu_ms": round(gpu_layer, 4), "cpu_ms": round(cpu_layer, 1),
                           "speedup": round(cpu_layer / gpu_layer, 1)},
            "sample": f"whole page, best of {reps} calls, OpenMP {threads} threads = the job's host share of "
                      f"{facts['nproc']} logical CPUs ({facts['model']}); oracle/focr_cpu_panels.c (AVX2 6x16 panels), "
                      f"oracle/focr_cpu_attention.c ({'16' if facts['oracle_build'] == 'v4' else '8'}-lane tiles, "
                      "online softmax, Fast exp)"}


def cpu_config3(np, gen, gpu_i16, facts, reps=2, gemv_seconds=5.0):
    """BASELINE config 3 on the host cores, as the reference runs it there:
    the INT16-activation x INT8-code prefill GEMM of the five shapes on its
    AVX-512 VNNI panels (oracle/focr_cpu_panels_i16.c: weights packed once as
    at load, activation quantization inside each call; bitwise the oracle),
    every logical CPU of the job's share, best of `reps` calls; and the INT8
    g64 decode GEMV W[4096x1024], M = 1, one thread per physical core over a
    1 GiB pool of copies, median of ~`gemv_seconds` s of calls."""
    import oracle

    threads = max(1, facts["share"])
    oracle.set_threads(threads)
    m = 6544
    gemm = {}
    for name, k, n, epi in (("literal", 1024, 4096, oracle.STORE), ("qkv", 768, 2048, oracle.STORE),
                            ("wo", 1024, 768, oracle.ADD), ("w13", 768, 4608, oracle.GLU),
                            ("w2", 2304, 768, oracle.ADD)):
        a = gen.normal((m, k), 1.0, 7)
        codes = gen.codes_uniform((n, k), -127, 127, np.int8, 8)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 9)
        panels = oracle.I16Panels(codes, scales, n, k)
        base = np.zeros((m, n), np.float32) if epi == oracle.ADD else None
        if panels.gemm(a, m, epilogue=epi, out=base) is None:
            panels.free()
            return {"skipped": "host CPU without AVX-512 VNNI"}
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            panels.gemm(a, m, epilogue=epi, out=base)
            t.append(time.perf_counter() - t0)
        panels.free()
        ms = min(t) * 1e3
        gemm[name] = {"cpu_ms": round(ms, 2), "cpu_tops": round(2.0 * m * k * n / (ms * 1e-3) / 1e12, 3)}
        if name in gpu_i16:
            gemm[name]["gpu_ms"] = gpu_i16[name]["ms"]
            gemm[name]["speedup"] = round(ms / gpu_i16[name]["ms"], 1)
        log(f"cpu i16 GEMM {name}: {ms:.1f} ms")
    ghz = (facts.get("max_mhz") or facts.get("mean_mhz") or 0) / 1000.0
    cores = max(1, facts["physical_cores_in_share"])
    macs = None
    if ghz:
        total_ms = sum(v["cpu_ms"] for v in gemm.values())
        total_macs = m * sum(k * n for _, k, n in ((0, 1024, 4096), (0, 768, 2048), (0, 1024, 768), (0, 768, 4608),
                                                    (0, 2304, 768)))
        macs = {"literal": round(m * 1024 * 4096 / (gemm["literal"]["cpu_ms"] * 1e-3) / (cores * ghz * 1e9), 2),
                "all_five": round(total_macs / (total_ms * 1e-3) / (cores * ghz * 1e9), 2)}
    # The INT8 GEMV on the decode team (one thread per physical core).
    oracle.set_threads(cores)
    n, k = 4096, 1024
    codes = gen.codes_uniform((n, k), -127, 127, np.int8, 1)
    scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 2)
    x = gen.normal((1, k), 1.0, 3)
    pool = [(codes.copy(), scales.copy()) for _ in range(max(2, (1 << 30) // codes.nbytes))]
    oracle.linear_decode(8, codes, scales, n, k, 64, x, 1, fast=True)
    times, i = [], 0
    t_end = time.perf_counter() + gemv_seconds
    while time.perf_counter() < t_end or len(times) < 5:
        c, sc = pool[i % len(pool)]
        t0 = time.perf_counter()
        oracle.linear_decode(8, c, sc, n, k, 64, x, 1, fast=True)
        times.append(time.perf_counter() - t0)
        i += 1
    times.sort()
    med = times[len(times) // 2]
    oracle.set_threads(1)
    return {"gemm": gemm, "gemm_threads": threads, "physical_cores": cores, "ghz_assumed": ghz or None,
            "gemm_macs_per_cycle_per_core": macs, "reference_macs_per_cycle_per_core": [24.5, 27.4],
            "gemv_i8_m1": {"cpu_us": round(med * 1e6, 2), "cpu_gbs": round(gemv_bytes(n, k, 1, 1) / med / 1e9, 2),
                           "threads": cores, "calls": len(times), "pool_copies": len(pool)},
            "kind": "port",
            "sample": f"GEMM: the five config-3 shapes at m = 6,544, best of {reps} calls, OpenMP {threads} threads "
                      f"(the job's host share of {facts['nproc']} logical CPUs, {facts['model']}), "
                      "oracle/focr_cpu_panels_i16.c (the reference's 6 x 32 vpdpwssd panels); GEMV: "
                      f"oracle/focr_cpu_gemv.c (the reference's AVX2 dot_q), {cores} threads, median over a 1 GiB pool"}


def cpu_layer(np, gen, gpu_layer, facts, steps=64):
    """BASELINE config 5 on the host cores with the same plan as the GPU's
    compact-cache run (INT16-activation x INT8-code projections, FP32 online
    attention, FP32 compact cache): the 16,320-row prefill (row scales, QKV on
    the VNNI panels, the QKV row step, attention on the 16-lane tiles, WO, W13
    + GLU, W2) and `steps` decode steps (the reference-order GEMVs, the row
    step, decode attention over the growing cache), with the same seeded
    weights and inputs as bench_layer, once; every logical CPU of the share."""
    import oracle

    threads = max(1, facts["share"])
    oracle.set_threads(threads)
    P, img, dim, heads, kv = 16384 - steps, 4096, 768, 16, 8
    qd, kd, ffn = heads * 64, kv * 64, 2304
    shapes = {"qkv": (qd + 2 * kd, dim), "wo": (dim, qd), "w13": (2 * ffn, dim), "w2": (dim, ffn)}
    mats, panels = {}, {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        codes = gen.codes_uniform((n, k), -127, 127, np.int8, 30 + 2 * i)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 31 + 2 * i)
        mats[name] = (codes, scales, n, k)
        panels[name] = oracle.I16Panels(codes, scales, n, k)
    sinks = gen.uniform(heads, -2.0, 2.0, 40)
    ang = gen.uniform((P + steps, heads, 32), -3.14159, 3.14159, 41)
    ang[:, 1::2, :16] = ang[:, 0::2, :16]
    rope = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    h = gen.normal((P, dim), 1.0, 42)
    xs = gen.normal((steps, 1, dim), 1.0, 43)
    stage = {}

    def timed(name, fn):
        t0 = time.perf_counter()
        r = fn()
        stage[name] = stage.get(name, 0.0) + (time.perf_counter() - t0) * 1e3
        return r

    if panels["qkv"].gemm(np.zeros((1, dim), np.float32), 1) is None:
        return {"skipped": "host CPU without AVX-512 VNNI"}
    t_prefill = time.perf_counter()
    rs = timed("row_scales", lambda: oracle.row_scales(h, dim))
    qkv = timed("qkv", lambda: panels["qkv"].gemm(h, P, row_scale=rs))
    q, pk, _, v = timed("qkv_rows", lambda: oracle.qkv_rows(qkv, P, rope[:P], heads, kv, P))
    attn = timed("attention", lambda: oracle.attention_prefill_fast(q, pk, v, P, P, P, heads, kv, 0, 0, img, sinks))
    h = timed("wo", lambda: panels["wo"].gemm(attn.reshape(P, -1), P, epilogue=oracle.ADD, out=h))
    rs = timed("row_scales", lambda: oracle.row_scales(h, dim))
    gated = timed("w13", lambda: panels["w13"].gemm(h, P, row_scale=rs, epilogue=oracle.GLU))
    h = timed("w2", lambda: panels["w2"].gemm(gated, P, epilogue=oracle.ADD, out=h))
    prefill_ms = (time.perf_counter() - t_prefill) * 1e3
    log(f"cpu layer prefill: {prefill_ms:.0f} ms {({k: round(t, 1) for k, t in stage.items()})}")
    # Decode over the compact cache: prefix keys per query head, generated
    # keys per KV head, values per KV head.
    gk = np.zeros((steps, kv, 64), np.float32)
    vals = np.zeros((P + steps, kv, 64), np.float32)
    vals[:P] = v.reshape(P, kv, 64)
    dec = lambda name, x, glu=False: (oracle.linear_decode_glu if glu else oracle.linear_decode)(
        8, mats[name][0], mats[name][1], mats[name][2], mats[name][3], 64, x, 1, fast=True)
    t_dec = time.perf_counter()
    for t in range(steps):
        x = xs[t]
        qkv1 = dec("qkv", x * oracle.row_scales(x, dim)[:, None])
        q1, _, nk, nv = oracle.qkv_rows(qkv1, 1, rope[P + t:P + t + 1], heads, kv, 0)
        gk[t] = nk[0]
        vals[P + t] = nv[0]
        a1 = oracle.attention_decode(q1, pk, gk[:t + 1], vals[:P + t + 1], 1, P, P + t + 1, heads, kv, P + t, 0, img,
                                     sinks, fast=True)
        x = x + dec("wo", a1.reshape(1, -1))
        g1 = dec("w13", x * oracle.row_scales(x, dim)[:, None], glu=True)
        x = x + dec("w2", g1)
    decode_us = (time.perf_counter() - t_dec) * 1e6 / steps
    for p in panels.values():
        p.free()
    oracle.set_threads(1)
    res = {"cpu_prefill_ms": round(prefill_ms, 1), "cpu_prefill_stage_ms": {k: round(t, 1) for k, t in stage.items()},
           "cpu_decode_us_per_step": round(decode_us, 1), "threads": threads, "kind": "port",
           "sample": f"one layer, prefill of {P} rows then {steps} decode steps, once; OpenMP {threads} threads "
                     f"(the job's host share of {facts['nproc']} logical CPUs, {facts['model']}); "
                     "oracle/focr_cpu_panels_i16.c, oracle/focr_cpu_attention.c, oracle/focr_cpu_gemv.c (GEMVs, "
                     "decode attention), oracle/focr_oracle.c (row scales, row step)"}
    if gpu_layer:
        res["gpu_prefill_ms"] = gpu_layer["prefill_ms"]
        res["gpu_decode_us_per_step"] = gpu_layer["decode_us_per_step"]
        res["prefill_speedup"] = round(prefill_ms / gpu_layer["prefill_ms"], 1)
        res["decode_speedup"] = round(decode_us / gpu_layer["decode_us_per_step"], 1)
    return res


def measured_traffic():
    """traffic_bytes_per_launch from the committed PMC summary, or None."""
    import re

    try:
        m = re.search(r"traffic_bytes_per_launch\s*=\s*(\d+)", TRAFFIC_FILE.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--ops", default="gemv,gemm,nearexact,i16,attention,layer,kv,screen,copy")
    ap.add_argument("--reps", type=int, default=20, help="timed launches per secondary op")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the kernels run on one GPU's share).", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import focr_hip as fh
    import gen

    ops = set(args.ops.split(","))
    torch.cuda.init()
    fh.default_context()
    log(f"device: {torch.cuda.get_device_name(0)}")
    head = bench_gemv(torch, fh, gen, np, 16, 1, args.steps, args.warmup, graph=not args.no_graph)
    log(f"gemv16 M=1: wall {head['wall_s'] * 1e3:.2f} ms / {args.steps} steps, launch {head['avg_launch_ms'] * 1e3:.2f} us"
        f" (event window of the timed replay {head['window_ms'] * 1e3:.2f} us per step)")
    ms_per_step = head["wall_s"] * 1e3 / args.steps
    value = head["bytes"] / (head["wall_s"] / args.steps) / 1e9
    achieved = head["bytes"] / (head["avg_launch_ms"] * 1e-3) / 1e9
    per_op = {"gemv_i16_m1": {"bytes": head["bytes"], "launch_us": round(head["avg_launch_ms"] * 1e3, 3),
                              "gbs_per_launch": round(achieved, 1), "gbs_whole_job": round(value, 1),
                              "timed_window_us_per_step": round(head["window_ms"] * 1e3, 3),
                              "pool_copies": head["pool_copies"]}}
    if "gemv" in ops:
        for bits, rows in ((16, 5), (8, 1), (8, 5)):
            r = bench_gemv(torch, fh, gen, np, bits, rows, max(200, args.steps // 4), 10, graph=not args.no_graph)
            key = f"gemv_i{bits}_m{rows}"
            per_op[key] = {"bytes": r["bytes"], "launch_us": round(r["avg_launch_ms"] * 1e3, 3),
                           "gbs_per_launch": round(r["bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9, 1),
                           "gbs_whole_job": round(r["bytes"] / (r["wall_s"] / r["steps"]) / 1e9, 1),
                           "frac_hbm_per_launch": round(r["bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
            log(f"{key}: {per_op[key]}")
        # The same INT8 kernel on larger single launches: the model's W13
        # (4608 x 768), a 16384 x 1024 matrix and the 65,536 x 768 vocabulary
        # head (the screened head's GEMV), each from a > 512 MB pool.
        for n, k in ((4608, 768), (16384, 1024), (65536, 768)):
            r = bench_gemv(torch, fh, gen, np, 8, 1, 200, 10, graph=not args.no_graph, n=n, k=k)
            key = f"gemv_i8_m1_{n}x{k}"
            per_op[key] = {"bytes": r["bytes"], "launch_us": round(r["avg_launch_ms"] * 1e3, 3),
                           "gbs_per_launch": round(r["bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9, 1),
                           "frac_hbm_per_launch": round(r["bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
            log(f"{key}: {per_op[key]}")
        per_op["gemv_i8_m1_sustained"] = bench_gemv_sustained(torch, fh, gen, np, graph=not args.no_graph)
        log(f"gemv_i8_m1_sustained: {per_op['gemv_i8_m1_sustained']}")
    if "gemm" in ops:
        per_op["prefill_f32"] = bench_gemm(torch, fh, gen, np, args.reps)
        log(f"prefill_f32: {per_op['prefill_f32']}")
    if "nearexact" in ops:
        per_op["prefill_i16codes"] = bench_gemm(torch, fh, gen, np, args.reps, bits=16)
        log(f"prefill_i16codes: {per_op['prefill_i16codes']}")
    if "i16" in ops:
        per_op["prefill_i16xi8"] = bench_i16(torch, fh, gen, np, args.reps)
        log(f"prefill_i16xi8: {per_op['prefill_i16xi8']}")
    if "attention" in ops:
        per_op["attention_prefill"] = bench_attention(torch, fh, gen, np, max(5, args.reps // 2))
        log(f"attention: {per_op['attention_prefill']}")
    if "layer" in ops:
        per_op["layer_int8_16k"] = bench_layer(torch, fh, gen, np)
        log(f"layer: {per_op['layer_int8_16k']}")
    if "kv" in ops:
        per_op["kv_decode_cold"] = bench_kv(torch, fh, gen, np)
        log(f"kv decode (cold): {per_op['kv_decode_cold']}")
    if "screen" in ops:
        per_op["screened_head_65536x768"] = bench_screen(torch, fh, gen, np)
        log(f"screened head: {per_op['screened_head_65536x768']}")
    if "copy" in ops:
        per_op["copy_256MiB"] = bench_copy(torch, 10)
        per_op["launch_floor"] = bench_launch_floor(torch)
        log(f"launch floor: {per_op['launch_floor']}")
    facts = host_facts()
    log(f"host: {facts}")
    if not args.no_cpu and "prefill_f32" in per_op and "attention_prefill" in per_op:
        per_op["prefill_page_vs_cpu"] = cpu_prefill_page(np, gen, per_op["prefill_f32"], per_op["attention_prefill"],
                                                         facts)
        log(f"prefill page vs CPU: {per_op['prefill_page_vs_cpu']}")
    if not args.no_cpu and "prefill_i16xi8" in per_op:
        per_op["config3_vs_cpu"] = cpu_config3(np, gen, per_op["prefill_i16xi8"], facts)
        log(f"config 3 vs CPU: {per_op['config3_vs_cpu']}")
        for name, r in per_op["config3_vs_cpu"].get("gemm", {}).items():
            per_op["prefill_i16xi8"][name]["cpu_ms"] = r["cpu_ms"]
        if "gemv_i8_m1" in per_op and "gemv_i8_m1" in per_op["config3_vs_cpu"]:
            per_op["gemv_i8_m1"]["cpu_us"] = per_op["config3_vs_cpu"]["gemv_i8_m1"]["cpu_us"]
            per_op["gemv_i8_m1"]["cpu_gbs"] = per_op["config3_vs_cpu"]["gemv_i8_m1"]["cpu_gbs"]
    if not args.no_cpu and "layer_int8_16k" in per_op:
        per_op["layer_int8_16k"]["cpu"] = cpu_layer(np, gen, per_op["layer_int8_16k"], facts)
        log(f"config 5 vs CPU: {per_op['layer_int8_16k']['cpu']}")
    cpu = None if args.no_cpu else cpu_baseline(np, gen, facts)
    line = {
        "metric": "decode GEMV HBM GB/s (INT16 group-64, W 4096x1024, M=1)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i16xf32",
        "data": "synthetic (seeded PCG64: codes uniform [-32768,32767], scales U(1e-6,4e-6), x ~ N(0,1))",
        "config": {"workload": "BASELINE configs[1]: near-exact INT16 g64 decode GEMV, W[4096x1024], M=1",
                   "pool_copies": head["pool_copies"], "graph_replay": not args.no_graph,
                   "infinity_cache_flushed_before_timing": head["cache_flushed"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "per_op": per_op,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
