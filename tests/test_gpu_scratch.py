"""The context scratch and HIP graph capture: a call that would grow the
scratch during capture is refused (FOCR_E_UNSUPPORTED, nothing launched);
after focr_ctx_reserve_scratch the same call captures, and every replay of
the graph, with eager work and synchronizations between the replays, equals
the eager result bit for bit."""
import numpy as np
import pytest

import gen
from gpu_util import assert_bitwise, host, to_dev

pytestmark = pytest.mark.gpu


def test_scratch_growth_refused_during_capture_then_reserved():
    import torch

    import focr_hip as fh

    ctx = fh.Context(0)
    m, k, n = 300, 768, 256
    codes = gen.codes_uniform((n, k), -127, 127, np.int8, 1)
    scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 2)
    lin = fh.QuantLinear(8, codes, scales, 64, ctx=ctx)
    x = to_dev(gen.normal((m, k), 1.0, 3))
    out = torch.empty((m, n), device="cuda:0")
    assert ctx.scratch_bytes() == 0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ctx.use_stream(torch.cuda.current_stream())
            out.zero_()
            with pytest.raises(fh.FocrError, match="stream capture"):
                lin.prefill(x, m, out=out, kernel=fh.PrefillProjection.I16)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() == 0
    del g

    # Reserve, capture, replay.
    ctx.reserve_scratch(8 << 20)
    reserved = ctx.scratch_bytes()
    assert reserved >= 8 << 20
    eager = host(lin.prefill(x, m, kernel=fh.PrefillProjection.I16))
    g = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ctx.use_stream(torch.cuda.current_stream())
            lin.prefill(x, m, out=out, kernel=fh.PrefillProjection.I16)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() == reserved
    for rep in range(3):
        out.fill_(float("nan"))
        lin.prefill(x, m, kernel=fh.PrefillProjection.I16)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bitwise(host(out), eager, f"replay {rep}")
    lin.free()
    ctx.close()


def test_stream_switch_waits_for_the_old_stream():
    # focr_ctx_set_stream orders the new stream after the work already queued
    # on the old one. A STORE prefill queued on stream A behind a clock sleep,
    # then (after the switch) an ADD prefill into the same output on stream B:
    # B's ADD must see A's STORE, as the same two calls on one stream do.
    import torch

    import focr_hip as fh

    ctx = fh.Context(0)
    m, k, n = 96, 256, 128
    lin = fh.Linear.from_f32(gen.normal((n, k), 0.05, 50), ctx=ctx)
    x1 = to_dev(gen.normal((m, k), 1.0, 51))
    x2 = to_dev(gen.normal((m, k), 1.0, 52))
    chain = fh.PrefillProjection.F32_CHAIN
    want = lin.prefill(x1, m, kernel=chain)
    lin.prefill(x2, m, out=want, epilogue=fh.Epilogue.ADD, kernel=chain)
    torch.cuda.synchronize()
    want = host(want)

    a_s, b_s = torch.cuda.Stream(), torch.cuda.Stream()
    out = torch.zeros((m, n), device="cuda:0")
    torch.cuda.synchronize()
    with torch.cuda.stream(a_s):
        torch.cuda._sleep(20_000_000)  # holds stream A for several milliseconds
    ctx.use_stream(a_s)
    lin.prefill(x1, m, out=out, kernel=chain)
    ctx.use_stream(b_s)
    lin.prefill(x2, m, out=out, epilogue=fh.Epilogue.ADD, kernel=chain)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert_bitwise(host(out), want, "ADD on the new stream after STORE on the old")
    lin.free()
    ctx.close()


def test_fp16_pair_paths_capture_and_replay():
    # The FP16-pair attention and GEMM keep their planes, exponents, the
    # non-finite flag and the split plan's partial states in the context
    # scratch and clear what must start at zero with a kernel (no memset
    # node). Once an eager call of each shape has sized the scratch, both
    # capture into one graph; every replay, with eager work between the
    # replays that rewrites the same scratch (a call whose K holds an infinity
    # raises the flag), equals the eager result bit for bit.
    import torch

    import focr_hip as fh

    ctx = fh.Context(0)
    L, image = 1000, (0, 300)
    q = to_dev(gen.normal(L * 16 * 64, 1.0, 61))
    k_np = gen.normal(L * 16 * 64, 1.0, 62)
    k = to_dev(k_np)
    v = to_dev(gen.normal(L * 8 * 64, 1.0, 63))
    sinks = to_dev(gen.uniform(16, -2.0, 2.0, 64))
    k_np[(500 * 16 + 3) * 64] = np.inf
    k_bad = to_dev(k_np)
    geom = fh.Geometry(0, *image)
    kv = fh.CompactKv.prefill(k, v, L, 16, 8)
    kv_bad = fh.CompactKv.prefill(k_bad, v, L, 16, 8)
    m, kk, n = 700, 1024, 768
    lin = fh.Linear.from_f32(gen.normal((n, kk), 0.05, 65), ctx=ctx)
    x = to_dev(gen.normal((m, kk), 1.0, 66))
    x2 = to_dev(gen.normal((m, kk), 1.0, 67))
    split = fh.PrefillProjection.F32_SPLIT
    opts = fh.PrefillOptions()
    att_eager = host(fh.attention_with(q, kv, L, geom, sinks, opts, ctx=ctx))
    gemm_eager = host(lin.prefill(x, m, kernel=split))
    torch.cuda.synchronize()
    sized = ctx.scratch_bytes()

    att_out = torch.empty(L * 16 * 64, device="cuda:0")
    gemm_out = torch.empty((m, n), device="cuda:0")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ctx.use_stream(torch.cuda.current_stream())
            fh.attention_with(q, kv, L, geom, sinks, opts, output=att_out, ctx=ctx)
            lin.prefill(x, m, out=gemm_out, kernel=split)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() == sized
    for rep in range(3):
        att_out.fill_(float("nan"))
        gemm_out.fill_(float("nan"))
        bad = fh.attention_with(q, kv_bad, L, geom, sinks, opts, ctx=ctx)  # eager work between replays
        lin.prefill(x2, m, kernel=split)
        torch.cuda.synchronize()
        assert not bool(torch.all(torch.isfinite(bad)))
        g.replay()
        torch.cuda.synchronize()
        assert_bitwise(host(att_out).reshape(att_eager.shape), att_eager, f"attention replay {rep}")
        assert_bitwise(host(gemm_out), gemm_eager, f"GEMM replay {rep}")
    assert ctx.scratch_bytes() == sized
    lin.free()
    ctx.close()
