"""focr_kv_attention_decode_noalloc, the decode attention over sealed Q8 /
Q16 records that allocates nothing (its partial states live in a fixed
per-GPU device array): called through the C ABI, its output equals the
allocating entry point's bit for bit (the same kernels and order), and the
oracle's within the FP32 tolerance, on two calls in a row, the second with
a smaller input (fewer rows over a shorter cache), so stale partial states
of the first call cannot leak into the second; with the cache's exact and
fast exp (focr_kv_set_fast_exp). On a fresh context it leaves the context
scratch unallocated, and it captures into a HIP graph with no scratch
reserved (the allocating entry point would be refused there), whose replays
equal the allocating entry point's output."""
import ctypes

import numpy as np
import pytest

import gen
import oracle
from gpu_util import assert_bitwise, host, max_rel, to_dev

pytestmark = pytest.mark.gpu
H, G = 16, 8


def sealed_cache(fh, bits, prefix, tail_rows, seed, ctx=None):
    import torch

    pk = gen.att_values(prefix * H * 64, seed, 0.75).reshape(prefix, H, 64)
    pk[:, 1::2, :32] = pk[:, 0::2, :32]  # paired temporal halves, as the seal requires
    v = gen.att_values(prefix * G * 64, seed + 1, 1.0).reshape(prefix, G, 64)
    kv = fh.KvSplit.seal(bits, to_dev(pk), to_dev(v), prefix, prefix + tail_rows, ctx=ctx)
    k_new = gen.att_values(tail_rows * G * 64, seed + 2, 0.75).reshape(tail_rows, G, 64)
    v_new = gen.att_values(tail_rows * G * 64, seed + 3, 1.0).reshape(tail_rows, G, 64)
    kv.append(to_dev(k_new), to_dev(v_new), tail_rows)
    torch.cuda.synchronize()
    return kv


def call_noalloc(fh, kv, q, rows, sinks, out):
    rc = fh.lib().focr_kv_attention_decode_noalloc(kv.ctx.handle, kv.handle, ctypes.c_void_p(q.data_ptr()), rows,
                                                   ctypes.c_void_p(sinks.data_ptr()), ctypes.c_void_p(out.data_ptr()))
    assert rc == 0, fh.lib().focr_last_error().decode()


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("bits", [8, 16])
def test_noalloc_decode_equals_the_allocating_entry_point(bits, fast):
    import torch

    import focr_hip as fh

    sinks = to_dev(gen.uniform(H, -2.0, 2.0, 7))
    # First call: 8 rows over 16,320 + 64 positions; second: 3 rows over 1,000 + 5.
    for prefix, tail_rows, rows, seed in ((16320, 64, 8, 11), (1000, 5, 3, 21)):
        kv = sealed_cache(fh, bits, prefix, tail_rows, seed).set_fast_exp(fast)
        q = to_dev(gen.att_values(rows * H * 64, seed + 5, 0.75).reshape(rows, H, 64))
        out = torch.full((rows, H, 64), float("nan"), device="cuda:0")
        call_noalloc(fh, kv, q, rows, sinks, out)
        want = kv.attention_decode(q, rows, sinks)
        torch.cuda.synchronize()
        assert_bitwise(host(out), host(want), f"no-alloc vs allocating, {rows} rows over {prefix}+{tail_rows}")
        pk, vals, gk = kv.dequantize()
        total = prefix + tail_rows
        ref = oracle.attention_decode(host(q), host(pk), host(gk), host(vals), rows, prefix, total, H, G,
                                      total - rows, 0, 0, host(sinks), exp_fast=fast)
        got = host(out)
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got - ref) <= 1e-5 * (1.0 + np.abs(ref)))
        assert max_rel(got, ref) <= 1e-5
        kv.free()


def test_noalloc_decode_allocates_nothing_and_captures():
    import torch

    import focr_hip as fh

    ctx = fh.Context(0)
    sinks = to_dev(gen.uniform(H, -2.0, 2.0, 41))
    kv = sealed_cache(fh, 8, 4096, 16, 43, ctx=ctx)
    rows = 5
    q = to_dev(gen.att_values(rows * H * 64, 45, 0.75).reshape(rows, H, 64))
    out = torch.full((rows, H, 64), float("nan"), device="cuda:0")
    call_noalloc(fh, kv, q, rows, sinks, out)
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() == 0, "the no-alloc entry point grew the context scratch"
    first = host(out).copy()

    # Capture with no scratch reserved: only the no-alloc entry point can be recorded.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ctx.use_stream(torch.cuda.current_stream())
            call_noalloc(fh, kv, q, rows, sinks, out)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() == 0
    want = host(kv.attention_decode(q, rows, sinks))  # the allocating entry point, eagerly (grows the scratch)
    torch.cuda.synchronize()
    assert ctx.scratch_bytes() > 0
    assert_bitwise(first, want, "eager no-alloc vs allocating")
    for rep in range(3):
        out.fill_(float("nan"))
        kv.attention_decode(q, rows, sinks)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bitwise(host(out), want, f"replay {rep}")
    del g
    kv.free()
    ctx.close()


def test_noalloc_decode_rejects_bad_arguments():
    import torch

    import focr_hip as fh

    kv = sealed_cache(fh, 8, 64, 2, 31)
    q = torch.zeros((3, H, 64), device="cuda:0")
    sinks = torch.zeros(H, device="cuda:0")
    out = torch.zeros((3, H, 64), device="cuda:0")
    rc = fh.lib().focr_kv_attention_decode_noalloc(kv.ctx.handle, kv.handle, ctypes.c_void_p(q.data_ptr()), 3,
                                                   ctypes.c_void_p(sinks.data_ptr()), ctypes.c_void_p(out.data_ptr()))
    assert rc == -2  # FOCR_E_SHAPE: more rows than appended positions
    assert fh.lib().focr_kv_attention_decode_noalloc(kv.ctx.handle, kv.handle, None, 1, None, None) == -1
    kv.free()
