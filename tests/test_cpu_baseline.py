"""The CPU baseline's performance restatements are bit for bit the oracle:
the FP32 panel GEMM (oracle/focr_cpu_panels.c: the reference's AVX2 6x16
FMA micro-kernel) for every epilogue, row scale and ragged shape (rows not a
multiple of 6, columns not a multiple of 16); the prefill attention tiles;
the INT16-activation x INT8-code GEMM on the reference's AVX-512 VNNI panels
(oracle/focr_cpu_panels_i16.c) with exception columns, tiny and non-finite
groups; the AVX2 decode GEMV and decode attention (oracle/focr_cpu_gemv.c)
with 8-, 16- and 32-bit weights, tails and exceptions."""
import numpy as np
import pytest

import gen
import oracle


@pytest.mark.parametrize("m,k,n", [(1, 7, 16), (7, 33, 34), (97, 128, 48), (200, 96, 130), (6, 768, 64)])
@pytest.mark.parametrize("epilogue", [oracle.STORE, oracle.GLU, oracle.ADD])
def test_fast_panels_are_bitwise_the_oracle(m, k, n, epilogue):
    oracle.set_threads(4)
    a = gen.values(m * k, 3 + m, 2.0).reshape(m, k)
    w = gen.matrix(n * k, 4 + n).reshape(n, k)
    rs = gen.uniform(m, 0.5, 1.5, 5) if m % 2 else None
    base = gen.values(m * n, 6, 1.0).reshape(m, n) if epilogue == oracle.ADD else None
    want = oracle.panel_gemm(a, m, k, w, n, rs, epilogue, out=base)
    got = oracle.panel_gemm_fast(a, m, k, w, n, rs, epilogue, out=base)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("L,image", [(70, (3, 65)), (300, (5, 262)), (161, (0, 0)), (600, (0, 300)), (40, (0, 3))])
@pytest.mark.parametrize("static", [False, True])
def test_fast_attention_is_bitwise_the_oracle(L, image, static):
    oracle.set_threads(4)
    q = (gen.normalized if static else lambda n, s: gen.att_values(n, s, 3.0))(L * 16 * 64, 7 + L)
    k = (gen.normalized if static else lambda n, s: gen.att_values(n, s, 3.0))(L * 16 * 64, 8 + L)
    v = gen.att_values(L * 8 * 64, 9 + L, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, *image, sinks, static=static, exp_fast=True)
    got = oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, *image, sinks, static=static)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fast_attention_with_generated_keys():
    oracle.set_threads(4)
    L, prefix, total, offset = 33, 100, 133, 100
    q = gen.att_values(L * 16 * 64, 71, 3.0)
    pk = gen.att_values(prefix * 16 * 64, 83, 3.0)
    gk = gen.att_values((total - prefix) * 8 * 64, 37, 3.0)
    v = gen.att_values(total * 8 * 64, 117, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    want = oracle.attention_prefill(q, pk, v, L, prefix, total, 16, 8, offset, 1, 90, sinks, generated_k=gk)
    got = oracle.attention_prefill_fast(q, pk, v, L, prefix, total, 16, 8, offset, 1, 90, sinks, generated_k=gk)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _vnni():
    return {"avx512f", "avx512_vnni"} <= oracle.cpu_flags()


@pytest.mark.parametrize("m,k,n", [(1, 64, 32), (7, 768, 64), (97, 1024, 96), (200, 2304, 32), (13, 128, 4608)])
@pytest.mark.parametrize("epilogue", [oracle.STORE, oracle.GLU, oracle.ADD])
def test_vnni_panels_are_bitwise_the_oracle(m, k, n, epilogue):
    if not _vnni():
        pytest.skip("host CPU without AVX-512 VNNI")
    oracle.set_threads(4)
    a = gen.values(m * k, 11 + m, 2.0).reshape(m, k)
    codes = gen.codes_uniform((n, k), -127, 127, np.int8, 12 + n)
    scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 13)
    cols = sorted({0, k // 3, k - 1})
    vals = gen.values(n * len(cols), 14, 0.5).reshape(n, len(cols))
    codes[:, cols] = 0
    if m > 2:
        a[1, :64] = 1e-40  # a tiny group: the f64 path and its rounded-up step
        a[2, 70 % k] = np.inf  # a non-finite group: NaN outputs for the row
    rs = gen.uniform(m, 0.5, 1.5, 15) if m % 2 else None
    base = gen.values(m * n, 16, 1.0).reshape(m, n) if epilogue == oracle.ADD else None
    want = oracle.i16_gemm(a, m, k, codes, scales, n, rs, epilogue, cols, vals, out=base)
    panels = oracle.I16Panels(codes, scales, n, k, cols, vals)
    got = panels.gemm(a, m, rs, epilogue, out=base)
    panels.free()
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_vnni_panels_reject_shapes_the_reference_rejects():
    with pytest.raises(ValueError):
        oracle.I16Panels(np.zeros((48, 64), np.int8), np.ones((48, 1), np.float32), 48, 64)
    with pytest.raises(ValueError):
        oracle.I16Panels(np.zeros((32, 100), np.int8), np.ones((32, 2), np.float32), 32, 100)


@pytest.mark.parametrize("bits", [8, 16, 32])
@pytest.mark.parametrize("n,k,rows,group", [(96, 1024, 1, 64), (40, 1000, 3, 32), (24, 77, 5, 64), (8, 4100, 2, 64)])
def test_fast_gemv_is_bitwise_the_oracle(bits, n, k, rows, group):
    oracle.set_threads(4)
    if bits == 32:
        codes, scales, ex = gen.values(n * k, 21, 0.1).reshape(n, k), None, (None, None)
    else:
        lo, hi, dt = (-127, 127, np.int8) if bits == 8 else (-32768, 32767, np.int16)
        codes = gen.codes_uniform((n, k), lo, hi, dt, 22)
        scales = gen.uniform((n, (k + group - 1) // group), 1e-4, 4e-4, 23)
        cols = [1, k // 2]
        codes[:, cols] = 0
        ex = (cols, gen.values(n * 2, 24, 0.5).reshape(n, 2))
    x = gen.values(rows * k, 25, 2.0).reshape(rows, k)
    for fn in (oracle.linear_decode, oracle.linear_decode_glu):
        want = fn(bits, codes, scales, n, k, group, x, rows, *ex)
        got = fn(bits, codes, scales, n, k, group, x, rows, *ex, fast=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), fn.__name__


@pytest.mark.parametrize("prefix,generated,rows,image", [(700, 9, 3, (0, 512)), (100, 0, 2, (10, 60)),
                                                           (64, 64, 8, (0, 0)), (1000, 5, 1, (0, 1000))])
def test_fast_decode_attention_is_bitwise_the_oracle(prefix, generated, rows, image):
    oracle.set_threads(4)
    heads, kv = 16, 8
    q = gen.att_values(rows * heads * 64, 31, 3.0).reshape(rows, heads, 64)
    pk = gen.att_values(prefix * heads * 64, 32, 3.0).reshape(prefix, heads, 64)
    gk = gen.att_values(max(generated, 1) * kv * 64, 33, 3.0).reshape(-1, kv, 64)
    v = gen.att_values((prefix + generated) * kv * 64, 34, 3.0).reshape(-1, kv, 64)
    sinks = gen.att_values(heads, 35, 2.0)
    total = prefix + generated
    args = (q, pk, gk, v, rows, prefix, total, heads, kv, total - rows, *image, sinks)
    want = oracle.attention_decode(*args)
    got = oracle.attention_decode(*args, fast=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
