"""Decode/verify GEMV and dequantization on the GPU against the oracle, bitwise
(src/quant/linear/integrated_tests.rs, src/kernels/tests.rs)."""
import math

import numpy as np
import pytest

import gen
import oracle
from gpu_util import F32, assert_bitwise, host, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def quantized(bits, n, k, group, seed, exc=None):
    """Matrix codes as quantize_bits makes them, with exception columns zeroed."""
    w = ((np.arange(n * k) * 7919 % 2003).astype(np.float32) - F32(1001.0)) / F32(977.0)
    w = (w * (gen.values(n * k, seed) + F32(1.5))).astype(np.float32).reshape(n, k)
    vals = None
    if exc:
        vals = w[:, exc].copy() * F32(300.0)
        w[:, exc] = 0.0
    codes, scales = oracle.quantize_bits(w, n, k, group, bits)
    return codes, scales, vals


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("k,group", [(768, 64), (1024, 64), (2304, 64), (65, 64), (31, 32), (100, 32), (768, 128), (520, 64)])
def test_decode_is_bitwise_the_reference_dot(fh, bits, k, group):
    n = 37
    codes, scales, _ = quantized(bits, n, k, group, 3)
    lin = fh.QuantLinear(bits, codes, scales, group)
    for rows in range(1, 9):
        x = ((np.arange(rows * k) * 104729 % 1009).astype(np.float32) - F32(504.0)) / F32(311.0)
        got = host(lin.linear(to_dev(x), rows))
        want = oracle.linear_decode(bits, codes, scales, n, k, group, x, rows)
        assert_bitwise(got, want, f"bits {bits} k {k} g {group} rows {rows}")


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("n,k,group,columns", [(37, 768, 64, [0]), (5, 1024, 64, [3, 511, 1023]),
                                              (3, 2304, 64, [17, 18, 1500, 2303]), (4, 65, 64, [64]),
                                              (2, 31, 32, [0, 30]), (37, 768, 32, [100, 700])])
def test_decode_exception_columns_in_ascending_order(fh, bits, n, k, group, columns):
    # integrated_tests.rs:195-252
    codes, scales, vals = quantized(bits, n, k, group, 5, exc=columns)
    lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=columns, exc_vals=vals)
    for rows in (1, 3, 8):
        x = ((np.arange(rows * k) * 104729 % 1009).astype(np.float32) - F32(504.0)) / F32(311.0)
        got = host(lin.linear(to_dev(x), rows))
        want = oracle.linear_decode(bits, codes, scales, n, k, group, x, rows, exc_cols=columns, exc_vals=vals)
        assert_bitwise(got, want, f"exceptions bits {bits} rows {rows}")


@pytest.mark.parametrize("bits", [8, 16, 32])
def test_decode_nonfinite_activations(fh, bits):
    # NaN and infinities in the activations travel as the reference's dot
    # makes them (QuantLinear::linear takes them; only the scalar reference
    # linear_f32 refuses them, linear.rs:289-291): bitwise, NaN by class,
    # infinities by sign, through the plain and the GLU GEMVs, an exception
    # column and zero weights included.
    n, k, group = 38, 768, 64
    columns = [5, 700]
    if bits == 32:
        w = gen.values(n * k, 41).reshape(n, k)
        w[3, ::5] = 0.0
        lin, args, kw = fh.Linear.from_f32(w), (32, w, None, n, k, 32), {}
    else:
        codes, scales, vals = quantized(bits, n, k, group, 43, exc=columns)
        lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=columns, exc_vals=vals)
        args, kw = (bits, codes, scales, n, k, group), dict(exc_cols=columns, exc_vals=vals)
    for rows in (1, 5, 8):
        x = gen.values(rows * k, 47 + rows).reshape(rows, k)
        x[0, 100] = np.nan
        if rows > 1:
            x[1, 5] = np.inf  # an exception column for the codes
            x[2, 300] = -np.inf
            x[3, 7], x[3, 9] = np.inf, -np.inf
            x[4, 700] = np.nan
        x = x.ravel()
        got = host(lin.linear(to_dev(x), rows))
        want = oracle.linear_decode(*args, x, rows, **kw)
        assert not np.all(np.isfinite(want))
        assert_bitwise(got, want, f"bits {bits} rows {rows}")
        assert np.array_equal(np.isinf(got) & (got > 0), np.isinf(want) & (want > 0))
        glu = host(lin.linear_glu(to_dev(x), rows))
        assert_bitwise(glu, oracle.linear_decode_glu(*args, x, rows, **kw), f"glu bits {bits} rows {rows}")


@pytest.mark.parametrize("in_dim,ffn", [(768, 2304), (65, 19), (1, 1), (1024, 64)])
def test_fp32_decode_and_glu(fh, in_dim, ffn):
    # src/kernels/tests.rs:48-82 (NaN, signed zeros, negatives in the weights)
    w = gen.values(2 * ffn * in_dim, 7)
    idx = np.arange(0, w.size, 97)
    w[idx] = np.array([math.nan, 0.0, -0.0, -3.0], np.float32)[idx % 4]
    w = w.reshape(2 * ffn, in_dim)
    lin = fh.Linear.from_f32(w)
    for rows in range(1, 9):
        x = gen.values(rows * in_dim, 11 + rows)
        packed = host(lin.linear(to_dev(x), rows))
        assert_bitwise(packed, oracle.linear_decode(32, w, None, 2 * ffn, in_dim, 32, x, rows), f"fp32 rows {rows}")
        fused = host(lin.linear_glu(to_dev(x), rows))
        assert_bitwise(fused, oracle.linear_decode_glu(32, w, None, 2 * ffn, in_dim, 32, x, rows), f"glu rows {rows}")


def test_fp32_linear_kat(fh):
    # src/kernels/tests.rs:109-117
    lin = fh.Linear.from_f32(np.array([[1, 10, 100], [-1, -2, -3]], np.float32))
    out = host(lin.linear(to_dev(np.array([1, 2, 3, 4, 5, 6], np.float32)), 2))
    assert out.ravel().tolist() == [321.0, -14.0, 654.0, -32.0]


@pytest.mark.parametrize("bits", [8, 16])
def test_quantized_glu(fh, bits):
    n, k = 2 * 96, 768
    codes, scales, vals = quantized(bits, n, k, 64, 9, exc=[5, 700])
    lin = fh.QuantLinear(bits, codes, scales, 64, exc_cols=[5, 700], exc_vals=vals)
    for rows in (1, 5, 8):
        x = gen.values(rows * k, 13 + rows) * F32(2.0)
        got = host(lin.linear_glu(to_dev(x), rows))
        want = oracle.linear_decode_glu(bits, codes, scales, n, k, 64, x, rows, exc_cols=[5, 700], exc_vals=vals)
        assert_bitwise(got, want, f"glu bits {bits} rows {rows}")


@pytest.mark.parametrize("rows", [1, 5])
def test_config2_int16_gemv_full_size(fh, rows):
    # W[4096 x 1024] int16 over [-32768, 32767], scales U(1e-6, 4e-6).
    n, k = 4096, 1024
    codes = gen.codes_uniform((n, k), -32768, 32767, np.int16, 1)
    scales = gen.uniform((n, k // 64), 1e-6, 4e-6, 2)
    x = gen.normal((rows, k), 1.0, 3)
    lin = fh.QuantLinear(16, codes, scales, 64)
    got = host(lin.linear(to_dev(x), rows))
    assert_bitwise(got, oracle.linear_decode(16, codes, scales, n, k, 64, x, rows), f"config 2 rows {rows}")


def test_config3_int8_gemv_full_size(fh):
    n, k = 4096, 1024
    codes = gen.codes_uniform((n, k), -127, 127, np.int8, 4)
    scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 5)
    x = gen.normal((1, k), 1.0, 6)
    lin = fh.QuantLinear(8, codes, scales, 64)
    got = host(lin.linear(to_dev(x), 1))
    assert_bitwise(got, oracle.linear_decode(8, codes, scales, n, k, 64, x, 1), "config 3 GEMV")


@pytest.mark.parametrize("bits,group", [(8, 64), (16, 64), (8, 32), (16, 128)])
@pytest.mark.parametrize("k", [300, 301])  # four weights per thread; element by element (k % 4 != 0)
def test_dequantize_is_bit_exact(fh, bits, group, k):
    n = 48
    exc = [0, 299]
    codes, scales, vals = quantized(bits, n, k, group, 11, exc=exc)
    scales = scales.copy()
    scales[0, 0] = np.float32(3e-39)  # subnormal scale
    lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=exc, exc_vals=vals)
    got = host(lin.dequantize())
    assert_bitwise(got, oracle.dequantize(bits, codes, scales, n, k, group, exc, vals), "dequant")


def test_w8_validation(fh):
    # src/quant/linear/integrated_tests.rs:455-460
    with pytest.raises(fh.FocrError, match="-128"):
        fh.QuantLinear.from_parts(1, 1, 64, np.array([-128], np.int8), [1.0])
    with pytest.raises(fh.FocrError):
        fh.QuantLinear.from_parts(1, 1, 64, np.array([1], np.int8), [0.0])
    with pytest.raises(fh.FocrError):
        fh.QuantLinear.from_parts(1, 1, 64, np.array([0], np.int8), [math.nan])
    with pytest.raises(fh.FocrError, match="sorted"):
        fh.QuantLinear(8, np.zeros((2, 64), np.int8), np.ones((2, 1), np.float32), 64, exc_cols=[5, 3],
                       exc_vals=np.zeros((2, 2), np.float32))
    with pytest.raises(fh.FocrError, match="nonzero code"):
        fh.QuantLinear(8, np.ones((2, 64), np.int8), np.ones((2, 1), np.float32), 64, exc_cols=[3],
                       exc_vals=np.zeros((2, 1), np.float32))


def test_shape_errors(fh):
    import torch

    lin = fh.QuantLinear(8, np.ones((32, 64), np.int8), np.ones((32, 1), np.float32), 64)
    x = torch.zeros(9 * 64, device="cuda:0")
    with pytest.raises(fh.FocrError):
        lin.linear(x, 9)  # decode takes 1..=8 rows
    odd = fh.QuantLinear(8, np.ones((3, 64), np.int8), np.ones((3, 1), np.float32), 64)
    with pytest.raises(fh.FocrError, match="GLU"):
        odd.linear_glu(torch.zeros(64, device="cuda:0"), 1)


@pytest.mark.parametrize("bits,n,k,group", [(8, 16384, 1024, 64), (8, 65536, 768, 64), (16, 16387, 520, 64),
                                            (8, 16386, 256, 32), (16, 20000, 100, 32)])
def test_large_matrices_several_tiles_per_wave(fh, bits, n, k, group):
    # From 4,096 wave tiles (16,384 channels) each wave computes several tiles
    # (1 or 2 rows); ragged last workgroups, every epilogue and exception
    # columns stay bitwise the reference's dot.
    codes = gen.codes_uniform((n, k), -127 if bits == 8 else -32768, 127 if bits == 8 else 32767,
                              np.int8 if bits == 8 else np.int16, 90)
    scales = gen.uniform((n, -(-k // group)), 1e-4, 4e-4, 91)
    cols = [3, k - 1]
    codes[:, cols] = 0
    vals = gen.normal((n, 2), 0.1, 92)
    lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=cols, exc_vals=vals)
    for rows in (1, 2, 3):
        x = gen.normal((rows, k), 1.0, 93 + rows)
        want = oracle.linear_decode(bits, codes, scales, n, k, group, x, rows, exc_cols=cols, exc_vals=vals)
        assert_bitwise(host(lin.linear(to_dev(x), rows)), want, f"large {n}x{k} rows {rows}")
        if n % 2 == 0:
            glu = oracle.linear_decode_glu(bits, codes, scales, n, k, group, x, rows, exc_cols=cols, exc_vals=vals)
            assert_bitwise(host(lin.linear_glu(to_dev(x), rows)), glu, f"large glu rows {rows}")
        base = gen.normal((rows, n), 1.0, 97)
        h = to_dev(base)
        lin.linear_ex(to_dev(x), rows, epilogue=fh.Epilogue.ADD, out=h)
        assert_bitwise(host(h), (base + want).astype(np.float32), f"large add rows {rows}")
    lin.free()


@pytest.mark.parametrize("bits,k", [(8, 6144), (16, 3072), (32, 2560), (8, 5160), (16, 2600)])
def test_long_rows_refill_the_weight_window(fh, bits, k):
    # Rows longer than the register window (more than 20 steps of 16-byte
    # chunks, 36 for FP32 weights) stage x directly and refill the weight
    # window as it is consumed: still bitwise the reference's dot, with the
    # 8-wide and scalar tails (k % 32 != 0) and an exception column.
    n, group = 70, 64
    if bits == 32:
        w = gen.normal((n, k), 0.02, 120)
        lin = fh.Linear.from_f32(w)
        x = gen.normal((2, k), 1.0, 121)
        for rows in (1, 2):
            want = oracle.linear_decode(32, w, None, n, k, 32, x[:rows], rows)
            assert_bitwise(host(lin.linear(to_dev(x[:rows]), rows)), want, f"fp32 k {k} rows {rows}")
        lin.free()
        return
    codes, scales, vals = quantized(bits, n, k, group, 122, exc=[k - 3])
    x = gen.normal((2, k), 1.0, 123)
    lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=[k - 3], exc_vals=vals)
    for rows in (1, 2):
        want = oracle.linear_decode(bits, codes, scales, n, k, group, x[:rows], rows, exc_cols=[k - 3], exc_vals=vals)
        assert_bitwise(host(lin.linear(to_dev(x[:rows]), rows)), want, f"bits {bits} k {k} rows {rows}")
    lin.free()


@pytest.mark.parametrize("bits", [8, 16])
def test_subnormal_scales_and_activations(fh, bits):
    # Rows of subnormal or tiny values quantize to subnormal group scales
    # (quantize_bits floors a nonzero scale at the least subnormal,
    # linear.rs:140-201) and a zero group to a zero scale: the dequantized
    # weights, the decode GEMVs (plain and GLU, with subnormal activations)
    # and the prefill projections on the codes (the exact-order chain; for
    # 8-bit codes the INT16-activation panels) are bitwise the reference's.
    n, k, group = 64, 768, 64
    w = gen.values(n * k, 51).reshape(n, k)
    w[3] *= np.float32(1e-40)
    w[4, :64] = 0.0
    w[5, 64:128] *= np.float32(1e-38)
    w[6] *= np.float32(2.0 ** -140)
    codes, scales = oracle.quantize_bits(w, n, k, group, bits)
    sc = np.asarray(scales)
    assert np.any((sc > 0) & (sc < 2.0 ** -126)) and np.any(sc == 0)
    lin = fh.QuantLinear(bits, codes, scales, group)
    dense = oracle.dequantize(bits, codes, scales, n, k, group)
    assert_bitwise(host(lin.dequantize()), dense, "dequant")
    for rows in (1, 5, 8):
        x = gen.values(rows * k, 53 + rows)
        x[::7] *= np.float32(1e-39)
        assert_bitwise(host(lin.linear(to_dev(x), rows)), oracle.linear_decode(bits, codes, scales, n, k, group, x, rows),
                       f"decode rows {rows}")
        assert_bitwise(host(lin.linear_glu(to_dev(x), rows)),
                       oracle.linear_decode_glu(bits, codes, scales, n, k, group, x, rows), f"glu rows {rows}")
    m = 37
    a = gen.normal((m, k), 1.0, 57)
    a[3] *= np.float32(1e-39)
    a[9, ::5] = np.float32(2.0 ** -149)
    got = host(lin.prefill(to_dev(a), m, kernel=fh.PrefillProjection.F32_CHAIN))
    assert_bitwise(got, oracle.panel_gemm(a, m, k, dense, n), "chain on codes")
    if bits == 8:
        got = host(lin.prefill(to_dev(a), m, kernel=fh.PrefillProjection.I16))
        assert_bitwise(got, oracle.i16_gemm(a, m, k, codes, scales, n), "INT16 panels")
