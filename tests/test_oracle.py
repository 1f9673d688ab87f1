"""Pins the CPU oracle (oracle/focr_oracle.c) before anything is checked against it.

Each test uses something the oracle's own formula cannot supply: a known answer
from the reference's tests (cited), a closed form, an f64 brute force with the
reference's error bound, an invariant the reference asserts, or a hand-derived
input on which a plausible mistake (a wrong pairing in a reduction tree, a
dropped term, a swapped operand) gives a different value.
"""
import math

import numpy as np
import pytest

import gen
import oracle

F32 = np.float32
EPS = float(np.finfo(np.float32).eps)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---- exp_poly (src/kernels/exp.rs:232-277) ---------------------------------
def test_exp_poly_special_values():
    assert oracle.exp_poly(0.0) == 1.0
    assert oracle.exp_poly(-88.0) == 0.0  # below EXP_MIN
    assert oracle.exp_poly(-math.inf) == 0.0
    assert oracle.exp_poly(89.0) == math.inf  # above EXP_MAX
    assert math.isnan(oracle.exp_poly(math.nan))
    assert oracle.exp_poly(1.0) == pytest.approx(math.e, rel=2 ** -22)


def test_exp_poly_is_a_cephes_quality_exp():
    # The published Cephes expf method stays within ~2 ulp of the true exp.
    xs = np.linspace(-87.0, 88.0, 40001, dtype=np.float32)
    worst = 0.0
    for x in xs:
        got = oracle.exp_poly(float(x))
        ref = math.exp(float(x))
        worst = max(worst, abs(got - ref) / ref)
    assert worst < 3 * 2 ** -24


# ---- A1: RTN quantizer and dequant (src/quant/linear/tests.rs:6-16) ---------
def test_rtn_kat_codes_ties_zero_and_signed_endpoints():
    w = np.zeros(128, dtype=np.float32)
    w[:8] = [254.0, -254.0, 1.0, 3.0, 5.0, -1.0, -3.0, -5.0]
    codes, scales = oracle.quantize_bits(w, 1, 128, 64, 8)
    assert scales.ravel().tolist() == [2.0, 0.0]
    assert codes.ravel()[:8].tolist() == [127, -127, 0, 2, 2, 0, -2, -2]
    restored = oracle.dequantize(8, codes, scales, 1, 128, 64)
    assert restored.ravel()[:8].tolist() == [254.0, -254.0, 0.0, 4.0, 4.0, 0.0, -4.0, -4.0]
    assert np.all(restored.ravel()[8:] == 0.0)


@pytest.mark.parametrize("k", [1, 31, 65, 127, 129, 257])
@pytest.mark.parametrize("g", [64, 128])
def test_rtn_partial_groups_error_bound(k, g):
    # src/quant/linear/tests.rs:19-35
    w = ((np.arange(3 * k) * 137 % 127).astype(np.float32) - F32(63.0)) / F32(19.0)
    codes, scales = oracle.quantize_bits(w, 3, k, g, 8)
    restored = oracle.dequantize(8, codes, scales, 3, k, g)
    groups = -(-k // g)
    for row in range(3):
        for col in range(k):
            s = float(scales[row, col // g])
            orig = float(w[row * k + col])
            assert abs(float(restored[row, col]) - orig) <= s / 2 + 2 * EPS * abs(orig)
    assert scales.shape == (3, groups)


def test_dequant_is_one_ieee_multiply_and_exceptions_replace():
    codes = np.array([[127, -127, 5, 0], [1, 2, 3, 4]], dtype=np.int8)
    scales = np.array([[0.1], [3.0e-39]], dtype=np.float32)  # one subnormal scale
    out = oracle.dequantize(8, codes, scales, 2, 4, 64, exc_cols=[3], exc_vals=[7.5, -1.25])
    expected = (codes.astype(np.float32) * scales).astype(np.float32)
    expected[:, 3] = [7.5, -1.25]
    assert np.array_equal(bits(out), bits(expected))


def test_w8_validation_rules():
    # src/quant/linear/integrated_tests.rs:455-460
    assert oracle.validate_w8(1, 1, 64, [-128], [1.0]) != 0
    assert oracle.validate_w8(1, 1, 64, [1], [0.0]) != 0
    assert oracle.validate_w8(1, 1, 64, [0], [math.nan]) != 0
    assert oracle.validate_w8(1, 1, 64, [0], [0.0]) == 0
    assert oracle.validate_w8(1, 1, 64, [5], [0.5]) == 0


# ---- A4/A5: decode dots (src/simd.rs:749-920) ------------------------------
def test_fp32_linear_kat():
    # src/kernels/tests.rs:109-117
    x = np.array([1, 2, 3, 4, 5, 6], dtype=np.float32)
    w = np.array([1, 10, 100, -1, -2, -3], dtype=np.float32)
    out = oracle.linear_decode(32, w, None, 2, 3, 32, x, 2)
    assert out.ravel().tolist() == [321.0, -14.0, 654.0, -32.0]


def _products_dot(products):
    """A dot whose products p_i = x_i * 1.0 are exact: x = p, w = 1."""
    p = np.asarray(products, dtype=np.float32)
    return oracle.dot(p, np.ones_like(p))


def test_dot_phase_combine_pairs_a0_a1_then_a2_a3():
    # (a0 + a1) + (a2 + a3) lane-wise (src/simd.rs:768): phases 0, 8, 16, 24.
    p = np.zeros(32, np.float32)
    p[0], p[8], p[16], p[24] = 2.0 ** 24, 1.0, -(2.0 ** 24), 1.0
    # (2^24 + 1 -> 2^24 ties even) + (-2^24 + 1) = 1. Pairing (a0+a2)+(a1+a3) gives 2.
    assert _products_dot(p) == 1.0


def test_dot_final_tree_order():
    # ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)) (src/simd.rs:260-262).
    p = np.zeros(8, np.float32)  # len 8: no 32-blocks, one 8-wide FMA step from 0
    p[0], p[4], p[1], p[5] = 2.0 ** 24, 1.0, 1.0, 0.0
    # v0+v4 = 2^24 (tie->even), v1+v5 = 1 -> 2^24 + 1 -> 2^24. A sequential sum
    # would also give 2^24, so add a case where it differs:
    assert _products_dot(p) == 2.0 ** 24
    p = np.zeros(8, np.float32)
    p[0], p[4], p[2], p[6], p[1] = 2.0 ** 24, 1.0, 1.0, 1.0, 1.0
    # (v0+v4)=2^24, (v1+v5)=1 -> 2^24; (v2+v6)=2 -> 2^24+2 exactly.
    # Sequential v0+v1+..: 2^24+1->2^24, +1->2^24, +1->2^24, +1 -> 2^24.
    assert _products_dot(p) == 2.0 ** 24 + 2


def test_dot_scalar_tail_is_unfused():
    # total += x * w (two roundings) after the tree (src/simd.rs:772-775).
    x = np.zeros(9, np.float32)
    w = np.zeros(9, np.float32)
    x[8], w[8] = 1.0 + 2.0 ** -12, 1.0 + 2.0 ** -12  # product 1 + 2^-11 + 2^-24
    x[0], w[0] = 1.0, -1.0  # tree total -1
    got = oracle.dot(x, w)
    # unfused: fl(p) = 1 + 2^-11 (tie to even drops 2^-24), -1 + that = 2^-11.
    # fused would keep 2^-11 + 2^-24.
    assert got == 2.0 ** -11


def test_dot_eight_wide_tail_continues_the_combined_lanes():
    # k = 40: one 32-block then one 8-wide FMA step into acc (src/simd.rs:769-771).
    x = np.zeros(40, np.float32)
    x[0], x[32] = 2.0 ** 24, 1.0
    x[8] = 1.0
    w = np.ones(40, np.float32)
    # acc0 = (2^24 + 1) -> 2^24; then fma(1, 1, 2^24) -> 2^24 (tie even).
    assert oracle.dot(x, w) == 2.0 ** 24


def test_dot_q_scale_per_32_block_and_f64_bound():
    k = 2304
    x = gen.values(k, 61)
    codes = ((np.arange(k) * 7919 % 255) - 127).astype(np.int8)
    scales = gen.values(k // 64, 5) * F32(0.01) + F32(0.02)
    got = oracle.dot_q(8, x, codes, scales, 64)
    w = codes.astype(np.float32) * np.repeat(scales, 64)
    exact = float(np.dot(x.astype(np.float64), w.astype(np.float64)))
    mag = float(np.abs(x.astype(np.float64) * w.astype(np.float64)).sum())
    assert abs(got - exact) <= 4 * k * EPS * mag + 1e-6
    # quantized dot == FP32 dot on fl(code*scale) (integrated_tests.rs:116)
    assert bits(got) == bits(oracle.dot(x, w))


@pytest.mark.parametrize("k", [31, 64, 65, 768, 1024, 2304])
def test_linear_decode_f64_bound(k):
    # src/quant/linear/integrated_tests.rs:35-67
    n = 9
    w = ((np.arange(n * k) * 137 % 193).astype(np.float32) - F32(96.0)) / F32(113.0)
    codes, scales = oracle.quantize_bits(w, n, k, 64, 8)
    dense = oracle.dequantize(8, codes, scales, n, k, 64)
    for rows in (1, 2, 4, 8):
        x = ((np.arange(rows * k) * 31 % 151).astype(np.float32) - F32(75.0)) / F32(97.0)
        out = oracle.linear_decode(8, codes, scales, n, k, 64, x, rows)
        xe = x.reshape(rows, k).astype(np.float64)
        exact = xe @ dense.astype(np.float64).T
        mag = np.abs(xe) @ np.abs(dense.astype(np.float64)).T
        assert np.all(np.abs(out - exact) <= 4 * k * EPS * mag + 1e-6)


def test_exception_fmas_follow_the_dot_in_column_order():
    # src/quant/linear.rs:84-118: fma(x_c, v, acc) ascending after the dot.
    k = 64
    x = np.zeros(k, np.float32)
    x[3] = x[10] = x[20] = 1.0
    codes = np.zeros((1, k), np.int8)
    scales = np.ones((1, 1), np.float32)
    vals = np.array([[2.0 ** 24, 1.0, 1.0]], np.float32)
    out = oracle.linear_decode(8, codes, scales, 1, k, 64, x, 1, exc_cols=[3, 10, 20], exc_vals=vals)
    assert out[0, 0] == 2.0 ** 24  # ascending: 2^24, +1 tie, +1 tie; descending gives 2^24 + 2
    vals = np.array([[1.0, 1.0, 2.0 ** 24]], np.float32)
    out = oracle.linear_decode(8, codes, scales, 1, k, 64, x, 1, exc_cols=[3, 10, 20], exc_vals=vals)
    assert out[0, 0] == 2.0 ** 24 + 2
    # fused: x = w = 1 + 2^-12 after acc = -1 keeps the 2^-24 term.
    x[:] = 0.0
    x[3], x[10] = 1.0, F32(1.0 + 2.0 ** -12)
    vals = np.array([[-1.0, F32(1.0 + 2.0 ** -12), 0.0]], np.float32)
    out = oracle.linear_decode(8, codes, scales, 1, k, 64, x, 1, exc_cols=[3, 10, 20], exc_vals=vals)
    assert out[0, 0] == F32(2.0 ** -11 + 2.0 ** -24)


def test_glu_is_gate_of_linear():
    # src/kernels/tests.rs:48-82: fused GLU == linear then squared_relu_gate.
    in_dim, ffn = 65, 19
    w = gen.values(2 * ffn * in_dim, 7)
    w[::97] = np.array([math.nan, 0.0, -0.0, -3.0], np.float32)[np.arange(0, w.size, 97) % 4]
    for rows in (1, 3, 8):
        x = gen.values(rows * in_dim, 11 + rows)
        packed = oracle.linear_decode(32, w, None, 2 * ffn, in_dim, 32, x, rows)
        fused = oracle.linear_decode_glu(32, w, None, 2 * ffn, in_dim, 32, x, rows)
        gate, up = packed[:, 0::2], packed[:, 1::2]
        relu = np.where(gate > 0, gate, F32(0.0))
        expected = (relu * relu) * up
        assert np.array_equal(bits(fused), bits(expected))


def test_squared_relu_glu_branches():
    assert oracle.squared_relu_glu(math.nan, 2.0) == 0.0
    assert bits(oracle.squared_relu_glu(-0.0, 2.0)) == bits(F32(0.0))
    assert oracle.squared_relu_glu(-3.0, 2.0) == 0.0
    assert oracle.squared_relu_glu(3.0, 2.0) == 18.0


# ---- A6: rms_scale (src/kernels/mod.rs:531-553) ----------------------------
def test_rms_scale_closed_form_constant_rows():
    for c in (1.0, 0.5, 3.0):
        row = np.full(768, c, np.float32)
        s2 = F32(c * c)
        expected = F32(1.0) / np.sqrt(F32(F32(768) * s2) / F32(768) + F32(EPS))
        assert bits(oracle.rms_scale(row)) == bits(expected)


def test_rms_tree_leaf_folds_16_8_4_2_1():
    # One 32-leaf: partial[i] += partial[i + w] for w = 16, 8, 4, 2, 1.
    x = np.zeros(32, np.float32)
    x[0] = 4096.0  # square 2^24
    x[16] = 1.0  # pairs with index 0 in the first fold: 2^24 + 1 -> 2^24
    x[1] = 1.0
    x[17] = 1.0  # index 1: 1 + 1 = 2, then folds into index 0: 2^24 + 2
    ssq = (2.0 ** 24 + 2)
    expected = F32(1.0) / np.sqrt(F32(F32(ssq) / F32(32)) + F32(EPS))
    assert bits(oracle.rms_scale(x)) == bits(expected)


def test_rms_tree_split_at_next_multiple_of_32():
    # len 96: middle = (48).next_multiple_of(32) = 64 -> [0,64) + [64,96).
    x = np.zeros(96, np.float32)
    x[0] = 4096.0  # 2^24 in the left half
    x[64] = 1.0  # right half leaf [64, 96): 1
    x[32] = 1.0  # left half second leaf: 1 -> left = 2^24 + 1 -> 2^24
    # left = 2^24, right = 1 -> 2^24 + 1 -> 2^24. A split at 48 would group
    # [0,48) = leaf[0,32) + leaf[32,48) and [48,96) holding x[64] -> same; so
    # also check against a brute-force f64 sum bound.
    s = oracle.rms_scale(x)
    expected = F32(1.0) / np.sqrt(F32(F32(2.0 ** 24) / F32(96)) + F32(EPS))
    assert bits(s) == bits(expected)


def test_rms_scale_f64_bound():
    for width in (768, 1024, 64, 2304):
        h = gen.values(width * 5, 9) * F32(3.0)
        got = oracle.row_scales(h, width)
        for r in range(5):
            row = h[r * width:(r + 1) * width].astype(np.float64)
            exact = 1.0 / math.sqrt(float((row * row).sum()) / width + EPS)
            assert abs(got[r] - exact) <= 8 * EPS * exact


# ---- A2: FP32 panel GEMM (src/kernels/panels/panel.rs:243-299) --------------
@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (13, 768, 48), (9, 7, 16), (20, 300, 32)])
def test_panel_gemm_f64_bound_and_identities(m, k, n):
    a = gen.matrix(m * k, 1)
    w = gen.matrix(n * k, 2)
    out = oracle.panel_gemm(a, m, k, w, n)
    ad, wd = a.reshape(m, k).astype(np.float64), w.reshape(n, k).astype(np.float64)
    exact = ad @ wd.T
    mag = np.abs(ad) @ np.abs(wd).T
    assert np.all(np.abs(out - exact) <= k * EPS * mag + 1e-6)
    gated = oracle.panel_gemm(a, m, k, w, n, epilogue=oracle.GLU)
    g, u = out[:, 0::2], out[:, 1::2]
    relu = np.where(g > 0, g, F32(0))
    assert np.array_equal(bits(gated), bits((relu * relu) * u))
    scale = (F32(0.5) + np.arange(m, dtype=np.float32) / F32(7.0)).astype(np.float32)
    scaled = (a.reshape(m, k) * scale[:, None]).astype(np.float32)
    direct = oracle.panel_gemm(scaled, m, k, w, n)
    folded = oracle.panel_gemm(a, m, k, w, n, row_scale=scale)
    assert np.array_equal(bits(direct), bits(folded))
    base = ((np.arange(m * n) % 17).astype(np.float32) - F32(8.0)).reshape(m, n)
    added = oracle.panel_gemm(a, m, k, w, n, epilogue=oracle.ADD, out=base)
    assert np.array_equal(bits(added), bits(base + out))


def test_panel_gemm_is_one_ascending_fma_chain():
    # k = 3 products 2^24, 1, 1 in order: chain fma(.., 1, 2^24) -> 2^24 twice.
    a = np.array([[2.0 ** 24, 1.0, 1.0]], np.float32)
    w = np.ones((16, 3), np.float32)
    out = oracle.panel_gemm(a, 1, 3, w, 16)
    assert np.all(out == 2.0 ** 24)
    a = np.array([[1.0, 1.0, 2.0 ** 24]], np.float32)
    out = oracle.panel_gemm(a, 1, 3, w, 16)
    assert np.all(out == 2.0 ** 24 + 2)


def test_panel_gemm_thread_independence():
    m, k, n = 37, 256, 64
    a, w = gen.matrix(m * k, 3), gen.matrix(n * k, 4)
    oracle.set_threads(1)
    one = oracle.panel_gemm(a, m, k, w, n)
    oracle.set_threads(4)
    four = oracle.panel_gemm(a, m, k, w, n)
    oracle.set_threads(1)
    assert np.array_equal(bits(one), bits(four))


# ---- A3: INT16 panels (src/kernels/panels/panel_i16/tests.rs) ----------------
def test_i16_quantizer_kat_ties_to_even():
    # panel_i16/tests.rs:372-377
    x = np.zeros(64, np.float32)
    x[0], x[1], x[2], x[3] = 32767.0, 2.5, 3.5, -2.5
    step, q = oracle.i16_quantize_group(x)
    assert step == 1.0
    assert q[:4].tolist() == [32767, 2, 4, -2]


def test_i16_quantizer_rounds_within_the_step():
    # panel_i16/tests.rs:358-371
    for seed in range(64):
        x = gen.noise(np.arange(64, dtype=np.uint64), 10 + seed) * F32(seed + 0.5)
        step, q = oracle.i16_quantize_group(x)
        absmax = F32(np.max(np.abs(x)))
        assert step == absmax / F32(32767.0)
        assert np.any(np.abs(q.astype(np.int32)) == 32767)
        inv = F32(32767.0) / absmax
        for c, v in zip(q, x):
            y = float(F32(v * inv))
            assert c == np.round(y)  # numpy rounds half to even
            assert abs(float(c) * float(step) - float(v)) <= 0.51 * float(step)


@pytest.mark.parametrize("absmax_bits", [None, 8192, 32767, 32768, 1])
def test_i16_quantizer_tiny_groups(absmax_bits):
    # panel_i16/tests.rs:378-413
    for absmax in ([1e-35, 1e-38] if absmax_bits is None else [np.array([absmax_bits], np.uint32).view(np.float32)[0]]):
        absmax = F32(absmax)
        x = (absmax * (F32(2.0) * np.arange(64, dtype=np.float32) / F32(63.0) - F32(1.0))).astype(np.float32)
        assert not np.isfinite(F32(32767.0) / absmax)
        step, q = oracle.i16_quantize_group(x)
        assert step > 0 and np.isfinite(step)
        assert float(step) * 32767.0 >= float(absmax)
        assert float(np.nextafter(step, F32(0))) * 32767.0 < float(absmax)
        assert np.any(q != 0)
        for c, v in zip(q, x):
            assert c == np.clip(np.round(float(v) / float(step)), -32767, 32767)


def test_i16_gemm_within_quantization_bound_of_exact():
    # panel_i16/tests.rs:230-298 bound: sum|w| * 0.51 absmax rs / 32767 + 4 (groups+1) 2^-24 mag
    for (m, k, n) in [(13, 768, 64), (6, 1024, 32)]:
        a = gen.i16_activations(m, k)
        codes, scales = gen.i16_weights(n, k)
        rs = (F32(0.5) + np.arange(m, dtype=np.float32) / F32(7.0)).astype(np.float32)
        got = oracle.i16_gemm(a, m, k, codes, scales, n, row_scale=rs)
        groups = k // 64
        w = codes.astype(np.float64) * np.repeat(scales.astype(np.float64), 64, axis=1)
        x = a.reshape(m, k).astype(np.float64) * rs.astype(np.float64)[:, None]
        exact = x @ w.T
        mag = np.abs(x) @ np.abs(w).T
        absmax = np.abs(a.reshape(m, k, ).reshape(m, groups, 64)).max(axis=2).astype(np.float64)  # [m][g]
        wsum = np.abs(w).reshape(n, groups, 64).sum(axis=2)  # [n][g]
        quant = (absmax * rs.astype(np.float64)[:, None]) @ wsum.T * 0.51 / 32767.0
        bound = quant + 4.0 * (groups + 1) * 2.0 ** -24 * mag + 1e-30
        assert np.all(np.abs(got - exact) <= bound)


def test_i16_gemm_group_sums_are_exact_integers():
    # Integer part against an int64 brute force, then the FP32 group epilogue.
    m, k, n = 5, 256, 32
    a = gen.i16_activations(m, k)
    codes, scales = gen.i16_weights(n, k)
    q, steps, _ = oracle.i16_quantize_rows(a, m, k)
    sums = (q.astype(np.int64).reshape(m, 1, k // 64, 64) * codes.astype(np.int64).reshape(1, n, k // 64, 64)).sum(-1)
    assert np.abs(sums).max() < 2 ** 31
    got = oracle.i16_gemm(a, m, k, codes, scales, n)
    acc = np.zeros((m, n), np.float32)
    for g in range(k // 64):
        s = (scales[None, :, g] * steps[:, None, g]).astype(np.float32)
        prod = sums[:, :, g].astype(np.float32).astype(np.float64) * s.astype(np.float64)
        # fma(f32(sum), s, acc): exact product + acc rounded once; f64 holds
        # the product exactly (24+24 bits) and the sum here without a tie.
        acc = (prod + acc.astype(np.float64)).astype(np.float32)
    assert np.array_equal(bits(got), bits(acc))


def test_i16_nonfinite_and_zero_rows():
    # panel_i16/tests.rs:307-355
    m, k, n = 8, 128, 32
    a = gen.i16_activations(m, k)
    a[5] = np.nan
    a[k + 70] = np.inf
    a[3 * k:4 * k] = 0.0
    for row, mag in enumerate([1e-35, 1e-37, 1e-38, np.array([1], np.uint32).view(np.float32)[0]]):
        a[(row + 4) * k:(row + 5) * k] = mag
    codes, scales = gen.i16_weights(n, k)
    out = oracle.i16_gemm(a, m, k, codes, scales, n)
    assert np.all(np.isnan(out[0])) and np.all(np.isnan(out[1]))
    assert np.all(bits(out[3]) == 0)
    assert np.all(np.isfinite(out[4:8]))
    assert np.any(out[4] != 0)
    assert np.all(out[7] == 0)


# ---- A7: attention (src/kernels/attention/prefill64/tests.rs) ---------------
CASES = [(70, 3, 65), (300, 5, 262), (257, 0, 257), (160, 16, 144), (129, 1, 128), (40, 0, 3), (95, 10, 90)]


def attention_f64(q, k, v, L, n_heads, n_kv, image, sinks):
    """f64 attention with the exact exp (prefill64/test_data.rs:38-81)."""
    q = q.reshape(L, n_heads, 64).astype(np.float64)
    k = k.reshape(L, n_heads, 64).astype(np.float64)
    v = v.reshape(L, n_kv, 64).astype(np.float64)
    out = np.zeros((L, n_heads, 64))
    pos = np.arange(L)
    img = (pos >= image[0]) & (pos < image[1])
    mask = (pos[None, :] > pos[:, None]) & ~(img[:, None] & img[None, :])
    for h in range(n_heads):
        logits = q[:, h] @ k[:, h].T / 8.0
        logits[mask] = -np.inf
        mx = logits.max(axis=1, keepdims=True)
        p = np.exp(logits - mx)
        den = p.sum(axis=1, keepdims=True)
        lse = mx[:, 0] + np.log(den[:, 0])
        sink = 1.0 / (1.0 + np.exp(float(sinks[h]) - lse))
        out[:, h] = (p @ v[:, h // (n_heads // n_kv)]) / den * sink[:, None]
    return out


@pytest.mark.parametrize("L,image_start,image_end", CASES)
def test_attention_close_to_f64(L, image_start, image_end):
    q = gen.att_values(L * 16 * 64, 17 + L, 3.0)
    k = gen.att_values(L * 16 * 64, 19 + L, 3.0)
    v = gen.att_values(L * 8 * 64, 23 + L, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    exact = attention_f64(q, k, v, L, 16, 8, (image_start, image_end), sinks)
    for exp_fast in (True, False):
        got = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, image_start, image_end, sinks, exp_fast=exp_fast)
        assert np.max(np.abs(got - exact) / (1.0 + np.abs(exact))) <= 2e-5


def test_attention_static_matches_online_on_bounded_scores():
    # Static tiles need |score| <= 8 (norm-8 heads): prefill64/test_data.rs:14-34.
    L = 300
    q = gen.normalized(L * 16 * 64, 17 + L)
    k = gen.normalized(L * 16 * 64, 19 + L)
    v = gen.values(L * 8 * 64, 23 + L, 3.0)
    sinks = gen.values(16, 29, 2.0)
    online = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, 5, 262, sinks)
    static = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, 5, 262, sinks, static=True)
    exact = attention_f64(q, k, v, L, 16, 8, (5, 262), sinks)
    assert np.max(np.abs(static - exact)) <= 2e-5 * max(1.0, np.max(np.abs(exact)))
    assert np.max(np.abs(online - exact)) <= 2e-5 * max(1.0, np.max(np.abs(exact)))


def test_attention_generated_keys_equal_expanded_prefix():
    # A compact cache with generated keys equals the expanded cache whose
    # prefix rows repeat the KV head (CompactKv, attention/mod.rs:78-151).
    prefix, total, L, off = 100, 133, 33, 100
    q = gen.att_values(L * 16 * 64, 71, 3.0)
    pk = gen.att_values(prefix * 16 * 64, 83, 3.0)
    gk = gen.att_values((total - prefix) * 8 * 64, 37, 3.0)
    v = gen.att_values(total * 8 * 64, 117, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    compact = oracle.attention_prefill(q, pk, v, L, prefix, total, 16, 8, off, 1, 90, sinks, generated_k=gk)
    expanded_k = np.concatenate([pk.reshape(prefix, 16, 64), np.repeat(gk.reshape(total - prefix, 8, 64), 2, axis=1)])
    expanded = oracle.attention_prefill(q, expanded_k, v, L, total, total, 16, 8, off, 1, 90, sinks)
    assert np.array_equal(bits(compact), bits(expanded))


# ---- A9: argmax (src/runner/mod.rs:946-949) ---------------------------------
def test_argmax_kat():
    assert oracle.argmax([2.0, 3.0, 3.0]) == 1
    with pytest.raises(ValueError):
        oracle.argmax([math.nan])
    with pytest.raises(ValueError):
        oracle.argmax([1.0, math.inf, 0.0])
