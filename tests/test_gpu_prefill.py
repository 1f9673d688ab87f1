"""Prefill projections on the GPU against the oracle:
INT16 panels bitwise (src/kernels/panels/panel_i16/tests.rs), FP32 exact-order
panels bitwise, and FP32 matrix cores and FP32 products from power-of-two
scaled FP16 pairs within the FP32 tolerance (src/kernels/panels/panel.rs:243-299)."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import EPS, F32, assert_bitwise, host, max_rel, oracle_threads, to_dev

pytestmark = pytest.mark.gpu

I16_SHAPES = [(1, 64, 32), (13, 768, 64), (97, 1024, 32), (50, 2304, 64), (7, 128, 96), (200, 768, 160), (130, 256, 416)]


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def run_prefill(fh, lin, a, m, rs, epi, kernel, base=None):
    out = None if base is None else to_dev(base)
    got = lin.prefill(to_dev(a), m, row_scale=None if rs is None else to_dev(rs), epilogue=epi, out=out, kernel=kernel)
    return host(got)


@pytest.mark.parametrize("m,k,n", I16_SHAPES)
def test_i16_panels_bitwise_every_epilogue(fh, m, k, n):
    a = gen.i16_activations(m, k)
    codes, scales = gen.i16_weights(n, k)
    rs = (F32(0.25) + np.arange(m, dtype=np.float32) / F32(9.0)).astype(np.float32)
    base = ((np.arange(m * n) % 13).astype(np.float32) - F32(6.0)).reshape(m, n)
    lin = fh.QuantLinear(8, codes, scales, 64)
    I16 = fh.PrefillProjection.I16
    assert_bitwise(run_prefill(fh, lin, a, m, rs, fh.Epilogue.STORE, I16),
                   oracle.i16_gemm(a, m, k, codes, scales, n, row_scale=rs), "store")
    assert_bitwise(run_prefill(fh, lin, a, m, None, fh.Epilogue.GLU, I16),
                   oracle.i16_gemm(a, m, k, codes, scales, n, epilogue=oracle.GLU), "glu")
    assert_bitwise(run_prefill(fh, lin, a, m, rs, fh.Epilogue.ADD, I16, base=base),
                   oracle.i16_gemm(a, m, k, codes, scales, n, row_scale=rs, epilogue=oracle.ADD, out=base), "add")


@pytest.mark.parametrize("m,k,n", [(13, 768, 64), (50, 2304, 64), (97, 1024, 32)])
def test_i16_exception_columns(fh, m, k, n):
    # panel_i16/tests.rs:156-227: two pairs share a group; huge inputs there.
    columns = [0, 1, k // 2, k // 2 + 1, k - 1]
    vals = (gen.noise(np.arange(n * len(columns), dtype=np.uint64), 4) * F32(0.1)).reshape(n, len(columns))
    a = gen.i16_activations(m, k).reshape(m, k)
    codes, scales = gen.i16_weights(n, k)
    codes = codes.copy()
    codes[:, columns] = 0
    for c in columns:
        a[:, c] = F32(100000.0) * (F32(1.0) + gen.noise(np.array([c], np.uint64), 5)[0])
    rs = (F32(0.25) + np.arange(m, dtype=np.float32) / F32(9.0)).astype(np.float32)
    lin = fh.QuantLinear(8, codes, scales, 64, exc_cols=columns, exc_vals=vals)
    I16 = fh.PrefillProjection.I16
    for epi, o_epi, r in ((fh.Epilogue.STORE, oracle.STORE, rs), (fh.Epilogue.GLU, oracle.GLU, None)):
        got = run_prefill(fh, lin, a, m, r, epi, I16)
        want = oracle.i16_gemm(a, m, k, codes, scales, n, row_scale=r, epilogue=o_epi, exc_cols=columns, exc_vals=vals)
        assert_bitwise(got, want, f"exceptions {epi.name}")


def test_i16_nonfinite_zero_and_tiny_rows(fh):
    # panel_i16/tests.rs:307-355
    m, k, n = 8, 128, 32
    a = gen.i16_activations(m, k)
    a[5] = np.nan
    a[k + 70] = np.inf
    a[3 * k:4 * k] = 0.0
    for row, mag in enumerate([1e-35, 1e-37, 1e-38, np.array([1], np.uint32).view(np.float32)[0]]):
        a[(row + 4) * k:(row + 5) * k] = mag
    codes, scales = gen.i16_weights(n, k)
    lin = fh.QuantLinear(8, codes, scales, 64)
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.I16)
    want = oracle.i16_gemm(a, m, k, codes, scales, n)
    assert_bitwise(got, want, "edge rows")
    assert np.all(np.isnan(got[0])) and np.all(got[3].view(np.uint32) == 0) and np.all(got[7] == 0)
    tiny = a[4 * k:]
    rs = np.array([1.0, 2.0, 1024.0, 1e6], np.float32)
    got = run_prefill(fh, lin, tiny, 4, rs, fh.Epilogue.STORE, fh.PrefillProjection.I16)
    assert_bitwise(got, oracle.i16_gemm(tiny, 4, k, codes, scales, n, row_scale=rs), "tiny rows scaled")


def test_i16_rejects_matrices_the_panels_cannot_hold(fh):
    import torch

    lin = fh.QuantLinear(16, np.zeros((32, 64), np.int16), np.ones((32, 1), np.float32), 64)
    with pytest.raises(fh.FocrError, match="fits_i16_panels"):
        lin.prefill(torch.zeros(9 * 64, device="cuda:0"), 9, kernel=fh.PrefillProjection.I16)


def test_config3_int8_prefill_full_size(fh):
    # BASELINE config 3 (literal shape): X[6544 x 1024] ~ N(0,1), W 4096 x 1024 int8, scales U(1e-4, 4e-4).
    m, k, n = 6544, 1024, 4096
    a = gen.normal((m, k), 1.0, 7)
    codes = gen.codes_uniform((n, k), -127, 127, np.int8, 8)
    scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 9)
    lin = fh.QuantLinear(8, codes, scales, 64)
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.I16)
    # Every output bitwise.
    oracle.set_threads(oracle_threads())
    assert_bitwise(got, oracle.i16_gemm(a, m, k, codes, scales, n), "config 3")
    assert np.all(np.isfinite(got))


F32_SHAPES = [(1, 64, 16), (13, 768, 48), (97, 1024, 32), (200, 2304, 64), (9, 7, 16), (130, 300, 160), (300, 192, 200)]


@pytest.mark.parametrize("bits", [32, 16, 8])
@pytest.mark.parametrize("m,k,n", F32_SHAPES)
def test_f32_chain_is_bitwise_the_panels(fh, bits, m, k, n):
    a = gen.matrix(m * k, 1).reshape(m, k)
    w = gen.matrix(n * k, 2).reshape(n, k)
    if bits == 32:
        lin, dense = fh.Linear.from_f32(w), w
    else:
        codes, scales = oracle.quantize_bits(w, n, k, 64, bits)
        lin = fh.QuantLinear(bits, codes, scales, 64)
        dense = oracle.dequantize(bits, codes, scales, n, k, 64)
    rs = (F32(0.5) + np.arange(m, dtype=np.float32) / F32(7.0)).astype(np.float32)
    base = ((np.arange(m * n) % 17).astype(np.float32) - F32(8.0)).reshape(m, n)
    CH = fh.PrefillProjection.F32_CHAIN
    assert_bitwise(run_prefill(fh, lin, a, m, rs, fh.Epilogue.STORE, CH), oracle.panel_gemm(a, m, k, dense, n, row_scale=rs), "store")
    assert_bitwise(run_prefill(fh, lin, a, m, None, fh.Epilogue.GLU, CH),
                   oracle.panel_gemm(a, m, k, dense, n, epilogue=oracle.GLU), "glu")
    assert_bitwise(run_prefill(fh, lin, a, m, None, fh.Epilogue.ADD, CH, base=base),
                   oracle.panel_gemm(a, m, k, dense, n, epilogue=oracle.ADD, out=base), "add")


@pytest.mark.parametrize("bits", [32, 16, 8])
@pytest.mark.parametrize("m,k,n", F32_SHAPES)
def test_f32_mfma_within_fp32_tolerance(fh, bits, m, k, n):
    a = gen.matrix(m * k, 3).reshape(m, k)
    w = gen.matrix(n * k, 4).reshape(n, k)
    if bits == 32:
        lin, dense = fh.Linear.from_f32(w), w
    else:
        codes, scales = oracle.quantize_bits(w, n, k, 64, bits)
        lin = fh.QuantLinear(bits, codes, scales, 64)
        dense = oracle.dequantize(bits, codes, scales, n, k, 64)
    rs = (F32(0.5) + np.arange(m, dtype=np.float32) / F32(7.0)).astype(np.float32)
    got = run_prefill(fh, lin, a, m, rs, fh.Epilogue.STORE, fh.PrefillProjection.F32_MFMA)
    want = oracle.panel_gemm(a, m, k, dense, n, row_scale=rs)
    ad = (a * rs[:, None]).astype(np.float32).astype(np.float64)
    mag = np.abs(ad) @ np.abs(dense.astype(np.float64)).T
    # Both orders are within (k-1) eps sum|a w| of the exact product.
    assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30)
    assert max_rel(got, want) <= 1e-5
    glu = run_prefill(fh, lin, a, m, rs, fh.Epilogue.GLU, fh.PrefillProjection.F32_MFMA)
    g, u = got[:, 0::2], got[:, 1::2]
    assert_bitwise(glu, (np.where(g > 0, g, F32(0)) ** 2 * u).astype(np.float32), "glu of store")


@pytest.mark.parametrize("m,k,n", F32_SHAPES)
def test_f32_split_within_fp32_tolerance(fh, m, k, n):
    # Rows of both operands as power-of-two scaled FP16 pairs, three pair
    # products per FP32 product on the FP16 matrix cores: the same tolerance
    # as the FP32 matrix cores; Glu and Add are the Store output passed
    # through them.
    a = gen.matrix(m * k, 3).reshape(m, k)
    w = gen.matrix(n * k, 4).reshape(n, k)
    lin = fh.Linear.from_f32(w)
    rs = (F32(0.5) + np.arange(m, dtype=np.float32) / F32(7.0)).astype(np.float32)
    S = fh.PrefillProjection.F32_SPLIT
    got = run_prefill(fh, lin, a, m, rs, fh.Epilogue.STORE, S)
    want = oracle.panel_gemm(a, m, k, w, n, row_scale=rs)
    ad = (a * rs[:, None]).astype(np.float32).astype(np.float64)
    mag = np.abs(ad) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30)
    assert max_rel(got, want) <= 1e-5
    glu = run_prefill(fh, lin, a, m, rs, fh.Epilogue.GLU, S)
    g, u = got[:, 0::2], got[:, 1::2]
    assert_bitwise(glu, (np.where(g > 0, g, F32(0)) ** 2 * u).astype(np.float32), "glu of store")
    base = gen.matrix(m * n, 5).reshape(m, n)
    add = run_prefill(fh, lin, a, m, rs, fh.Epilogue.ADD, S, base=base)
    assert_bitwise(add, (base + got).astype(np.float32), "add of store")


def test_f32_split_error_is_fp32_level(fh):
    # Against the exact (f64) product: the split kernel's error is of the
    # FP32 matrix-core kernel's order (each pair holds its value to 2^-22, the
    # lo.lo product left out is below 2^-21 |a w|, the FP32 sums' own
    # rounding dominates).
    m, k, n = 384, 2304, 256
    a = gen.normal((m, k), 1.0, 21)
    w = gen.normal((n, k), 0.02, 22)
    lin = fh.Linear.from_f32(w)
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    err = {}
    for kern in (fh.PrefillProjection.F32_SPLIT, fh.PrefillProjection.F32_MFMA, fh.PrefillProjection.F32_CHAIN):
        got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, kern).astype(np.float64)
        err[kern.name] = (float(np.max(np.abs(got - exact) / mag)), float(np.sqrt(np.mean(((got - exact) / mag) ** 2))))
    assert err["F32_SPLIT"][0] <= 2 * max(err["F32_MFMA"][0], err["F32_CHAIN"][0]), err
    assert err["F32_SPLIT"][1] <= 2 * max(err["F32_MFMA"][1], err["F32_CHAIN"][1]), err


@pytest.mark.parametrize("m", [2048, 2176])
def test_f32_split_tile_heights(fh, m):
    # Launch shapes of the FP16-pair kernel: 2,048 rows x 4,096 outputs fill
    # one whole round of 128-row tiles; 2,176 rows leave a last round at most
    # half full, which runs as 64-row tiles after the whole rounds (the small
    # shapes above run as 64-row tiles only). Every output within the FP32
    # bound, Store and Add.
    k, n = 256, 4096
    oracle.set_threads(oracle_threads())
    a = gen.normal((m, k), 1.0, 37)
    w = gen.normal((n, k), 0.02, 38)
    lin = fh.Linear.from_f32(w)
    S = fh.PrefillProjection.F32_SPLIT
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, S)
    want = oracle.panel_gemm_fast(a, m, k, w, n)
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30)
    base = gen.matrix(m * n, 39).reshape(m, n)
    add = run_prefill(fh, lin, a, m, None, fh.Epilogue.ADD, S, base=base)
    assert_bitwise(add, (base + got).astype(np.float32), "add of store")


def test_f32_split_power_of_two_row_scaling_is_exact(fh):
    # Each row of A and of W takes its own power-of-two scale, so scaling row
    # i of A by 2^a_i and row j of W by 2^b_j scales output (i, j) by exactly
    # 2^(a_i + b_j): bitwise, for exponents from -40 to 40.
    m, k, n = 200, 1024, 160
    rng = np.random.default_rng(31)
    a = gen.normal((m, k), 1.0, 32)
    w = gen.normal((n, k), 0.02, 33)
    ea = rng.integers(-40, 41, m)
    ew = rng.integers(-40, 41, n)
    S = fh.PrefillProjection.F32_SPLIT
    base = run_prefill(fh, fh.Linear.from_f32(w), a, m, None, fh.Epilogue.STORE, S)
    scaled = run_prefill(fh, fh.Linear.from_f32(np.ldexp(w, ew[:, None]).astype(np.float32)),
                         np.ldexp(a, ea[:, None]).astype(np.float32), m, None, fh.Epilogue.STORE, S)
    back = np.ldexp(scaled, -(ea[:, None] + ew[None, :])).astype(np.float32)
    assert np.array_equal(back.view(np.uint32), base.view(np.uint32))


def test_f32_split_wide_row_magnitudes(fh):
    # Rows of A spanning 2^-40 .. 2^40 and columns within a row spanning
    # 2^-20 .. 1 of its largest: every output within 2 k eps of the
    # magnitude sum against the exact product.
    m, k, n = 128, 768, 192
    rng = np.random.default_rng(34)
    a = (gen.normal((m, k), 1.0, 35) * np.ldexp(1.0, rng.integers(-40, 41, (m, 1)))
         * np.ldexp(1.0, rng.integers(-20, 1, (1, k)))).astype(np.float32)
    w = gen.normal((n, k), 0.02, 36)
    got = run_prefill(fh, fh.Linear.from_f32(w), a, m, None, fh.Epilogue.STORE,
                      fh.PrefillProjection.F32_SPLIT).astype(np.float64)
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got - exact) <= 2 * k * EPS * mag), float(np.max(np.abs(got - exact) / mag))


def tiny_rows():
    """Rows of A (and of W) that are zero, tiny normals or FP32 subnormals,
    beside ordinary ones (m, k, n = 12, 64, 64)."""
    m, k, n = 12, 64, 64
    a = gen.normal((m, k), 1.0, 37)
    scale = [0.0, 2.0 ** -100, 2.0 ** -110, 2.0 ** -118, 2.0 ** -124, 2.0 ** -126, 2.0 ** -130, 2.0 ** -140,
             1.0, 1.0, 1.0, 2.0 ** 100]
    a = (a * np.array(scale)[:, None]).astype(np.float32)
    a[9, :] = 0.0
    a[9, ::7] = np.float32(2.0 ** -149)  # the least subnormal, alone in a zero row
    a[10, 0] = np.float32(2.0 ** -140)  # a subnormal among normal values
    w = gen.normal((n, k), 0.02, 38)
    w[5] *= np.float32(2.0 ** -120)
    w[6] *= np.float32(2.0 ** -135)
    w[7] = 0.0
    return a, w, m, k, n


def test_f32_split_zero_tiny_and_subnormal_rows(fh):
    # A zero row gives zero outputs, and every output is within 2 k eps of
    # the magnitude sum plus one subnormal step (the final rounding into the
    # subnormal range) of the exact product; against the reference's panels,
    # whose products round one by one in the subnormal range, within twice
    # that plus k steps.
    a, w, m, k, n = tiny_rows()
    got = run_prefill(fh, fh.Linear.from_f32(w), a, m, None, fh.Epilogue.STORE,
                      fh.PrefillProjection.F32_SPLIT).astype(np.float64)
    assert np.all(got[0] == 0.0) and np.all(got[:, 7] == 0.0)
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = 2 * k * EPS * mag + 2.0 ** -149
    assert np.all(np.abs(got - exact) <= bound), float(np.max((np.abs(got - exact) - bound) / np.maximum(mag, 1e-300)))
    want = oracle.panel_gemm(a, m, k, w, n).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * k * EPS * mag + k * 2.0 ** -149)


def test_f32_chain_and_mfma_zero_tiny_and_subnormal_rows(fh):
    # The same rows through the FP32 kernels: the exact-order chain bitwise
    # the reference's panels (subnormal products and sums included), the FP32
    # matrix cores within 2 k eps of the magnitude sum plus k subnormal steps
    # of the panels.
    a, w, m, k, n = tiny_rows()
    lin = fh.Linear.from_f32(w)
    want = oracle.panel_gemm(a, m, k, w, n)
    chain = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.F32_CHAIN)
    assert_bitwise(chain, want, "chain, tiny rows")
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.F32_MFMA).astype(np.float64)
    mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = 2 * k * EPS * mag + k * 2.0 ** -149
    d = np.abs(got - want)
    assert np.all(d <= bound), float(np.max((d - bound) / np.maximum(mag, 1e-300)))


@pytest.mark.parametrize("bits", [32, 16, 8])
def test_f32_chain_and_mfma_nonfinite_rows(fh, bits):
    # Infinite and NaN inputs: the exact-order chain bitwise the reference's
    # panels (Store and Glu); the FP32 matrix cores with the panels' NaN and
    # signed-infinity pattern (an infinity meets a zero weight as NaN, and
    # opposite infinities cancel to NaN, in any order) and their finite
    # values within the FP32 tolerance; FP32 weights and code weights
    # (fl(code * scale) formed in the kernels).
    m, k, n = 20, 256, 64
    a = gen.matrix(m * k, 25).reshape(m, k)
    a[3, 17] = np.inf
    a[4, 2], a[4, 9] = np.inf, -np.inf
    a[6, 40] = -np.inf
    a[7, 5] = np.nan
    w = gen.matrix(n * k, 26).reshape(n, k)
    w[::3, 17] = 0.0
    w[:, 40] = np.abs(w[:, 40]) + np.float32(0.5)
    if bits == 32:
        lin = fh.Linear.from_f32(w)
    else:
        codes, scales = oracle.quantize_bits(w, n, k, 64, bits)
        lin = fh.QuantLinear(bits, codes, scales, 64)
        w = oracle.dequantize(bits, codes, scales, n, k, 64)
    want = oracle.panel_gemm(a, m, k, w, n)
    assert np.any(np.isnan(want[3])) and np.any(np.isinf(want[3])) and np.all(np.isinf(want[6]) & (want[6] < 0))
    chain = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.F32_CHAIN)
    assert_bitwise(chain, want, "chain, non-finite rows")
    glu = run_prefill(fh, lin, a, m, None, fh.Epilogue.GLU, fh.PrefillProjection.F32_CHAIN)
    assert_bitwise(glu, oracle.panel_gemm(a, m, k, w, n, epilogue=oracle.GLU), "chain glu, non-finite rows")
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue.STORE, fh.PrefillProjection.F32_MFMA)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got) & (got > 0), np.isinf(want) & (want > 0))
    assert np.array_equal(np.isinf(got) & (got < 0), np.isinf(want) & (want < 0))
    fin = np.isfinite(want)
    mag = np.abs(np.where(np.isfinite(a), a, 0).astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got[fin].astype(np.float64) - want[fin]) <= 2 * k * EPS * mag[fin] + 1e-30)


def test_f32_split_nonfinite_rows_are_the_panels_and_codes_are_refused(fh):
    # A row of A' or of W holding an infinity or NaN cannot go through the
    # FP16 pairs (inf * 0 = NaN against a zero half): every output it reaches
    # is the reference's FP32 chain, bitwise the panels (their NaN and
    # signed infinities), through Store, Glu and Add, with a row scale that
    # overflows a finite input to an infinity; the other outputs within the
    # FP32 tolerance and the tiles' other rows unaffected.
    m, k, n = 150, 256, 192
    a = gen.matrix(m * k, 23).reshape(m, k)
    a[3, 17] = np.inf
    a[4, 2], a[4, 9] = np.inf, -np.inf
    a[7, 5] = np.nan
    a[140, 100] = np.float32(3e38)  # times the row scale 4: an infinity in A'
    w = gen.matrix(n * k, 24).reshape(n, k)
    w[::3, 17] = 0.0
    w[11, 30] = np.nan
    w[64, 200] = -np.inf
    w[130, 0] = np.inf
    rs = np.ones(m, np.float32)
    rs[140] = 4.0
    lin = fh.Linear.from_f32(w)
    S = fh.PrefillProjection.F32_SPLIT
    bad_rows, bad_cols = [3, 4, 7, 140], [11, 64, 130]
    keep_r = [r for r in range(m) if r not in bad_rows]
    keep_c = [c for c in range(n) if c not in bad_cols]
    base = ((np.arange(m * n) % 17).astype(np.float32) - F32(8.0)).reshape(m, n)
    for epi, o_epi in ((fh.Epilogue.STORE, oracle.STORE), (fh.Epilogue.GLU, oracle.GLU), (fh.Epilogue.ADD, oracle.ADD)):
        got = run_prefill(fh, lin, a, m, rs, epi, S, base=base if o_epi == oracle.ADD else None)
        want = oracle.panel_gemm(a, m, k, w, n, row_scale=rs, epilogue=o_epi, out=base if o_epi == oracle.ADD else None)
        cols = keep_c if o_epi != oracle.GLU else [c for c in range(n // 2) if 2 * c not in bad_cols and 2 * c + 1 not in bad_cols]
        hit = np.ones(got.shape, bool)
        hit[np.ix_(keep_r, cols)] = False
        assert_bitwise(got[hit], want[hit], f"flagged outputs {epi.name}")
        assert not np.all(np.isfinite(want[hit]))
        assert max_rel(got[np.ix_(keep_r, cols)], want[np.ix_(keep_r, cols)]) <= 1e-5, epi.name
    codes, scales = oracle.quantize_bits(np.nan_to_num(w, posinf=0.0, neginf=0.0), n, k, 64, 8)
    q = fh.QuantLinear(8, codes, scales, 64)
    with pytest.raises(fh.FocrError) as e:
        run_prefill(fh, q, a, m, None, fh.Epilogue.STORE, S)
    assert e.value.code == fh.FOCR_E_UNSUPPORTED


def test_f32_split_nonfinite_rows_in_128_row_tiles(fh):
    # Enough tiles for the 128-row kernel: the flagged row and column are
    # the panels' bitwise, and every other output is bitwise the call on the
    # same inputs with the non-finite values replaced by zeros.
    m, k, n = 6544, 256, 1280
    a = gen.normal((m, k), 1.0, 27)
    w = gen.normal((n, k), 0.02, 28)
    bad_a, bad_w = a.copy(), w.copy()
    bad_a[5000, 33] = np.inf
    bad_a[77, 250] = np.nan
    bad_w[700, 3] = -np.inf
    S = fh.PrefillProjection.F32_SPLIT
    got = run_prefill(fh, fh.Linear.from_f32(bad_w), bad_a, m, None, fh.Epilogue.STORE, S)
    clean = run_prefill(fh, fh.Linear.from_f32(np.nan_to_num(bad_w, neginf=0.0)), np.nan_to_num(bad_a, nan=0.0, posinf=0.0),
                        m, None, fh.Epilogue.STORE, S)
    keep = np.ones((m, n), bool)
    keep[[77, 5000], :] = False
    keep[:, 700] = False
    assert np.array_equal(got[keep].view(np.uint32), clean[keep].view(np.uint32))
    for r in (77, 5000):
        assert_bitwise(got[r], oracle.panel_gemm(bad_a[r:r + 1], 1, k, bad_w, n)[0], f"row {r}")
    assert_bitwise(got[:, 700], oracle.panel_gemm(bad_a, m, k, bad_w[700:701], 1)[:, 0], "column 700")
    assert not np.any(np.isfinite(got[:, 700])) and not np.any(np.isfinite(got[5000]))


@pytest.mark.parametrize("bits", [16, 8])
def test_f32_mfma_on_codes_keeps_exception_columns(fh, bits):
    # Codes on the matrix cores: k a multiple of 64 takes the DMA kernel (codes
    # loaded into registers, exceptions added before the epilogue); k = 100
    # the register-staged kernel (exceptions in place).
    for m, k, n in ((13, 768, 64), (40, 1024, 96), (9, 192, 32), (9, 100, 48)):
        columns = [0, k // 2, k - 1]
        w = gen.matrix(n * k, 6).reshape(n, k)
        vals = (w[:, columns] * F32(300.0)).astype(np.float32)
        w[:, columns] = 0.0
        codes, scales = oracle.quantize_bits(w, n, k, 64 if k % 64 == 0 else 32, bits)
        group = 64 if k % 64 == 0 else 32
        lin = fh.QuantLinear(bits, codes, scales, group, exc_cols=columns, exc_vals=vals)
        dense = oracle.dequantize(bits, codes, scales, n, k, group, exc_cols=columns, exc_vals=vals)
        a = gen.matrix(m * k, 7).reshape(m, k)
        base = gen.matrix(m * n, 8).reshape(m, n)
        for epi, o_epi in ((fh.Epilogue.STORE, oracle.STORE), (fh.Epilogue.ADD, oracle.ADD)):
            got = run_prefill(fh, lin, a, m, None, epi, fh.PrefillProjection.F32_MFMA,
                              base=base if epi == fh.Epilogue.ADD else None)
            want = oracle.panel_gemm(a, m, k, dense, n, epilogue=o_epi, out=base.copy() if o_epi == oracle.ADD else None)
            assert max_rel(got, want) <= 1e-5, (bits, m, k, n, epi.name)


@pytest.mark.parametrize("name,k,n,epi", [("qkv", 768, 2048, 0), ("wo", 1024, 768, 2), ("w13", 768, 4608, 1),
                                          ("w2", 2304, 768, 2), ("literal", 1024, 4096, 0)])
def test_config1_fp32_gemm_checkpoint_shapes(fh, name, k, n, epi):
    # X ~ N(0,1), W ~ N(0, 0.02), m = 6544. Every output
    # against the FP32 panels (their AVX2 micro-kernel, bitwise panel_gemm):
    # the MFMA and split kernels within the FP32 tolerance, the chain kernel
    # bitwise.
    m = 6544
    a = gen.normal((m, k), 1.0, 10)
    w = gen.normal((n, k), 0.02, 11)
    lin = fh.Linear.from_f32(w)
    base = gen.normal((m, n), 1.0, 12) if epi == 2 else None
    oracle.set_threads(oracle_threads())
    want = oracle.panel_gemm_fast(a, m, k, w, n, epilogue=epi, out=base)
    got = run_prefill(fh, lin, a, m, None, fh.Epilogue(epi), fh.PrefillProjection.F32_MFMA, base=base)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 1e-5, name
    if epi == 0:
        mag = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
        assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30), name
    chain = run_prefill(fh, lin, a, m, None, fh.Epilogue(epi), fh.PrefillProjection.F32_CHAIN, base=base)
    assert_bitwise(chain, want, f"{name} chain")
    split = run_prefill(fh, lin, a, m, None, fh.Epilogue(epi), fh.PrefillProjection.F32_SPLIT, base=base)
    assert np.all(np.isfinite(split))
    assert max_rel(split, want) <= 1e-5, f"{name} split"
    if epi == 0:
        assert np.all(np.abs(split.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30), f"{name} split"


@pytest.mark.parametrize("bits", [16, 8])
@pytest.mark.parametrize("name,k,n,epi", [("qkv", 768, 2048, 0), ("wo", 1024, 768, 2), ("w13", 768, 4608, 1),
                                          ("w2", 2304, 768, 2), ("literal", 1024, 4096, 0)])
def test_codes_at_checkpoint_shapes(fh, bits, name, k, n, epi):
    # Near-exact mode's prefill (INT16 codes on the FP32 panels) and INT8
    # codes on the FP32 paths, at every checkpoint shape: the codes are read
    # as codes (no FP32 weight buffer). Chain bitwise the FP32 panels on the
    # dequantized matrix, matrix cores within the FP32 tolerance; a row scale
    # and three exception columns.
    m = 1000
    a = gen.normal((m, k), 1.0, 20)
    w = gen.normal((n, k), 0.02, 21)
    columns = [3, k // 3, k - 2]
    vals = (w[:, columns] * F32(40.0)).astype(np.float32)
    w[:, columns] = 0.0
    codes, scales = oracle.quantize_bits(w, n, k, 64, bits)
    lin = fh.QuantLinear(bits, codes, scales, 64, exc_cols=columns, exc_vals=vals)
    dense = oracle.dequantize(bits, codes, scales, n, k, 64, exc_cols=columns, exc_vals=vals)
    rs = gen.uniform(m, 0.5, 1.5, 22)
    base = gen.normal((m, n), 1.0, 23) if epi == 2 else None
    oracle.set_threads(oracle_threads())
    want = oracle.panel_gemm_fast(a, m, k, dense, n, row_scale=rs, epilogue=epi, out=base)
    chain = run_prefill(fh, lin, a, m, rs, fh.Epilogue(epi), fh.PrefillProjection.F32_CHAIN, base=base)
    assert_bitwise(chain, want, f"{name} chain on {bits}-bit codes")
    got = run_prefill(fh, lin, a, m, rs, fh.Epilogue(epi), fh.PrefillProjection.F32_MFMA, base=base)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 1e-5, name
    if epi == 0:
        ad = (a * rs[:, None]).astype(np.float32).astype(np.float64)
        mag = np.abs(ad) @ np.abs(dense.astype(np.float64)).T
        assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * k * EPS * mag + 1e-30), name


def test_codes_prefill_capture_is_independent_of_later_calls(fh):
    # A graph captured over prefills on codes holds no context buffer that a
    # later, larger eager prefill could free: its replays equal the eager
    # result bit for bit, with larger code prefills run between them.
    import torch

    ctx = fh.Context(0)
    m, k, n = 300, 768, 256
    w = gen.normal((n, k), 0.02, 30)
    codes, scales = oracle.quantize_bits(w, n, k, 64, 16)
    lin = fh.QuantLinear(16, codes, scales, 64, ctx=ctx)
    wb = gen.normal((4 * n, 2 * k), 0.02, 31)
    codes_b, scales_b = oracle.quantize_bits(wb, 4 * n, 2 * k, 64, 8)
    big = fh.QuantLinear(8, codes_b, scales_b, 64, ctx=ctx)
    x = to_dev(gen.normal((m, k), 1.0, 32))
    xb = to_dev(gen.normal((2 * m, 2 * k), 1.0, 33))
    out_m = torch.empty((m, n), device="cuda:0")
    out_c = torch.empty((m, n), device="cuda:0")
    eager_m = host(lin.prefill(x, m, kernel=fh.PrefillProjection.F32_MFMA))
    eager_c = host(lin.prefill(x, m, kernel=fh.PrefillProjection.F32_CHAIN))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ctx.use_stream(torch.cuda.current_stream())
            lin.prefill(x, m, out=out_m, kernel=fh.PrefillProjection.F32_MFMA)
            lin.prefill(x, m, out=out_c, kernel=fh.PrefillProjection.F32_CHAIN)
    ctx.use_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    for rep in range(3):
        out_m.fill_(float("nan"))
        out_c.fill_(float("nan"))
        big.prefill(xb, 2 * m, kernel=fh.PrefillProjection.F32_MFMA)  # larger eager calls between replays
        big.prefill(xb, 2 * m, kernel=fh.PrefillProjection.F32_CHAIN)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bitwise(host(out_m), eager_m, f"matrix-core replay {rep}")
        assert_bitwise(host(out_c), eager_c, f"chain replay {rep}")
    del g
    lin.free()
    big.free()
    ctx.close()
