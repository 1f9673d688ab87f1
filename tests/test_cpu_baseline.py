"""The CPU baseline's performance restatement of the FP32 panel GEMM
(oracle/focr_cpu_panels.c: the reference's AVX2 6x16 FMA micro-kernel) is bit
for bit the oracle's panel GEMM, for every epilogue, row scale and ragged
shape (rows not a multiple of 6, columns not a multiple of 16)."""
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
