"""The sealed split KV cache on the GPU (focr_kv_*) against the oracle: the
decoded prefix and tail are bit for bit the oracle's records (Kv::Q8 and
Kv::Q16), the refusals are the reference's, and decode attention over the
records is within FP32 rounding of the compact decode oracle over the decoded
values (src/quant/kv.rs; kv.rs:7-17: decode over records is the compact
kernel over their decoded values). With the cache's fast exp
(SplitPrefix::with_fast_exp) the oracle takes the per-key probabilities from
its exp_poly, as the reference's decode does, and the bound is the same."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import F32, assert_bitwise, host, to_dev
from test_oracle_kv import pair_cache

pytestmark = pytest.mark.gpu

N_HEADS, N_KV = 16, 8


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def max_rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def oracle_cache(bits, k, v, prefix_len, tail_k, tail_v, capacity):
    sealed = oracle.kv_seal(bits, k, v, prefix_len, N_HEADS, N_KV)
    assert not isinstance(sealed, int), sealed
    tail = oracle.kv_tail(bits, N_KV, capacity - prefix_len)
    for i in range(len(tail_k)):
        oracle.kv_push(bits, tail_k[i], tail_v[i], N_KV, capacity - prefix_len, i, tail)
    return oracle.kv_dequantize(bits, sealed, prefix_len, N_HEADS, N_KV, tail, capacity - prefix_len, len(tail_k))


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("prefix_len", [1, 37, 1000])
def test_seal_and_append_are_bitwise_the_oracle(fh, bits, prefix_len):
    k, v = pair_cache(prefix_len, N_KV, 11, 2.0)
    cap = prefix_len + 9
    tk = gen.normal((9, N_KV, 64), 1.5, 12)
    tv = gen.normal((9, N_KV, 64), 1.5, 13)
    tk[4, 3, 50] = np.nan  # that block decodes to NaN
    kv = fh.KvSplit.seal(bits, to_dev(k), to_dev(v), prefix_len, cap, N_HEADS, N_KV)
    kv.append(to_dev(tk[:5]), to_dev(tv[:5]), 5)
    kv.append(to_dev(tk[5:9]), to_dev(tv[5:9]), 4)
    assert kv.info()[:4] == (bits, prefix_len, 9, cap)
    pk, vals, gk = (host(t) for t in kv.dequantize())
    wpk, wvals, wgk = oracle_cache(bits, k, v, prefix_len, tk, tv, cap)
    assert_bitwise(pk, wpk, "prefix keys")
    assert_bitwise(vals, wvals, "values")
    assert_bitwise(gk, wgk, "generated keys")
    assert np.all(np.isnan(gk[4, 3, 32:])) and np.all(np.isfinite(gk[4, 3, :32]))
    kv.free()


@pytest.mark.parametrize("bits", [8, 16])
def test_tiny_subnormal_and_zero_blocks_are_bitwise_the_oracle(fh, bits):
    # Positions and tail blocks scaled into the tiny-normal and subnormal
    # range, and zero ones: their steps (floored at the least subnormal, 0
    # for a zero block) and codes are the oracle's: the decoded records are
    # bitwise.
    P = 70
    k, v = pair_cache(P, N_KV, 31, 2.0)
    for p, f in ((3, 1e-39), (4, 2.0 ** -140), (5, 0.0), (6, 1e-37), (50, 2.0 ** -149)):
        k[p] *= np.float32(f)
        v[p] *= np.float32(f)
    cap = P + 6
    tk = gen.normal((6, N_KV, 64), 1.5, 32)
    tv = gen.normal((6, N_KV, 64), 1.5, 33)
    tk[1] *= np.float32(1e-40)
    tv[2, 3] *= np.float32(2.0 ** -135)
    tk[4, 5] = 0.0
    tv[5] = 0.0
    kv = fh.KvSplit.seal(bits, to_dev(k), to_dev(v), P, cap, N_HEADS, N_KV)
    kv.append(to_dev(tk), to_dev(tv), 6)
    pk, vals, gk = (host(t) for t in kv.dequantize())
    wpk, wvals, wgk = oracle_cache(bits, k, v, P, tk, tv, cap)
    assert_bitwise(pk, wpk, "prefix keys")
    assert_bitwise(vals, wvals, "values")
    assert_bitwise(gk, wgk, "generated keys")
    assert np.any((wvals != 0) & (np.abs(wvals) < 2.0 ** -126)) and np.all(wvals[5] == 0)
    kv.free()


def test_refusals(fh):
    P = 6
    k, v = pair_cache(P, N_KV, 21)
    bad = k.copy()
    bad[2, 5, 3] = np.nextafter(bad[2, 5, 3], F32(np.inf))
    with pytest.raises(fh.FocrError, match="temporal keys differ"):
        fh.KvSplit.seal(8, to_dev(bad), to_dev(v), P, P + 2, N_HEADS, N_KV)
    nan = v.copy()
    nan[4, 7, 63] = np.nan
    with pytest.raises(fh.FocrError, match="nonfinite"):
        fh.KvSplit.seal(16, to_dev(k), to_dev(nan), P, P + 2, N_HEADS, N_KV)
    with pytest.raises(fh.FocrError) as e:
        fh.KvSplit.seal(8, to_dev(k), to_dev(v), P, P + 2, 16, 4)
    assert e.value.code == -2
    kv = fh.KvSplit.seal(8, to_dev(k), to_dev(v), P, P + 2, N_HEADS, N_KV)
    one = gen.normal((3, N_KV, 64), 1.0, 22)
    with pytest.raises(fh.FocrError) as e:
        kv.append(to_dev(one), to_dev(one), 3)  # capacity for 2
    assert e.value.code == -2
    kv.free()


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("prefix_len,tail,rows", [(64, 1, 1), (700, 3, 3), (2000, 8, 8), (129, 5, 2)])
def test_decode_within_fp32_rounding_of_the_compact_oracle(fh, bits, prefix_len, tail, rows, fast):
    k, v = pair_cache(prefix_len, N_KV, 31)
    cap = prefix_len + 16
    tk = gen.normal((tail, N_KV, 64), 1.0, 32)
    tv = gen.normal((tail, N_KV, 64), 1.0, 33)
    kv = fh.KvSplit.seal(bits, to_dev(k), to_dev(v), prefix_len, cap, N_HEADS, N_KV)
    kv.append(to_dev(tk), to_dev(tv), tail)
    assert kv.fast_exp is False  # SplitPrefix::from_compact leaves it off
    kv.set_fast_exp(fast)
    assert kv.fast_exp is fast
    q = gen.normal((rows, N_HEADS, 64), 1.0, 34)
    sinks = gen.uniform(N_HEADS, -2.0, 2.0, 35)
    got = host(kv.attention_decode(to_dev(q), rows, to_dev(sinks)))
    pk, vals, gk = oracle_cache(bits, k, v, prefix_len, tk, tv, cap)
    total = prefix_len + tail
    want = oracle.attention_decode(q, pk, gk, vals, rows, prefix_len, total, N_HEADS, N_KV, total - rows, 0, 0, sinks,
                                   exp_fast=fast)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 1e-5
    assert np.all(np.abs(got - want) <= 1e-5 * (1 + np.abs(want)))
    kv.free()


def test_config5_decode_over_q8_records(fh):
    # BASELINE config 5's decode: a 16,320-row prefix, 64 generated
    # positions, one query row at 16,384 (sampled against the oracle), with
    # the fast exp the reference's runner gives Q8 caches in fast mode.
    P, T = 16320, 64
    k, v = pair_cache(P, N_KV, 41)
    tk = gen.normal((T, N_KV, 64), 1.0, 42)
    tv = gen.normal((T, N_KV, 64), 1.0, 43)
    kv = fh.KvSplit.seal(8, to_dev(k), to_dev(v), P, P + T, N_HEADS, N_KV)
    kv.append(to_dev(tk), to_dev(tv), T)
    kv.set_fast_exp(fh.default_fast_exp(8, True))
    q = gen.normal((1, N_HEADS, 64), 1.0, 44)
    sinks = gen.uniform(N_HEADS, -2.0, 2.0, 45)
    got = host(kv.attention_decode(to_dev(q), 1, to_dev(sinks)))
    pk, vals, gk = oracle_cache(8, k, v, P, tk, tv, P + T)
    want = oracle.attention_decode(q, pk, gk, vals, 1, P, P + T, N_HEADS, N_KV, P + T - 1, 0, 0, sinks, exp_fast=True)
    assert max_rel(got, want) <= 1e-5
    bits, plen, tlen, cap, nbytes = kv.info()
    assert (bits, plen, tlen) == (8, P, T) and nbytes == N_KV * (P * 176 + T * 144)
    kv.free()


def test_fused_row_step_is_bitwise_the_unfused_one(fh):
    # focr_kv_qkv_rows = focr_qkv_rows (rows past the prefix) + focr_kv_append,
    # bit for bit: queries, and the decoded tail keys and values.
    import torch

    P, cap = 40, 60
    k, v = pair_cache(P, N_KV, 51)
    unfused = fh.KvSplit.seal(8, to_dev(k), to_dev(v), P, cap, N_HEADS, N_KV)
    fused = fh.KvSplit.seal(8, to_dev(k), to_dev(v), P, cap, N_HEADS, N_KV)
    width = N_HEADS * 64 + 2 * N_KV * 64
    for step, rows in enumerate([1, 3, 8]):
        qkv = gen.normal((rows, width), 2.0, 60 + step)
        if step == 1:
            qkv[2, N_HEADS * 64 + N_KV * 64 + 100] = np.inf  # a value block of group 1 decodes to NaN
        ang = gen.uniform((rows, N_HEADS, 32), -3.2, 3.2, 70 + step)
        rope = to_dev(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
        gk = torch.empty((rows, N_KV, 64), device="cuda")
        vv = torch.empty((rows, N_KV, 64), device="cuda")
        q1 = fh.qkv_rows(to_dev(qkv), rows, rope, N_HEADS, N_KV, 0, generated_k=gk, v=vv)
        unfused.append(gk, vv, rows)
        q2 = fused.qkv_rows(to_dev(qkv), rows, rope)
        assert_bitwise(host(q2), host(q1), f"step {step} queries")
    assert fused.info()[2] == unfused.info()[2] == 12
    for a, b, what in zip(fused.dequantize(), unfused.dequantize(), ("prefix keys", "values", "generated keys")):
        assert_bitwise(host(a), host(b), what)
    vals = host(fused.dequantize()[1])
    assert np.all(np.isnan(vals[P + 1 + 2, 1, 32:64])) and np.all(np.isfinite(vals[P + 1 + 2, 1, :32]))
    fused.free()
    unfused.free()


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("prefix_len,tail", [(700, 2), (16320, 5)])
def test_decode_row_is_bitwise_the_two_calls(fh, bits, fast, prefix_len, tail):
    # focr_kv_decode_row = focr_kv_qkv_rows (one row) + focr_kv_attention_decode
    # (rows = 1), bit for bit: query, output, and the records it appends.
    import torch

    k, v = pair_cache(prefix_len, N_KV, 81)
    cap = prefix_len + tail + 4
    tk = to_dev(gen.normal((tail, N_KV, 64), 1.0, 82))
    tv = to_dev(gen.normal((tail, N_KV, 64), 1.0, 83))
    two = fh.KvSplit.seal(bits, to_dev(k), to_dev(v), prefix_len, cap, N_HEADS, N_KV)
    one = fh.KvSplit.seal(bits, to_dev(k), to_dev(v), prefix_len, cap, N_HEADS, N_KV)
    for kv in (two, one):
        kv.append(tk, tv, tail)
        kv.set_fast_exp(fast)
    sinks = to_dev(gen.uniform(N_HEADS, -2.0, 2.0, 84))
    width = N_HEADS * 64 + 2 * N_KV * 64
    for step in range(3):
        qkv = gen.normal((1, width), 2.0, 90 + step)
        if step == 2:
            qkv[0, N_HEADS * 64 + N_KV * 64 + 3 * 64 + 7] = np.inf  # group 3's first value block decodes to NaN
        ang = gen.uniform((1, N_HEADS, 32), -3.2, 3.2, 95 + step)
        rope = to_dev(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
        q2 = two.qkv_rows(to_dev(qkv), 1, rope)
        out2 = two.attention_decode(q2, 1, sinks)
        q1 = torch.empty_like(q2)
        out1 = one.decode_row(to_dev(qkv), rope, sinks, q=q1)
        assert one.info()[2] == two.info()[2] == tail + step + 1
        assert_bitwise(host(q1), host(q2), f"step {step} query")
        assert_bitwise(host(out1), host(out2), f"step {step} output")
        if step < 2:
            assert np.all(np.isfinite(host(out1)))
        else:
            o = host(out1)[0]  # heads 6 and 7 read group 3's values: dims 0-31 NaN, the rest finite
            assert np.all(np.isnan(o[6:8, :32])) and np.all(np.isfinite(o[6:8, 32:]))
            assert np.all(np.isfinite(o[:6])) and np.all(np.isfinite(o[8:]))
    for a, b, what in zip(one.dequantize(), two.dequantize(), ("prefix keys", "values", "generated keys")):
        assert_bitwise(host(a), host(b), what)
    one.free()
    two.free()
