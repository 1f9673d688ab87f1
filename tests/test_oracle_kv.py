"""The sealed split KV cache's oracle (Kv::Q8 / Kv::Q16, src/quant/kv.rs and
src/quant/kv/codec.rs) against closed forms: BF16 rounding up of the step,
ties-to-even codes, the clamp, |decoded - value| <= step / 2, exact round
trips, the record layout (temporal half shared by a GQA pair) and the
reference's refusals. CPU only."""
import numpy as np
import pytest

import gen
import oracle

F32 = np.float32


def f32_bits(x):
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def test_bf16_up_closed_form():
    for x in (1.0, 0.5, 3.0, 1e-3, 7.0e-39, 1.4e-45, 0.0, 65504.0):
        bits = f32_bits(x)
        want = (bits >> 16) + (1 if bits & 0xFFFF else 0)
        assert oracle.bf16_up(x) == want, x
        assert oracle.bf16_f32(want) >= F32(x)
    assert oracle.bf16_up(float("nan")) == 0x7FC0
    assert oracle.bf16_up(1.0) == 0x3F80 and oracle.bf16_f32(0x3F80) == 1.0


def pair_cache(prefix_len, n_kv, seed, scale=1.0):
    """Compact prefix keys [P][2 n_kv][64] whose paired heads share the
    temporal half, and values [P][n_kv][64]."""
    k = gen.normal((prefix_len, 2 * n_kv, 64), scale, seed)
    k[:, 1::2, :32] = k[:, 0::2, :32]
    v = gen.normal((prefix_len, n_kv, 64), scale, seed + 1)
    return k, v


@pytest.mark.parametrize("bits", [8, 16])
def test_seal_layout_steps_and_error_bound(bits):
    P, n_kv = 37, 8
    k, v = pair_cache(P, n_kv, 3, 2.0)
    codes, scales = oracle.kv_seal(bits, k, v, P, 2 * n_kv, n_kv)
    limit = 127.0 if bits == 8 else 32767.0
    tail = oracle.kv_tail(bits, n_kv, 4)
    pk, vals, _ = oracle.kv_dequantize(bits, (codes, scales), P, 2 * n_kv, n_kv, tail, 4, 0)
    for g in range(n_kv):
        for t in range(P):
            rec = np.concatenate([k[t, 2 * g, :32], k[t, 2 * g, 32:], k[t, 2 * g + 1, 32:], v[t, g]])
            for blk in range(5):
                block = rec[32 * blk:32 * blk + 32]
                step = oracle.bf16_f32(int(scales[g, t, blk]))
                # The smallest BF16 at or above absmax / limit (in f64, rounded to f32).
                assert step == oracle.bf16_f32(oracle.bf16_up(float(F32(np.abs(block).max() / limit))))
                c = codes[g, t, 32 * blk:32 * blk + 32].astype(np.float64)
                assert np.all(np.abs(c) <= limit)
                assert np.all(np.abs(block.astype(np.float64) - c * step) <= step / 2)
    # Layout: both heads of a pair decode the shared temporal half; values follow.
    assert np.array_equal(pk[:, 0::2, :32], pk[:, 1::2, :32])
    assert np.all(np.abs(pk - k) <= np.abs(k).max() / limit)
    assert np.all(np.abs(vals - v) <= np.abs(v).max() / limit)


@pytest.mark.parametrize("bits", [8, 16])
def test_round_trip_of_multiples_of_the_step_and_ties(bits):
    # One block per record part: values that are multiples of a power-of-two
    # step decode exactly; half steps round to even.
    limit = 127 if bits == 8 else 32767
    P, n_kv = 1, 1
    k = np.zeros((P, 2, 64), np.float32)
    v = np.zeros((P, 1, 64), np.float32)
    k[0, 0, 0] = k[0, 1, 0] = F32(limit)  # temporal block: step exactly 1.0
    k[0, 0, 1:5] = k[0, 1, 1:5] = np.array([0.5, 1.5, 2.5, -3.5], np.float32)
    k[0, 0, 32] = F32(-limit / 4)  # spatial block of head 0: step 0.25
    k[0, 0, 33:36] = np.array([3.25, -0.125, 0.375], np.float32)  # 13 exact, -0.5 -> -0 (even), 1.5 -> 2
    codes, scales = oracle.kv_seal(bits, k, v, P, 2, 1)
    assert oracle.bf16_f32(int(scales[0, 0, 0])) == 1.0
    assert codes[0, 0, :5].tolist() == [limit, 0, 2, 2, -4]
    assert oracle.bf16_f32(int(scales[0, 0, 1])) == 0.25
    assert codes[0, 0, 32:36].tolist() == [-limit, 13, 0, 2]
    # All-zero blocks: step 0, codes 0 (the head-1 spatial and the value blocks).
    assert scales[0, 0, 2] == 0 and scales[0, 0, 3] == 0 and scales[0, 0, 4] == 0


def test_seal_refuses_what_the_reference_refuses():
    P, n_kv = 5, 2
    k, v = pair_cache(P, n_kv, 9)
    bad = k.copy()
    bad[3, 1, 7] = np.nextafter(bad[3, 1, 7], F32(np.inf))  # temporal half differs inside a pair
    assert oracle.kv_seal(8, bad, v, P, 4, 2) == -1
    nan = v.copy()
    nan[2, 1, 40] = np.nan
    assert oracle.kv_seal(8, k, nan, P, 4, 2) == -2
    assert oracle.kv_seal(8, k, v, P, 4, 3) == -4  # heads must be 2 x KV heads


@pytest.mark.parametrize("bits", [8, 16])
def test_tail_push_and_nonfinite_blocks(bits):
    n_kv, cap = 3, 6
    tail = oracle.kv_tail(bits, n_kv, cap)
    ks = gen.normal((cap, n_kv, 64), 1.5, 21)
    vs = gen.normal((cap, n_kv, 64), 1.5, 22)
    ks[2, 1, 40] = np.inf  # block 1 of record (group 1, position 2) holds an infinity
    for i in range(4):
        oracle.kv_push(bits, ks[i], vs[i], n_kv, cap, i, tail)
    k0, v0 = pair_cache(1, n_kv, 30)
    sealed = oracle.kv_seal(bits, k0, v0, 1, 2 * n_kv, n_kv)
    _, vals, gk = oracle.kv_dequantize(bits, sealed, 1, 2 * n_kv, n_kv, tail, cap, 4)
    limit = 127.0 if bits == 8 else 32767.0
    for i in range(4):
        for g in range(n_kv):
            if (i, g) == (2, 1):
                assert np.all(np.isnan(gk[i, g, 32:])) and np.all(np.isfinite(gk[i, g, :32]))
                continue
            for blk in range(2):
                ref = ks[i, g, 32 * blk:32 * blk + 32]
                assert np.all(np.abs(gk[i, g, 32 * blk:32 * blk + 32] - ref) <= np.abs(ref).max() / limit)
            assert np.all(np.abs(vals[1 + i, g] - vs[i, g]) <= np.abs(vs[i, g]).max() / limit)
