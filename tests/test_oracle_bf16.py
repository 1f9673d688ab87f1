"""Pins the oracle's BF16 prefill attention (A8) with the reference's own
checks: the f64 bound on BF16-rounded operands of
src/kernels/attention/prefill64/bf16.rs (matches_bf16_operand_reference), the
static variant's bound and exp2 polynomial bound
(prefill64/bf16/static_shift/tests.rs), and the BF16 rounding rule."""
import numpy as np
import pytest

import gen
import oracle

CASES = [(70, 3, 65), (300, 5, 262), (257, 0, 257), (129, 1, 128), (40, 0, 3), (95, 10, 90)]


def f64_attention(q, k, v, L, heads, kv_heads, image_start, image_end, sinks, shift=True):
    """Exact-exp f64 attention (prefill64/test_data.rs:38-81 and bf16.rs:853-890)."""
    q = q.reshape(L, heads, 64).astype(np.float64)
    k = k.reshape(L, heads, 64).astype(np.float64)
    v = v.reshape(L, kv_heads, 64).astype(np.float64)
    pos = np.arange(L)
    image = (pos >= image_start) & (pos < image_end)
    visible = (pos[None, :] <= pos[:, None]) | (image[:, None] & image[None, :])
    out = np.zeros((L, heads, 64))
    for h in range(heads):
        logits = q[:, h, :] @ k[:, h, :].T / 8.0
        logits = np.where(visible, logits, -np.inf)
        m = logits.max(axis=1, keepdims=True) if shift else np.zeros((L, 1))
        e = np.exp(logits - m)
        den = e.sum(axis=1, keepdims=True)
        lse = (m + np.log(den))[:, 0]
        sink = 1.0 / (1.0 + np.exp(sinks[h] - lse))
        out[:, h, :] = (e @ v[:, h // (heads // kv_heads), :]) / den * sink[:, None]
    return out


def test_bf16_round_ties_to_even_and_nan():
    one_ulp = np.float32(2.0 ** -7)
    x = np.array([1.0, 1 + 2.0 ** -8, 1 + 2.0 ** -8 + 2.0 ** -9, 1 + 3 * 2.0 ** -8, -2.5, 3.0e38, np.nan], np.float32)
    got = oracle.bf16_round(x)
    assert got[0] == 1.0 and got[1] == 1.0  # tie -> even (mantissa 0)
    assert got[2] == 1 + one_ulp  # above the half-way point
    assert got[3] == 1 + 2 * one_ulp  # tie -> even (mantissa 2)
    assert got[4] == -2.5
    assert np.isnan(got[6])
    assert (got.view(np.uint32)[:6] & 0xFFFF).tolist() == [0] * 6


def test_exp2_minimax_within_the_reference_bound():
    # static_shift/tests.rs:29-58: every 509th FP32 value in [-120, 120].
    bits = np.arange(0, np.float32(120.0).view(np.uint32) + 1, 509, dtype=np.uint32)
    ts = np.concatenate([bits.view(np.float32), -bits.view(np.float32)])
    worst = max(abs(float(oracle.exp2_minimax(t)) / 2.0 ** float(t) - 1.0) for t in ts[::7])
    assert worst < 7.6e-5
    assert worst > 1e-6  # a degree-3 polynomial, not the exact exp2


@pytest.mark.parametrize("L,image_start,image_end", CASES)
def test_bf16_online_within_the_reference_f64_bound(L, image_start, image_end):
    # BF16-exact operands, as the reference's test makes them (bf16.rs:683-694),
    # so the short tiles' FP32 path sees the same values.
    heads, kv_heads = 16, 8
    r = oracle.bf16_round
    q = r(gen.values(L * heads * 64, 17 + L, 3.0))
    k = r(gen.values(L * heads * 64, 19 + L, 3.0))
    v = r(gen.values(L * kv_heads * 64, 23 + L, 3.0))
    sinks = gen.values(heads, 29, 2.0)
    got = oracle.attention_prefill_bf16(q, k, v, L, heads, kv_heads, image_start, image_end, sinks,
                                        static=False, exp_fast=False)
    want = f64_attention(q, k, v, L, heads, kv_heads, image_start, image_end, sinks)
    worst = np.abs(got - want).max()
    assert worst <= 3.0 * 2.0 ** -9 + 2e-3, worst
    # The probabilities really are rounded: the FP32 kernel on the same
    # operands is much closer to f64 than the BF16 one.
    f32 = oracle.attention_prefill(q, k, v, L, L, L, heads, kv_heads, 0, image_start, image_end, sinks,
                                   static=False, exp_fast=False)
    assert np.abs(f32 - want).max() < 1e-4 < worst


@pytest.mark.parametrize("L,image_start,image_end", CASES)
def test_bf16_static_within_the_reference_f64_bound(L, image_start, image_end):
    heads, kv_heads = 16, 8
    r = oracle.bf16_round
    q = r(gen.normalized(L * heads * 64, 17 + L))
    k = r(gen.normalized(L * heads * 64, 19 + L))
    v = r(gen.values(L * kv_heads * 64, 23 + L, 3.0))
    sinks = gen.values(heads, 29, 2.0)
    got = oracle.attention_prefill_bf16(q, k, v, L, heads, kv_heads, image_start, image_end, sinks,
                                        static=True, exp_fast=True)
    want = f64_attention(q, k, v, L, heads, kv_heads, image_start, image_end, sinks, shift=False)
    worst = np.abs(got - want).max()
    assert worst <= 3.0 * 2.0 * (2.0 ** -8 + 7.5e-5) + 1e-4, worst
    online = oracle.attention_prefill_bf16(q, k, v, L, heads, kv_heads, image_start, image_end, sinks,
                                           static=False, exp_fast=True)
    assert np.abs(online - want).max() <= 3.0 * 2.0 ** -9 + 2e-3


def test_bf16_tiles_are_independent():
    L, heads, kv_heads = 300, 16, 8
    q = gen.values(L * heads * 64, 5, 3.0)
    k = gen.values(L * heads * 64, 6, 3.0)
    v = gen.values(L * kv_heads * 64, 7, 3.0)
    sinks = gen.values(heads, 29, 2.0)
    whole = oracle.attention_prefill_bf16(q, k, v, L, heads, kv_heads, 5, 262, sinks)
    part = oracle.attention_prefill_bf16(q, k, v, L, heads, kv_heads, 5, 262, sinks, tiles=(3, 5))
    assert np.array_equal(whole[96:160].view(np.uint32), part[96:160].view(np.uint32))
