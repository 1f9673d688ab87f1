"""Pins the oracle's QKV row step and decode attention (CPU only).

orc_qkv_rows restates fused_row / split_norm_rope + append_unique_heads
(src/model/fused.rs:101-123, src/model/rope.rs:14-86, src/model/cache.rs:202-216);
orc_attention_decode restates online::head (src/kernels/attention/online.rs:96-150).
Checks that a plausible mistake fails: f64 restatements with bounds, exact
rotations (cos, sin) in {0, +-1} that expose a sign or pairing error, the
compact == expanded cache identity the reference asserts
(decode64.rs compact_case), a single-key closed form, and GQA indexing.
"""
import math

import numpy as np
import pytest

import gen
import oracle

F32_EPS = float(np.finfo(np.float32).eps)
H, G = 16, 8


def rope_table(rows, seed, exact=None):
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-3.2, 3.2, size=(rows, H, 32))
    t = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    if exact is not None:
        t[...] = np.asarray(exact, dtype=np.float32)
    return t


def qkv_input(rows, seed):
    x = gen.values(rows * (H * 64 + 2 * G * 64), seed, 4.0).reshape(rows, -1)
    x[0, 3] = 0.0
    x[0, 70] = 1e-30
    x[0, 200] = 3e4
    return x


def f64_norm_rope(head, factors):
    x = head.astype(np.float64)
    y = x / np.sqrt(np.mean(x * x) + F32_EPS)
    c, s = factors[:, 0].astype(np.float64), factors[:, 1].astype(np.float64)
    a, b = y[0::2], y[1::2]
    out = np.empty(64)
    out[0::2] = a * c - b * s
    out[1::2] = a * s + b * c
    return out


@pytest.mark.parametrize("prefix_rows", [0, 3, 5])
def test_qkv_rows_against_f64(prefix_rows):
    rows = 5
    x = qkv_input(rows, 11)
    rope = rope_table(rows, 12)
    q, pk, gk, v = oracle.qkv_rows(x, rows, rope, H, G, prefix_rows)
    for r in range(rows):
        for h in range(H):
            want = f64_norm_rope(x[r, h * 64:(h + 1) * 64], rope[r, h])
            np.testing.assert_allclose(q[r, h], want, rtol=0, atol=4e-6 * 8)
            if r < prefix_rows:
                kv = h // (H // G)
                want = f64_norm_rope(x[r, H * 64 + kv * 64:H * 64 + (kv + 1) * 64], rope[r, h])
                np.testing.assert_allclose(pk[r, h], want, rtol=0, atol=4e-6 * 8)
        np.testing.assert_array_equal(v[r].ravel(), x[r, H * 64 + G * 64:])


def test_qkv_rows_exact_rotations_pin_signs_and_pairs():
    rows = 2
    x = qkv_input(rows, 21)
    ident = rope_table(rows, 0, exact=[1.0, 0.0])
    quarter = rope_table(rows, 0, exact=[0.0, 1.0])
    half = rope_table(rows, 0, exact=[-1.0, 0.0])
    q0, *_ = oracle.qkv_rows(x, rows, ident, H, G, rows)
    q1, *_ = oracle.qkv_rows(x, rows, quarter, H, G, rows)
    q2, *_ = oracle.qkv_rows(x, rows, half, H, G, rows)
    # (a, b) -> (a cos - b sin, a sin + b cos): a quarter turn is (-b, a),
    # a half turn (-a, -b), exactly (products by 0 and +-1 are exact).
    np.testing.assert_array_equal(q1[..., 0::2], -q0[..., 1::2])
    np.testing.assert_array_equal(q1[..., 1::2], q0[..., 0::2])
    np.testing.assert_array_equal(q2, -q0)
    # Without rotation a head is x * scale with one scale per head.
    for r in range(rows):
        for h in range(H):
            head = x[r, h * 64:(h + 1) * 64]
            scale = np.float32(oracle.rms_scale(head))
            np.testing.assert_array_equal(q0[r, h], head * scale)


def test_generated_keys_are_the_first_expanded_head_of_each_group():
    # compact == expanded (cache.rs:202-216 debug_assert; decode64.rs compact_case).
    rows = 4
    x = qkv_input(rows, 31)
    rope = rope_table(rows, 32)
    q_a, pk, _, v_a = oracle.qkv_rows(x, rows, rope, H, G, rows)
    q_b, _, gk, v_b = oracle.qkv_rows(x, rows, rope, H, G, 0)
    np.testing.assert_array_equal(q_a, q_b)
    np.testing.assert_array_equal(v_a, v_b)
    np.testing.assert_array_equal(gk, pk[:, 0::2])
    # Paired heads differ only through their rotation: with one rotation for
    # both heads of a group, their prefix keys are identical.
    rope_same = rope.copy()
    rope_same[:, 1::2] = rope_same[:, 0::2]
    _, pk2, _, _ = oracle.qkv_rows(x, rows, rope_same, H, G, rows)
    np.testing.assert_array_equal(pk2[:, 0::2], pk2[:, 1::2])


def f64_decode(q, pk, gk, v, rows, prefix, total, offset, image, sinks, n_kv=G):
    """Exact softmax attention with the sink factor, in f64."""
    rep = H // n_kv
    out = np.zeros((rows, H, 64))
    for r in range(rows):
        a = offset + r
        end = image[1] if image[0] <= a < image[1] else a + 1
        for h in range(H):
            keys = np.array([pk[j, h] if j < prefix else gk[j - prefix, h // rep] for j in range(end)], np.float64)
            vals = v[:end, h // rep].astype(np.float64)
            s = keys @ q[r, h].astype(np.float64) / 8.0
            m = s.max()
            p = np.exp(s - m)
            lse = m + np.log(p.sum())
            out[r, h] = (p @ vals) / p.sum() / (1.0 + np.exp(sinks[h] - lse))
    return out


def decode_case(total, prefix, rows, offset, image, seed, n_kv=G, scale=0.75):
    q = gen.att_values(rows * H * 64, 41 + seed, scale).reshape(rows, H, 64)
    pk = gen.att_values(max(prefix, 1) * H * 64, 53 + seed, scale).reshape(-1, H, 64)[:prefix]
    gk = gen.att_values(max(total - prefix, 1) * n_kv * 64, 67 + seed, scale).reshape(-1, n_kv, 64)[:total - prefix]
    v = gen.att_values(total * n_kv * 64, 79 + seed, 1.0).reshape(total, n_kv, 64)
    sinks = np.array([[-1000.0, 1000.0, 0.0, 2.25][h % 4] for h in range(H)], np.float32)
    got = oracle.attention_decode(q, pk, gk, v, rows, prefix, total, H, n_kv, offset, image[0], image[1], sinks)
    return q, pk, gk, v, sinks, got


@pytest.mark.parametrize("total,prefix,rows,offset,image", [
    (1, 1, 1, 0, (0, 0)), (17, 9, 1, 16, (1, 8)), (129, 0, 1, 128, (0, 0)), (161, 129, 1, 160, (1, 128)),
    (161, 129, 3, 60, (1, 128)), (257, 128, 2, 255, (1, 128)), (300, 200, 4, 296, (0, 150))])
def test_decode_against_f64(total, prefix, rows, offset, image):
    q, pk, gk, v, sinks, got = decode_case(total, prefix, rows, offset, image, total)
    want = f64_decode(q, pk, gk, v, rows, prefix, total, offset, image, sinks)
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= 1e-5 * (1.0 + np.abs(want)))


@pytest.mark.parametrize("n_kv", [4, 8, 16])
def test_decode_compact_equals_expanded(n_kv):
    total, prefix, rows, offset, image = 257, 129, 1, 256, (1, 128)
    q, pk, gk, v, sinks, got = decode_case(total, prefix, rows, offset, image, 5, n_kv=n_kv)
    rep = H // n_kv
    keys = np.concatenate([pk, np.repeat(gk, rep, axis=1)], axis=0)
    vals = np.repeat(v, rep, axis=1)
    expanded = oracle.attention_decode(q, keys, None, vals, rows, total, total, H, H, offset, image[0], image[1], sinks)
    np.testing.assert_array_equal(got.view(np.uint32), expanded.view(np.uint32))


@pytest.mark.parametrize("total,prefix,rows,offset,image", [
    (17, 9, 1, 16, (1, 8)), (161, 129, 3, 60, (1, 128)), (300, 200, 4, 296, (0, 150))])
def test_fast_exp_decode_against_f64(total, prefix, rows, offset, image):
    # SplitPrefix::fast_exp changes the per-key exps only: same bound as exact.
    q, pk, gk, v, sinks, exact = decode_case(total, prefix, rows, offset, image, total)
    fast = oracle.attention_decode(q, pk, gk, v, rows, prefix, total, H, G, offset, image[0], image[1], sinks,
                                   exp_fast=True)
    want = f64_decode(q, pk, gk, v, rows, prefix, total, offset, image, sinks)
    assert np.all(np.abs(fast - want) <= 1e-5 * (1.0 + np.abs(want)))
    assert not np.array_equal(fast.view(np.uint32), exact.view(np.uint32))  # the switch does something


def fma32(a, b, c):
    """fl32(a * b + c) for float32 operands whose exact sum f64 holds."""
    return np.float32(float(a) * float(b) + float(c))


def test_fast_exp_decode_two_key_closed_form():
    # Two keys with scores 0 and x < 0 (one-hot q and k), sinks -1000 (scale
    # exactly 1), integer values: p0 = exp(0), p1 = exp_poly(x), out =
    # fma(p1, v1, p0 * v0) / (p0 + p1). The exact path takes expf(x) instead.
    xs = np.array([-0.3711, -1.0, -2.5, -0.0625, -7.75, -13.0, -0.9, -4.1, -0.01, -20.5, -3.3, -1.7, -0.55, -6.2,
                   -11.9, -2.05], np.float32)
    q = np.zeros((1, H, 64), np.float32)
    q[0, :, 0] = 8.0
    pk = np.zeros((2, H, 64), np.float32)
    pk[1, :, 0] = xs
    v = gen.uniform((2, G, 64), -8.0, 8.0, 7).round().astype(np.float32)
    sinks = np.full(H, -1000.0, np.float32)
    for exp_fast in (True, False):
        got = oracle.attention_decode(q, pk, None, v, 1, 2, 2, H, G, 1, 0, 0, sinks, exp_fast=exp_fast)
        for h in range(H):
            x = np.float32(np.float32(xs[h] * np.float32(8.0)) * np.float32(0.125))
            assert x == xs[h]
            p0 = np.float32(oracle.exp_poly(0.0)) if exp_fast else np.float32(1.0)
            p1 = np.float32(oracle.exp_poly(float(x))) if exp_fast else np.float32(math.exp(float(x)))
            den = np.float32(p0 + p1)
            for d in range(64):
                o = fma32(p1, v[1, h // 2, d], np.float32(p0 * v[0, h // 2, d]))
                assert got[0, h, d] == np.float32(o / den), (exp_fast, h, d)
    assert oracle.exp_poly(0.0) == 1.0
    # Some of these inputs separate exp_poly from expf, so the two paths differ.
    assert any(np.float32(oracle.exp_poly(float(x))) != np.float32(math.exp(float(x))) for x in xs)


def test_decode_single_key_closed_form():
    # One visible key: p = 1, den = 1, lse = s, out = v / (1 + exp(sink - s)).
    q = gen.att_values(H * 64, 3, 0.5).reshape(1, H, 64)
    k = gen.att_values(H * 64, 4, 0.5).reshape(1, H, 64)
    v = gen.att_values(G * 64, 5, 2.0).reshape(1, G, 64)
    sinks = np.linspace(-2, 2, H).astype(np.float32)
    got = oracle.attention_decode(q, k, None, v, 1, 1, 1, H, G, 0, 0, 0, sinks)
    for h in range(H):
        s = np.float32(oracle.dot(q[0, h], k[0, h])) * np.float32(0.125)
        # expf correctly rounded (f64 exp, rounded once), as glibc's is on these inputs.
        e = np.float32(math.exp(float(np.float32(sinks[h]) - s)))
        scale = np.float32(1.0) / (np.float32(1.0) + e)
        np.testing.assert_array_equal(got[0, h], (v[0, h // 2] / np.float32(1.0)) * scale)
