"""The screened vocabulary head's oracle against what pins it: the reference's
own tests (src/head_screen.rs:522-699, re-run here on the same LCG heads), the
full FP32 argmax, the bound's premise under the adversarial rounding
direction, and closed forms. CPU only."""
import math

import numpy as np
import pytest

import oracle

F32 = np.float32


class Lcg:
    """The reference tests' generator (src/head_screen.rs:527-535)."""

    def __init__(self, seed):
        self.s = seed

    def next(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
        return float(F32(F32(self.s >> 40) / F32(1 << 24)) * F32(2.0) - F32(1.0))

    def take(self, n, mul=1.0):
        return np.array([self.next() for _ in range(n)], dtype=np.float32) * F32(mul)


def full_argmax(x, head, vocab, dim):
    logits = oracle.linear_decode(32, head, None, vocab, dim, 64, x, 1)[0]
    return oracle.argmax(logits)


def test_kappa_closed_form():
    # kappa = (0.5 (1+2^-20) + g(n) 127.5 (1+2^-20) + g(n+groups+8) 127) (1+1e-3) + 2e-3, rounded up.
    u = 2.0 ** -24
    g = lambda n: n * u / (1 - n * u)
    for dim in (64, 768, 1024, 4096):
        k = (0.5 * (1 + 2.0 ** -20) + g(dim) * 127.5 * (1 + 2.0 ** -20) + g(dim + dim // 64 + 8) * 127.0) * 1.001 + 2e-3
        if k < 0.53:
            assert oracle.screen_kappa(dim) == np.nextafter(F32(k), F32(np.inf))
        else:
            # "screened head bound is unexpectedly loose": a 4096-wide head is refused.
            assert dim == 4096 and math.isnan(oracle.screen_kappa(dim))
    with pytest.raises(ValueError):
        oracle.screen_build(np.ones((1, 4096), np.float32), 1, 4096)


def test_quantization_ties_to_even_and_scale():
    # One group whose absmax is 127 (scale 1.0): codes are RNE of the values.
    row = np.zeros(64, dtype=np.float32)
    row[:8] = [127.0, -127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.25]
    codes, scales, wmax, _ = oracle.screen_build(row, 1, 64)
    assert scales[0, 0] == F32(1.0) and wmax == 127.0
    assert codes[0, :8].tolist() == [127, -127, 0, 2, 2, 0, -2, 3]
    # An all-zero group has scale 0 and codes 0; a tiny group gets the smallest subnormal scale floor.
    zero = np.zeros(64, dtype=np.float32)
    c0, s0, _, _ = oracle.screen_build(zero, 1, 64)
    assert s0[0, 0] == 0 and not c0.any()
    tiny = np.zeros(64, dtype=np.float32)
    tiny[0] = np.float32(1e-45)
    _, s1, _, _ = oracle.screen_build(tiny, 1, 64)
    assert s1[0, 0] == np.float32(1.4e-45)


def test_rejects_nonfinite_weights():
    head = np.full(4 * 64, 0.25, dtype=np.float32)
    head[70] = np.inf
    with pytest.raises(ValueError):
        oracle.screen_build(head, 4, 64)


def test_bound_covers_adversarial_rounding_direction():
    vocab, dim = 64, 768
    head = Lcg(5).take(vocab * dim).reshape(vocab, dim)
    codes, scales, _, kappa = oracle.screen_build(head, vocab, dim)
    for row in range(vocab):
        w_hat = codes[row].astype(np.float32) * np.repeat(scales[row], 64)
        x = np.where(head[row] >= w_hat, F32(1.0), F32(-1.0)).astype(np.float32)
        exact = float(np.dot(x.astype(np.float64), head[row].astype(np.float64)))
        norms = np.abs(x).reshape(-1, 64).sum(axis=1).astype(np.float32)
        q, s = oracle.screen_row(x, codes[row], scales[row], norms, dim)
        assert abs(exact - q) <= kappa * s, row


@pytest.fixture(scope="module")
def tie_head():
    vocab, dim = 3000, 768
    rng = Lcg(11)
    head = rng.take(vocab * dim, 0.05).reshape(vocab, dim)
    for dst, src in ((2000, 17), (2500, 17), (40, 1999)):
        head[dst] = head[src]
    return head, rng


def test_screened_argmax_equals_full_argmax_including_ties(tie_head):
    head, rng = tie_head
    vocab, dim = head.shape
    codes, scales, wmax, kappa = oracle.screen_build(head, vocab, dim)
    for trial in range(60):
        x = rng.take(dim, 3.0)
        if trial % 3 == 0:
            target = 17 if trial % 2 == 0 else 1999
            x = (head[target] * F32(40.0)).astype(np.float32)
        token, cand, _ = oracle.screen_select(x, head, codes, scales, vocab, dim, wmax, kappa)
        assert token is not None, trial
        assert cand >= 1
        assert token == full_argmax(x, head, vocab, dim), trial
        if trial % 3 == 0:
            # The planted ties: the first copy wins.
            assert token in (17, 40), (trial, token)


def test_nonfinite_or_degenerate_inputs_fall_back():
    vocab, dim = 2048, 64
    head = Lcg(3).take(vocab * dim).reshape(vocab, dim)
    codes, scales, wmax, kappa = oracle.screen_build(head, vocab, dim)
    x = np.full(dim, 0.5, dtype=np.float32)
    x[7] = np.nan
    assert oracle.screen_select(x, head, codes, scales, vocab, dim, wmax, kappa)[:2] == (None, 0)
    # All-zero input ties every row: past the candidate limit.
    zero = np.zeros(dim, dtype=np.float32)
    assert oracle.screen_select(zero, head, codes, scales, vocab, dim, wmax, kappa)[:2] == (None, oracle.SCREEN_LIMIT + 1)
    huge = np.full(dim, np.finfo(np.float32).max / 4, dtype=np.float32)
    assert oracle.screen_select(huge, head, codes, scales, vocab, dim, wmax, kappa)[0] is None


def test_bound_holds_for_every_row_and_token_is_the_full_argmax():
    # |L_v - q_v| <= B_v for the FP32 logit L_v of every row, and the token
    # is the full head's first-index argmax.
    vocab, dim = 512, 128
    rng = np.random.default_rng(7)
    head = rng.normal(0, 0.05, (vocab, dim)).astype(np.float32)
    codes, scales, wmax, kappa = oracle.screen_build(head, vocab, dim)
    x = rng.normal(0, 1, dim).astype(np.float32)
    token, cand, upper = oracle.screen_select(x, head, codes, scales, vocab, dim, wmax, kappa)
    ok, norms = oracle.screen_prepare(x, dim, wmax)
    assert ok and token is not None and 1 <= cand <= vocab
    logits = oracle.linear_decode(32, head, None, vocab, dim, 64, x, 1)[0]
    assert token == oracle.argmax(logits)
    for v in range(vocab):
        q, s = oracle.screen_row(x, codes[v], scales[v], norms, dim)
        bound = float(kappa) * float(s) + 2.0 ** -100
        assert abs(float(logits[v]) - q) <= bound * (1 + 1e-6), v
        assert upper[v] >= F32(q)
