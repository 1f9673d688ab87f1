"""The screened vocabulary head on the GPU (focr_screen_*) against the oracle
and the full FP32 head: the token, the candidate count and the fallback of
every input are the oracle's, the bounds q + B of every vocabulary row are the
oracle's bit for bit, and every token is the full head's first-index argmax
(src/head_screen.rs:522-699 scenarios)."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import F32, to_dev
from test_oracle_screen import Lcg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def oracle_select(x, head, parts):
    codes, scales, wmax, kappa = parts
    vocab, dim = head.shape
    token, cand, _ = oracle.screen_select(x, head, codes, scales, vocab, dim, wmax, kappa)
    return token, cand


def assert_bounds_bitwise(screen, xs, head, parts, inputs=None):
    """q + B of every row for the inputs (all by default) of the last select,
    bit for bit."""
    codes, scales, wmax, kappa = parts
    vocab, dim = head.shape
    got = screen.bounds(len(xs))
    for r in range(len(xs)) if inputs is None else inputs:
        x = xs[r]
        want = oracle.screen_select(x, head, codes, scales, vocab, dim, wmax, kappa)[2]
        np.testing.assert_array_equal(got[r].view(np.uint32), want.view(np.uint32), err_msg=f"input {r}")


@pytest.fixture(scope="module")
def tie_case(fh):
    vocab, dim = 3000, 768
    rng = Lcg(11)
    head = rng.take(vocab * dim, 0.05).reshape(vocab, dim)
    for dst, src in ((2000, 17), (2500, 17), (40, 1999)):
        head[dst] = head[src]
    parts = oracle.screen_build(head, vocab, dim)
    screen = fh.ScreenedHead.build(head)
    lin = fh.Linear.from_f32(head)
    return head, rng, parts, screen, lin


def test_constants_are_the_oracle_build(fh, tie_case):
    head, _, parts, screen, _ = tie_case
    assert screen.constants() == (parts[2], parts[3])


def test_token_and_candidates_equal_the_oracle_and_the_full_argmax(fh, tie_case):
    head, rng, parts, screen, lin = tie_case
    vocab, dim = head.shape
    for trial in range(60):
        x = rng.take(dim, 3.0)
        if trial % 3 == 0:
            x = (head[17 if trial % 2 == 0 else 1999] * F32(40.0)).astype(np.float32)
        xd = to_dev(x)
        (token, cand), = screen.select(xd, 1, lin)
        want = oracle_select(x, head, parts)
        assert (token, cand) == want, trial
        logits = lin.linear(xd, 1)
        assert token == fh.argmax(logits, 1, vocab)[0], trial


def test_select_rows_equals_select_per_row(fh):
    vocab, dim = 2100, 768
    rng = Lcg(29)
    head = rng.take(vocab * dim, 0.05).reshape(vocab, dim)
    for dst, src in ((1500, 3), (900, 1200)):
        head[dst] = head[src]
    parts = oracle.screen_build(head, vocab, dim)
    screen = fh.ScreenedHead.from_parts(parts[0], parts[1], parts[2], parts[3])
    lin = fh.Linear.from_f32(head)
    for rows in range(1, 9):
        xs = rng.take(rows * dim, 3.0).reshape(rows, dim)
        xs[0] = head[3] * F32(40.0)
        if rows > 2:
            xs[2, 5] = np.nan
        joint = screen.select(to_dev(xs), rows, lin)
        finite = [r for r in range(rows) if np.isfinite(xs[r]).all()]
        assert_bounds_bitwise(screen, xs, head, parts, finite)
        for r in range(rows):
            single = screen.select(to_dev(xs[r]), 1, lin)[0]
            assert joint[r] == single == oracle_select(xs[r], head, parts), (rows, r)
        if rows > 2:
            assert joint[2] == (None, 0)


def test_nonfinite_or_degenerate_inputs_fall_back(fh):
    vocab, dim = 2048, 64
    head = Lcg(3).take(vocab * dim).reshape(vocab, dim)
    screen = fh.ScreenedHead.build(head)
    lin = fh.Linear.from_f32(head)
    x = np.full(dim, 0.5, dtype=np.float32)
    x[7] = np.nan
    assert screen.select(to_dev(x), 1, lin) == [(None, 0)]
    zero = np.zeros(dim, dtype=np.float32)
    assert screen.select(to_dev(zero), 1, lin) == [(None, fh.SCREEN_LIMIT + 1)]
    huge = np.full(dim, np.finfo(np.float32).max / 4, dtype=np.float32)
    assert screen.select(to_dev(huge), 1, lin)[0][0] is None


def test_build_and_upload_checks(fh):
    head = np.full((4, 64), 0.25, dtype=np.float32)
    head[1, 6] = np.inf
    with pytest.raises(fh.FocrError) as e:
        fh.ScreenedHead.build(head)
    assert e.value.code == -5
    with pytest.raises(fh.FocrError) as e:
        fh.ScreenedHead.build(np.ones((3, 100), np.float32))
    assert e.value.code == -2
    with pytest.raises(fh.FocrError) as e:
        fh.ScreenedHead.build(np.ones((3, 4096), np.float32))
    assert e.value.code == -3
    ok = np.ones((2, 64), np.float32)
    codes, scales, wmax, kappa = oracle.screen_build(ok, 2, 64)
    for bad in (0.0, 0.6, float("nan")):
        with pytest.raises(fh.FocrError):
            fh.ScreenedHead.from_parts(codes, scales, wmax, bad)


def test_vocabulary_head_at_checkpoint_size(fh):
    # The 65,536 x 768 head; activations as a final rms_norm leaves them.
    vocab, dim = 65536, 768
    head = gen.normal((vocab, dim), 0.02, 40)
    parts = oracle.screen_build(head, vocab, dim)
    screen = fh.ScreenedHead.build(head)
    lin = fh.Linear.from_f32(head)
    xs = gen.normal((4, dim), 1.0, 41)
    xs[3] = head[12345] * F32(60.0)
    got = screen.select(to_dev(xs), 4, lin)
    assert_bounds_bitwise(screen, xs, head, parts)
    logits = lin.linear(to_dev(xs), 4)
    full = fh.argmax(logits, 4, vocab)
    for r in range(4):
        assert got[r] == oracle_select(xs[r], head, parts), r
        assert got[r][0] == full[r], r
    assert got[3][0] == 12345


def test_odd_vocabulary_and_narrow_head(fh):
    # A vocabulary that is no multiple of the 16-row tiles or of 4, dim 128.
    vocab, dim = 1001, 128
    rng = np.random.default_rng(5)
    head = rng.normal(0, 0.05, (vocab, dim)).astype(np.float32)
    head[1000] = head[999]
    parts = oracle.screen_build(head, vocab, dim)
    screen = fh.ScreenedHead.build(head)
    lin = fh.Linear.from_f32(head)
    xs = rng.normal(0, 1, (3, dim)).astype(np.float32)
    xs[1] = head[999] * F32(30.0)
    got = screen.select(to_dev(xs), 3, lin)
    assert_bounds_bitwise(screen, xs, head, parts)
    for r in range(3):
        assert got[r] == oracle_select(xs[r], head, parts), r
    assert got[1][0] == 999
