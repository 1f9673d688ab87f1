"""RMS row scales (bitwise) and greedy argmax on the GPU."""
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


@pytest.mark.parametrize("width", [768, 1024, 2304, 4096, 64, 96, 33, 1, 5000])
def test_row_scales_bitwise(fh, width):
    rows = 37
    h = gen.values(rows * width, 9) * F32(3.0)
    h[:width] = F32(1.0)  # closed form row
    got = host(fh.row_scales(to_dev(h), width))
    assert_bitwise(got, oracle.row_scales(h, width), f"width {width}")


def test_row_scales_extreme_rows(fh):
    # Rows whose squares underflow (subnormal and tiny values: the sum stays
    # at or near 0 and the scale at 1 / sqrt(eps)), overflow (|x| ~ 1e20: an
    # infinite sum, scale 0), a zero row, NaN and infinities: bitwise the
    # reference's sum_squares_pairwise and rms_scale (mod.rs:531-553).
    width = 768
    rows = [gen.values(width, 61 + r) for r in range(10)]
    rows[0] *= np.float32(1e-39)
    rows[1] *= np.float32(1e-20)
    rows[2] *= np.float32(1e20)
    rows[3][:] = 0.0
    rows[4][100] = np.nan
    rows[5][7] = np.inf
    rows[6][:] = np.float32(2.0 ** -149)
    rows[7] *= np.float32(3e-23)
    rows[8][::3] = np.float32(1.8e19)
    h = np.concatenate(rows).astype(np.float32)
    want = oracle.row_scales(h, width)
    assert want[3] == want[0] and want[2] == 0.0 and np.isnan(want[4]) and want[5] == 0.0
    assert_bitwise(host(fh.row_scales(to_dev(h), width)), want, "extreme rows")


def test_row_scales_full_prefill(fh):
    m, width = 6544, 768
    h = gen.normal((m, width), 1.0, 30)
    assert_bitwise(host(fh.row_scales(to_dev(h), width)), oracle.row_scales(h, width), "6544 rows")


def test_argmax(fh):
    # src/runner/mod.rs:946-949
    assert fh.argmax(to_dev(np.array([2.0, 3.0, 3.0], np.float32)), 1, 3) == [1]
    with pytest.raises(fh.FocrError, match="nonfinite"):
        fh.argmax(to_dev(np.array([math.nan], np.float32)), 1, 1)
    vocab = 65536
    logits = gen.normal((5, vocab), 1.0, 31)
    logits[2, 777] = logits[2, 9999] = np.float32(50.0)  # tie: first index wins
    got = fh.argmax(to_dev(logits), 5, vocab)
    assert got == [oracle.argmax(row) for row in logits]
    assert got[2] == 777
    logits[4, 12345] = np.inf
    with pytest.raises(fh.FocrError):
        fh.argmax(to_dev(logits), 5, vocab)


def test_argmax_unaligned_rows_and_ties(fh):
    # vocab 1001: rows after the first are not 16-byte aligned; ties inside one
    # thread's values, across threads and across waves; an all-equal row.
    vocab = 1001
    logits = gen.normal((4, vocab), 1.0, 32)
    logits[0, 5] = logits[0, 5 + 4096 % vocab] = logits[0, 900] = np.float32(9.0)
    logits[1, 1000] = logits[1, 999] = np.float32(9.0)
    logits[2, :] = np.float32(-3.5)
    logits[3, 64] = logits[3, 63] = np.float32(7.0)
    got = fh.argmax(to_dev(logits), 4, vocab)
    assert got == [oracle.argmax(row) for row in logits] == [5, 999, 0, 63]
    big = gen.normal((2, 70001), 1.0, 33)
    big[1, 65537] = big[1, 70000] = np.float32(40.0)
    assert fh.argmax(to_dev(big), 2, 70001) == [oracle.argmax(r) for r in big]


def test_argmax_ties_across_partial_workgroups(fh):
    # Rows are split into 2,048-logit partials combined per row: a tie across
    # a partial boundary, across distant partials and inside one, a maximum in
    # the ragged last partial, and many rows (one launch batch each 65,535).
    vocab = 3 * 2048 + 5
    logits = gen.normal((6, vocab), 1.0, 34)
    logits[0, 2047] = logits[0, 2048] = np.float32(9.0)
    logits[1, 6000] = logits[1, 100] = np.float32(9.0)
    logits[2, 4100] = logits[2, 4101] = np.float32(9.0)
    logits[3, vocab - 1] = np.float32(9.0)
    logits[4, :] = np.float32(0.25)
    logits[5, vocab - 5:] = np.float32(9.0)
    got = fh.argmax(to_dev(logits), 6, vocab)
    assert got == [oracle.argmax(row) for row in logits] == [2047, 100, 4100, vocab - 1, 0, vocab - 5]
    many = gen.normal((3000, 64), 1.0, 35)
    assert fh.argmax(to_dev(many), 3000, 64) == [int(np.argmax(r)) for r in many]
