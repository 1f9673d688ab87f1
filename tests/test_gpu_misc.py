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
