"""The oracle against the committed fixtures (CPU only): the reference's own
known-answer vectors (tests/golden/kats.json, with their source file:line)
and the frozen oracle outputs of tests/golden/vectors.npz, recomputed bit
for bit."""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "kats.json").read_text())


def _f(values):
    return np.array([math.nan if v == "nan" else v for v in values], dtype=np.float32)


def test_rtn_w8_kat():
    kat = KATS["rtn_w8"]
    w = np.zeros(kat["in"], np.float32)
    w[:8] = kat["weights_head"]
    codes, scales = oracle.quantize_bits(w, kat["out"], kat["in"], kat["group"], 8)
    assert scales.ravel().tolist() == kat["scales"]
    assert codes.ravel()[:8].tolist() == kat["codes_head"]
    restored = oracle.dequantize(8, codes, scales, kat["out"], kat["in"], kat["group"])
    assert restored.ravel()[:8].tolist() == kat["dequantized_head"]
    assert np.all(restored.ravel()[8:] == 0.0)


def test_w8_validation_kat():
    for case in KATS["w8_validation"]["reject"]:
        assert oracle.validate_w8(1, 1, 64, case["codes"], _f(case["scales"])) != 0


def test_fp32_linear_kat():
    kat = KATS["fp32_linear"]
    out = oracle.linear_decode(32, _f(kat["weights"]), None, kat["out"], kat["in"], 32, _f(kat["input"]), kat["rows"])
    assert out.ravel().tolist() == kat["output"]


def test_i16_quantizer_kats():
    kat = KATS["i16_quantizer_ties"]
    x = np.zeros(64, np.float32)
    x[:4] = kat["x_head"]
    step, q = oracle.i16_quantize_group(x)
    assert float(step) == kat["step"] and q[:4].tolist() == kat["codes_head"]
    tiny = KATS["i16_quantizer_tiny_groups"]
    for absmax in list(np.float32(tiny["absmax"])) + [np.array([b], np.uint32).view(np.float32)[0]
                                                       for b in tiny["absmax_bits"]]:
        x = (absmax * (2.0 * np.arange(64, dtype=np.float32) / np.float32(63) - 1.0)).astype(np.float32)
        step, q = oracle.i16_quantize_group(x)
        assert 0.0 < float(step) < math.inf
        assert float(step) * 32767.0 >= float(absmax)
        assert np.any(q != 0)


def test_argmax_kat():
    kat = KATS["argmax"]
    assert oracle.argmax(kat["logits"]) == kat["token"]
    for bad in kat["reject"]:
        with pytest.raises(ValueError):
            oracle.argmax(_f(bad))


def test_oracle_reproduces_the_frozen_vectors():
    import sys

    sys.path.insert(0, str(GOLDEN))
    import make_vectors

    fresh = make_vectors.vectors()
    frozen = np.load(GOLDEN / "vectors.npz")
    assert sorted(frozen.files) == sorted(make_vectors.OUTPUTS)
    for name in make_vectors.OUTPUTS:
        a, b = np.asarray(fresh[name]), frozen[name]
        assert a.shape == b.shape, name
        if a.dtype.kind == "f":
            same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
            assert same.all(), name
        else:
            assert np.array_equal(a, b), name
