"""The HIP library against the committed fixture vectors
(tests/golden/vectors.npz, the oracle's frozen outputs): bitwise for the
integer-exact and single-order operators, FP32 / BF16 tolerance for the
attention kernels."""
import sys
from pathlib import Path

import numpy as np
import pytest

from gpu_util import assert_bitwise, host, max_rel, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
H, G = 16, 8


@pytest.fixture(scope="module")
def case():
    sys.path.insert(0, str(GOLDEN))
    import make_vectors

    import focr_hip

    return focr_hip, make_vectors.vectors(), np.load(GOLDEN / "vectors.npz")


def test_gemv_and_dequant(case):
    fh, v, want = case
    x = to_dev(v["gemv_x"])
    rows, k = v["gemv_x"].shape
    for bits in (8, 16):
        lin = fh.QuantLinear(bits, v[f"gemv{bits}_codes"], v[f"gemv{bits}_scales"], 64,
                             exc_cols=v[f"gemv{bits}_exc_cols"], exc_vals=v[f"gemv{bits}_exc_vals"])
        assert_bitwise(host(lin.linear(x, rows)), want[f"gemv{bits}_out"], f"gemv{bits}")
        assert_bitwise(host(lin.linear_glu(x, rows)), want[f"gemv{bits}_glu"], f"glu{bits}")
        assert_bitwise(host(lin.dequantize()), want[f"dequant{bits}"], f"dequant{bits}")
        lin.free()
    lin = fh.Linear.from_f32(v["gemv32_w"])
    assert_bitwise(host(lin.linear(x, rows)), want["gemv32_out"], "gemv32")
    lin.free()


def test_row_scales(case):
    fh, v, want = case
    assert_bitwise(host(fh.row_scales(to_dev(v["rms_h"]), 768)), want["rms_out"], "rms")


def test_prefill_projections(case):
    fh, v, want = case
    m, k = v["panel_a"].shape
    lin = fh.Linear.from_f32(v["panel_w"])
    a, rs = to_dev(v["panel_a"]), to_dev(v["panel_rs"])
    chain = fh.PrefillProjection.F32_CHAIN
    assert_bitwise(host(lin.prefill(a, m, row_scale=rs, kernel=chain)), want["panel_store"], "store")
    assert_bitwise(host(lin.prefill(a, m, row_scale=rs, epilogue=fh.Epilogue.GLU, kernel=chain)), want["panel_glu"],
                   "glu")
    out = to_dev(v["panel_base"])
    lin.prefill(a, m, epilogue=fh.Epilogue.ADD, out=out, kernel=chain)
    assert_bitwise(host(out), want["panel_add"], "add")
    got = host(lin.prefill(a, m, row_scale=rs, kernel=fh.PrefillProjection.F32_MFMA))
    assert max_rel(got, want["panel_store"]) <= 1e-5
    lin.free()
    m3, k3 = v["i16_a"].shape
    lin = fh.QuantLinear(8, v["i16_codes"], v["i16_scales"], 64)
    a3 = to_dev(v["i16_a"])
    i16 = fh.PrefillProjection.I16
    assert_bitwise(host(lin.prefill(a3, m3, row_scale=to_dev(v["i16_rs"]), kernel=i16)), want["i16_store"], "i16")
    assert_bitwise(host(lin.prefill(a3, m3, epilogue=fh.Epilogue.GLU, kernel=i16)), want["i16_glu"], "i16 glu")
    lin.free()


def close(got, want, tol):
    assert np.all(np.abs(got - want) <= tol * (1.0 + np.abs(want)))


def test_attention(case):
    fh, v, want = case
    L = 40
    kv = fh.CompactKv.prefill(to_dev(v["att_k"]), to_dev(v["att_v"]), L, H, G)
    geo = fh.Geometry(0, 3, 33)
    got = host(fh.attention_with(to_dev(v["att_q"]), kv, L, geo, to_dev(v["att_sinks"])))
    close(got.reshape(want["att_online"].shape), want["att_online"], 1e-5)
    kvn = fh.CompactKv.prefill(to_dev(v["att_kn"]), to_dev(v["att_v"]), L, H, G)
    got = host(fh.attention_with(to_dev(v["att_qn"]), kvn, L, geo, to_dev(v["att_sinks"]),
                                 fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC)))
    close(got.reshape(want["att_static"].shape), want["att_static"], 1e-5)
    out = to_dev(np.zeros(L * H * 64, np.float32))
    assert fh.attention_prefill_bf16(to_dev(v["att_q"]), kv, L, geo, to_dev(v["att_sinks"]), out,
                                     fh.PrefillOptions(softmax=fh.Softmax.ONLINE))
    # The BF16 bar: max|d| / max|ref| <= 2e-3 (as tests/test_gpu_attention_bf16.py).
    assert max_rel(host(out).reshape(want["att_bf16"].shape), want["att_bf16"]) <= 2e-3


def test_decode_attention_and_qkv_rows(case):
    fh, v, want = case
    total, prefix, rows = 97, 61, 2
    kv = fh.CompactKv(to_dev(v["dec_pk"]), to_dev(v["dec_gk"]), to_dev(v["dec_v"]), prefix, total, H, G, 64)
    got = host(fh.attention_decode(to_dev(v["dec_q"]), kv, rows, fh.Geometry(total - rows, 1, 40),
                                   to_dev(v["att_sinks"])))
    close(got, want["dec_out"], 1e-5)
    import torch

    pk = torch.empty((2, H, 64), device="cuda")
    gk = torch.empty((2, G, 64), device="cuda")
    vv = torch.empty((4, G, 64), device="cuda")
    q = fh.qkv_rows(to_dev(v["qkv_in"]), 4, to_dev(v["qkv_rope"]), H, G, 2, prefix_k=pk, generated_k=gk, v=vv)
    for name, t in (("qkv_q", q), ("qkv_pk", pk), ("qkv_gk", gk), ("qkv_v", vv)):
        assert_bitwise(host(t), want[name], name)


def test_argmax(case):
    fh, v, want = case
    logits = v["argmax_logits"]
    assert fh.argmax(to_dev(logits), 1, logits.size) == [int(want["argmax_token"][0])]


@pytest.mark.parametrize("bits", [8, 16])
def test_sealed_kv_records(case, bits):
    # Seal, append (one block holding an infinity decodes to NaN), the decoded
    # records bit for bit, and decode attention over them within FP32 rounding.
    fh, v, want = case
    P, T, cap = 9, 3, 16
    kv = fh.KvSplit.seal(bits, to_dev(v["kv_pk"]), to_dev(v["kv_v"]), P, cap, H, G)
    kv.append(to_dev(v["kv_tk"][:2]), to_dev(v["kv_tv"][:2]), 2)
    got = host(kv.attention_decode(to_dev(v["kv_q"]), 2, to_dev(v["att_sinks"])))
    close(got, want[f"kv{bits}_dec"], 1e-5)
    kv.append(to_dev(v["kv_tk"][2:]), to_dev(v["kv_tv"][2:]), T - 2)
    pk, vals, gk = (host(t) for t in kv.dequantize())
    assert_bitwise(pk, want[f"kv{bits}_pk"], "prefix keys")
    assert_bitwise(vals, want[f"kv{bits}_v"], "values")
    assert_bitwise(gk, want[f"kv{bits}_gk"], "generated keys")
    kv.free()


def test_screened_head(case):
    fh, v, want = case
    wmax, kappa = (float(c) for c in want["screen_consts"])
    built = fh.ScreenedHead.build(v["screen_head"])
    assert built.constants() == (wmax, kappa)
    stored = fh.ScreenedHead.from_parts(want["screen_codes"], want["screen_scales"], wmax, kappa)
    head = fh.Linear.from_f32(v["screen_head"])
    for screen in (built, stored):
        picks = screen.select(to_dev(v["screen_x"]), 2, head)
        assert [tok for tok, _ in picks] == [int(t) for t in want["screen_token"]]
        screen.free()
    head.free()
