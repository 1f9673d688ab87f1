"""A packed model file uploaded to the GPU (focr_hip.packed.load_packed): the
mapped matrices, exception columns, sinks, FP32 head and INT8 screen on the
device compute bitwise what the same arrays uploaded directly compute, and a
decoder layer and the screened head run from the file's handles
(load_packed, src/model/packed.rs:190-310)."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import assert_bitwise, host, to_dev
from test_packed import small_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    from focr_hip import packed as pk

    parts = small_model(7, exceptions=True)
    parts["screen"] = oracle.screen_build(parts["output"], 65536, 768)
    path = tmp_path_factory.mktemp("gpu_packed") / "model.safetensors"
    pk.write_packed(path, **parts)
    model = pk.load_packed(path, verify=True)
    yield model, parts
    model.free()


def test_matrices_are_the_files_bytes(fh, packed):
    model, parts = packed
    assert len(model.layers) == 22 and model.profile.label() == "w8-body-kv-q8"
    x = gen.normal((3, 2304), 1.0, 80)
    for i in (0, 3, 21):
        for name, attr in zip(("attention.wqkv", "attention.wo", "feed_forward.w13", "feed_forward.w2"),
                              ("qkv", "wo", "w13", "w2")):
            src = parts["layers"][i][name]
            got = getattr(model.layers[i], attr)
            n, k = src["codes"].shape
            assert got.dimensions() == (n, k)
            xi = np.ascontiguousarray(x[:, :k])
            want = oracle.linear_decode(8, src["codes"], src["scales"], n, k, 64, xi, 3, src.get("exc_cols"),
                                        src.get("exc_vals"))
            assert_bitwise(host(got.linear(to_dev(xi), 3)), want, f"layer {i} {name}")
        assert_bitwise(host(model.layers[i].sinks), parts["layers"][i]["sinks"], "sinks")
    assert model.layers[3].w2.n_exc == 2


def test_screened_head_from_the_file(fh, packed):
    model, parts = packed
    assert model.screen.constants() == tuple(parts["screen"][2:])
    x = gen.normal((2, 768), 1.0, 81)
    logits = host(model.head.linear(to_dev(x), 2))
    want = oracle.linear_decode(32, parts["output"], None, 65536, 768, 32, x, 2)
    assert_bitwise(logits, want, "FP32 head")
    for (token, _), row in zip(model.screen.select(to_dev(x), 2, model.head), want):
        assert token is None or token == int(np.argmax(row))


def test_decoder_layer_from_the_file(fh, packed):
    # The file's layer 3 (with exception columns in W2) against the same
    # arrays uploaded directly: prefill and a decode step bitwise equal.
    import torch

    model, parts = packed
    L = model.layers[3]
    src = parts["layers"][3]
    direct = [fh.QuantLinear(8, src[n]["codes"], src[n]["scales"], 64, exc_cols=src[n].get("exc_cols"),
                             exc_vals=src[n].get("exc_vals"))
              for n in ("attention.wqkv", "attention.wo", "feed_forward.w13", "feed_forward.w2")]
    rows = 96
    ang = gen.uniform((rows + 1, 16, 32), -3.2, 3.2, 82)
    ang[:, 1::2, :16] = ang[:, 0::2, :16]
    rope = to_dev(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
    h0 = gen.normal((rows, 768), 1.0, 83)
    x0 = gen.normal((1, 768), 1.0, 84)
    outs = []
    for lins, sinks in (((L.qkv, L.wo, L.w13, L.w2), L.sinks), (direct, to_dev(src["sinks"]))):
        layer = fh.DecoderLayer(*lins, sinks, capacity=rows + 4, kv_bits=model.profile.kv_bits())
        h, x = to_dev(h0), to_dev(x0)
        layer.prefill(h, rope[:rows], 0, 48)
        layer.decode(x, rope[rows:rows + 1])
        torch.cuda.synchronize()
        outs.append((host(h), host(x)))
        layer.free()
    assert_bitwise(outs[0][0], outs[1][0], "prefill rows")
    assert_bitwise(outs[0][1], outs[1][1], "decode row")
    assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
    for d in direct:
        d.free()
