"""BASELINE config 5 end to end, at its size: one INT8 decoder layer with the
checkpoint's shapes (dim 768, 16 query / 8 KV heads, FFN 2304) prefills 16,320
rows whose image interval is [0, 4096), then runs 64 greedy decode steps
until the cache holds 16,384 positions — Model::forward_layers for one layer
(src/model/mod.rs:513-691), fast mode's projections (the INT16 panels for the
prefill, src/model/mod.rs:956-1007; the INT8 decode GEMVs, mod.rs:421-492)
with the FP32 online prefill attention, over the compact FP32 cache
(Kv::Compact) and over sealed Q8 records (Kv::Q8, seal_layer,
src/model/cache.rs:218-276).

Every stage's output is compared whole against the oracle's composition of
the same steps:
  - prefill: the QKV projection, the queries, prefix keys and values bitwise;
    the attention within the FP32 tolerance; the layer output bitwise the
    oracle's WO / W13 / W2 steps over the layer's own attention output, and
    within 1e-4 of the oracle's whole composition;
  - Q8: the sealed records bitwise the oracle's seal of the same cache;
  - each decode step: the appended key and value bitwise (Q8: their records),
    the attention within the FP32 tolerance of the oracle over the same
    cache, the step output bitwise over the layer's own attention and within
    1e-4 of the oracle's composition.
"""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import assert_bitwise, host, max_rel, oracle_threads, to_dev

pytestmark = pytest.mark.gpu
H, G, DIM, FFN = 16, 8, 768, 2304
PREFIX, STEPS, IMAGE = 16320, 64, (0, 4096)


def close(got, want, tol=1e-5):
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= tol * (1.0 + np.abs(want))), float(np.max(np.abs(got - want)))
    assert max_rel(got, want) <= tol


def rope_table(rows, seed):
    # Paired temporal halves (the checkpoint's 2D RoPE), which the Q8 seal needs.
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-3.2, 3.2, size=(rows, H, 32))
    ang[:, 1::2, :16] = ang[:, 0::2, :16]
    return np.ascontiguousarray(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32))


def weights(seed):
    def q8(n, k, s):
        return gen.codes_uniform((n, k), -127, 127, np.int8, s), gen.uniform((n, k // 64), 1e-4, 4e-4, s + 1)
    return {"qkv": q8(H * 64 + 2 * G * 64, DIM, seed), "wo": q8(DIM, H * 64, seed + 2),
            "w13": q8(2 * FFN, DIM, seed + 4), "w2": q8(DIM, FFN, seed + 6)}


def after_attention_prefill(w, h, attn):
    """WO + residual, rms row scale, W13 + GLU, W2 + residual on the panels."""
    rows = h.shape[0]
    h = oracle.i16_gemm(attn.reshape(rows, -1), rows, H * 64, *w["wo"], DIM, epilogue=oracle.ADD, out=h)
    gated = oracle.i16_gemm(h, rows, DIM, *w["w13"], 2 * FFN, row_scale=oracle.row_scales(h, DIM),
                            epilogue=oracle.GLU)
    return oracle.i16_gemm(gated, rows, FFN, *w["w2"], DIM, epilogue=oracle.ADD, out=h)


def dec(w, name, x, glu=False):
    fn = oracle.linear_decode_glu if glu else oracle.linear_decode
    codes, scales = w[name]
    return fn(8, codes, scales, codes.shape[0], codes.shape[1], 64, x, x.shape[0])


def after_attention_decode(w, h, attn):
    h = h + dec(w, "wo", attn.reshape(h.shape[0], -1))
    gated = dec(w, "w13", h * oracle.row_scales(h, DIM)[:, None], glu=True)
    return h + dec(w, "w2", gated)


@pytest.mark.parametrize("kv_bits", [8, 32])
def test_config5_layer_prefill_then_64_decode_steps(kv_bits):
    import torch

    import focr_hip as fh

    oracle.set_threads(oracle_threads())
    w = weights(500)
    lins = {name: fh.QuantLinear(8, *w[name], 64) for name in w}
    sinks = gen.uniform(H, -2.0, 2.0, 501)
    layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], to_dev(sinks),
                            capacity=PREFIX + STEPS, projection=fh.PrefillProjection.I16, kv_bits=kv_bits)
    h0 = gen.normal((PREFIX, DIM), 1.0, 502)
    rope = rope_table(PREFIX, 503)
    h = to_dev(h0)
    print(f"config 5 kv_bits={kv_bits}: prefill of {PREFIX} rows", flush=True)
    layer.prefill(h, to_dev(rope), *IMAGE)
    torch.cuda.synchronize()

    # ---- prefill, stage by stage
    qkv = oracle.i16_gemm(h0, PREFIX, DIM, *w["qkv"], H * 64 + 2 * G * 64, row_scale=oracle.row_scales(h0, DIM))
    assert_bitwise(host(layer._buf("qkv", (PREFIX, qkv.shape[1]))), qkv, "QKV projection")
    q, pk, _, v = oracle.qkv_rows(qkv, PREFIX, rope, H, G, PREFIX)
    del qkv
    assert_bitwise(host(layer._buf("q", (PREFIX, H, 64))), q, "queries")
    assert_bitwise(host(layer.prefix_k[:PREFIX]), pk, "prefix keys")
    assert_bitwise(host(layer.v[:PREFIX]), v, "values")
    want_attn = oracle.attention_prefill_fast(q, pk, v, PREFIX, PREFIX, PREFIX, H, G, 0, *IMAGE, sinks)
    got_attn = host(layer._buf("attn", (PREFIX, H, 64)))
    close(got_attn, want_attn)
    got_h = host(h)
    assert_bitwise(got_h, after_attention_prefill(w, h0, got_attn), "prefill output over the layer's attention")
    assert max_rel(got_h, after_attention_prefill(w, h0, want_attn)) <= 1e-4
    del got_attn, want_attn, q

    # ---- the cache the decode steps attend over
    if kv_bits == 8:
        sealed = oracle.kv_seal(8, pk, v, PREFIX, H, G)
        assert not isinstance(sealed, int), sealed
        tail = oracle.kv_tail(8, G, STEPS)
        got = layer.split.dequantize()
        want = oracle.kv_dequantize(8, sealed, PREFIX, H, G, tail, STEPS, 0)
        assert_bitwise(host(got[0]), want[0], "sealed prefix keys")
        assert_bitwise(host(got[1]), want[1], "sealed values")
        pk, v = want[0], want[1]
        gk = np.zeros((0, G, 64), np.float32)
    else:
        gk = np.zeros((0, G, 64), np.float32)

    # ---- 64 greedy decode steps to 16,384 positions
    for step in range(STEPS):
        pos = PREFIX + step
        x0 = gen.normal((1, DIM), 1.0, 600 + step)
        rope_m = rope_table(1, 700 + step)
        x = to_dev(x0)
        layer.decode(x, to_dev(rope_m))
        torch.cuda.synchronize()
        qkv = dec(w, "qkv", x0 * oracle.row_scales(x0, DIM)[:, None])
        q, _, new_k, new_v = oracle.qkv_rows(qkv, 1, rope_m, H, G, 0)
        assert_bitwise(host(layer._buf("dq", (1, H, 64))), q, f"step {step} query")
        if kv_bits == 8:
            oracle.kv_push(8, new_k[0], new_v[0], G, STEPS, step, tail)
            got = layer.split.dequantize()
            _, vals, gk = oracle.kv_dequantize(8, sealed, PREFIX, H, G, tail, STEPS, step + 1)
            assert_bitwise(host(got[2]), gk, f"step {step} generated key records")
            assert_bitwise(host(got[1])[PREFIX:], vals[PREFIX:], f"step {step} value records")
            v = vals
        else:
            assert_bitwise(host(layer.generated_k[step:step + 1]), new_k, f"step {step} key")
            assert_bitwise(host(layer.v[pos:pos + 1]), new_v, f"step {step} value")
            gk = np.concatenate([gk, new_k])
            v = np.concatenate([v, new_v])
        # Fast mode's Q8 records decode with the fast exp (default_fast_exp).
        want_attn = oracle.attention_decode(q, pk, gk, v, 1, PREFIX, pos + 1, H, G, pos, *IMAGE, sinks,
                                            exp_fast=kv_bits == 8)
        got_attn = host(layer._buf("dattn", (1, H, 64)))
        close(got_attn, want_attn)
        got_x = host(x)
        assert_bitwise(got_x, after_attention_decode(w, x0, got_attn), f"step {step} output over its attention")
        assert max_rel(got_x, after_attention_decode(w, x0, want_attn)) <= 1e-4, step
    assert layer.len == PREFIX + STEPS == 16384
    layer.free()
    for lin in lins.values():
        lin.free()
