"""Writes tests/golden/vectors.npz: the oracle's outputs (oracle/focr_oracle.c,
focr_kv.c and focr_screen.c, the C restatements of the reference's operators)
for small seeded inputs of every hot-path operator. The inputs are not stored: `vectors()` regenerates
them from the seeded generators of tests/gen.py, and the file keeps only the
keys listed in OUTPUTS. Committed so that the oracle's results are frozen
(tests/test_golden.py recomputes them bit for bit) and so that the GPU tests
compare the HIP library with fixed vectors (tests/test_gpu_golden.py).

Run from the repository root: python tests/golden/make_vectors.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
for p in (ROOT / "oracle", ROOT / "tests"):
    sys.path.insert(0, str(p))

import gen  # noqa: E402
import oracle  # noqa: E402

H, G = 16, 8


def vectors():
    v = {}
    # A1 / A4 / A5: decode GEMV, INT8 / INT16 codes and FP32 weights, 3 rows,
    # k with an 8-wide and a scalar tail (k % 32 = 13), exception columns.
    n, k, rows = 40, 237, 3
    x = gen.values(rows * k, 1, 2.0).reshape(rows, k)
    v["gemv_x"] = x
    for bits, lo, hi, dt in ((8, -127, 127, np.int8), (16, -32767, 32767, np.int16)):
        codes = gen.codes_uniform((n, k), lo, hi, dt, 2 + bits)
        codes[:, [5, 100]] = 0
        scales = gen.uniform((n, -(-k // 64)), 1e-4, 4e-4, 3 + bits)
        exc_cols = np.array([5, 100], np.int32)
        exc_vals = gen.values(n * 2, 4 + bits, 0.5).reshape(n, 2)
        v[f"gemv{bits}_codes"], v[f"gemv{bits}_scales"] = codes, scales
        v[f"gemv{bits}_exc_cols"], v[f"gemv{bits}_exc_vals"] = exc_cols, exc_vals
        v[f"gemv{bits}_out"] = oracle.linear_decode(bits, codes, scales, n, k, 64, x, rows, exc_cols, exc_vals)
        v[f"gemv{bits}_glu"] = oracle.linear_decode_glu(bits, codes, scales, n, k, 64, x, rows, exc_cols, exc_vals)
        v[f"dequant{bits}"] = oracle.dequantize(bits, codes, scales, n, k, 64, exc_cols, exc_vals)
    w = gen.values(n * k, 9, 0.1).reshape(n, k)
    v["gemv32_w"], v["gemv32_out"] = w, oracle.linear_decode(32, w, None, n, k, 32, x, rows)
    # A6: row scales (two widths with irregular trees).
    h = gen.values(5 * 768, 10, 3.0).reshape(5, 768)
    v["rms_h"], v["rms_out"] = h, oracle.row_scales(h, 768)
    # A2: FP32 panel GEMM with a row scale, Store / Glu / Add.
    m, k2, n2 = 19, 96, 48
    a = gen.values(m * k2, 11).reshape(m, k2)
    w2 = gen.matrix(n2 * k2, 12).reshape(n2, k2)
    rs = gen.uniform(m, 0.5, 1.5, 13)
    base = gen.values(m * n2, 14).reshape(m, n2)
    v["panel_a"], v["panel_w"], v["panel_rs"], v["panel_base"] = a, w2, rs, base
    v["panel_store"] = oracle.panel_gemm(a, m, k2, w2, n2, rs, oracle.STORE)
    v["panel_glu"] = oracle.panel_gemm(a, m, k2, w2, n2, rs, oracle.GLU)
    v["panel_add"] = oracle.panel_gemm(a, m, k2, w2, n2, None, oracle.ADD, out=base)
    # A3: INT16-activation x INT8-code GEMM (the reference's test generators).
    m3, k3, n3 = 41, 128, 64
    a3 = gen.i16_activations(m3, k3).reshape(m3, k3)
    c3, s3 = gen.i16_weights(n3, k3)
    v["i16_a"], v["i16_codes"], v["i16_scales"], v["i16_rs"] = a3, c3, s3, gen.uniform(m3, 0.5, 1.5, 15)
    v["i16_store"] = oracle.i16_gemm(a3, m3, k3, c3, s3, n3, row_scale=v["i16_rs"])
    v["i16_glu"] = oracle.i16_gemm(a3, m3, k3, c3, s3, n3, epilogue=oracle.GLU)
    # A7: FP32 prefill attention (online fast exp, static), 40 tokens, image [3, 33).
    L = 40
    q = gen.att_values(L * H * 64, 16, 3.0)
    kk = gen.att_values(L * H * 64, 17, 3.0)
    vv = gen.att_values(L * G * 64, 18, 3.0)
    sinks = gen.att_values(H, 19, 2.0)
    v["att_q"], v["att_k"], v["att_v"], v["att_sinks"] = q, kk, vv, sinks
    v["att_online"] = oracle.attention_prefill(q, kk, vv, L, L, L, H, G, 0, 3, 33, sinks)
    qn, kn = gen.normalized(L * H * 64, 20), gen.normalized(L * H * 64, 21)
    v["att_qn"], v["att_kn"] = qn, kn
    v["att_static"] = oracle.attention_prefill(qn, kn, vv, L, L, L, H, G, 0, 3, 33, sinks, static=True)
    # A8: BF16 prefill attention (online), same inputs.
    v["att_bf16"] = oracle.attention_prefill_bf16(q, kk, vv, L, H, G, 3, 33, sinks)
    # Decode attention: 2 rows over 61 prefix + 36 generated keys, image [1, 40).
    total, prefix, rows = 97, 61, 2
    v["dec_q"] = gen.att_values(rows * H * 64, 22, 0.75).reshape(rows, H, 64)
    v["dec_pk"] = gen.att_values(prefix * H * 64, 23, 0.75).reshape(prefix, H, 64)
    v["dec_gk"] = gen.att_values((total - prefix) * G * 64, 24, 0.75).reshape(-1, G, 64)
    v["dec_v"] = gen.att_values(total * G * 64, 25, 1.0).reshape(total, G, 64)
    v["dec_out"] = oracle.attention_decode(v["dec_q"], v["dec_pk"], v["dec_gk"], v["dec_v"], rows, prefix, total, H,
                                           G, total - rows, 1, 40, sinks)
    # QKV rows: 4 rows, the first 2 prefix rows.
    qkv = gen.values(4 * (H * 64 + 2 * G * 64), 26, 4.0).reshape(4, -1)
    ang = gen.uniform((4, H, 32), -3.2, 3.2, 27)
    rope = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    v["qkv_in"], v["qkv_rope"] = qkv, rope
    v["qkv_q"], v["qkv_pk"], v["qkv_gk"], v["qkv_v"] = oracle.qkv_rows(qkv, 4, rope, H, G, 2)
    # Sealed Q8 and Q16 KV records (Kv::Q8 / Kv::Q16): a 9-position prefix
    # whose GQA pairs share the temporal half, 3 generated positions (one
    # value block holding an infinity), decoded as the compact cache; decode
    # attention of 2 rows over the first two generated positions.
    P, T, cap = 9, 3, 16
    kp = gen.values(P * H * 64, 29, 2.0).reshape(P, H, 64)
    kp[:, 1::2, :32] = kp[:, 0::2, :32]
    vp = gen.values(P * G * 64, 30, 2.0).reshape(P, G, 64)
    tk = gen.values(T * G * 64, 31, 1.5).reshape(T, G, 64)
    tv = gen.values(T * G * 64, 32, 1.5).reshape(T, G, 64)
    tv[2, 4, 40] = np.inf
    v["kv_pk"], v["kv_v"], v["kv_tk"], v["kv_tv"] = kp, vp, tk, tv
    kq = gen.values(2 * H * 64, 33, 1.0).reshape(2, H, 64)
    v["kv_q"] = kq
    for bits in (8, 16):
        sealed = oracle.kv_seal(bits, kp, vp, P, H, G)
        tail = oracle.kv_tail(bits, G, cap - P)
        for i in range(T):
            oracle.kv_push(bits, tk[i], tv[i], G, cap - P, i, tail)
        dpk, dv, dgk = oracle.kv_dequantize(bits, sealed, P, H, G, tail, cap - P, T)
        v[f"kv{bits}_pk"], v[f"kv{bits}_v"], v[f"kv{bits}_gk"] = dpk, dv, dgk
        # Decode over the finite part of the cache: 2 rows at the first two
        # generated positions (the NaN block is in the third).
        v[f"kv{bits}_dec"] = oracle.attention_decode(kq, dpk, dgk[:2], dv[:P + 2], 2, P, P + 2, H, G, P, 0, 0,
                                                     v["att_sinks"])
    # The INT8 screen of a 512 x 128 FP32 head: codes, scales and constants,
    # and the exact greedy token of 2 inputs.
    head = gen.values(512 * 128, 34, 0.05).reshape(512, 128)
    sc_codes, sc_scales, sc_wmax, sc_kappa = oracle.screen_build(head, 512, 128)
    v["screen_head"], v["screen_codes"], v["screen_scales"] = head, sc_codes, sc_scales
    v["screen_consts"] = np.array([sc_wmax, sc_kappa], np.float32)
    sx = gen.values(2 * 128, 35, 1.0).reshape(2, 128)
    v["screen_x"] = sx
    v["screen_token"] = np.array([oracle.argmax(oracle.linear_decode(32, head, None, 512, 128, 32, sx[r:r + 1], 1)[0])
                                  for r in range(2)], np.int64)
    # A9: argmax over one row.
    logits = gen.values(1000, 28)
    v["argmax_logits"], v["argmax_token"] = logits, np.array([oracle.argmax(logits)], np.int64)
    return v


OUTPUTS = ("gemv8_out", "gemv8_glu", "dequant8", "gemv16_out", "gemv16_glu", "dequant16", "gemv32_out", "rms_out",
           "panel_store", "panel_glu", "panel_add", "i16_store", "i16_glu", "att_online", "att_static", "att_bf16",
           "dec_out", "qkv_q", "qkv_pk", "qkv_gk", "qkv_v", "argmax_token", "kv8_pk", "kv8_v", "kv8_gk", "kv8_dec",
           "kv16_pk", "kv16_v", "kv16_gk", "kv16_dec", "screen_codes", "screen_scales", "screen_consts",
           "screen_token")
FILE = Path(__file__).resolve().parent / "vectors.npz"

if __name__ == "__main__":
    v = vectors()
    np.savez_compressed(FILE, **{name: v[name] for name in OUTPUTS})
    out = FILE
    print(f"wrote {out} ({out.stat().st_size} bytes)")
