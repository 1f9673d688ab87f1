"""The decode step's operators and one whole decoder layer on the GPU against
the oracle: the QKV row step (bitwise), the decode GEMV with the rms row
scale and residual folded in (bitwise), decode attention (FP32 tolerance),
and DecoderLayer's prefill and decode steps (Model::forward_layers for one
layer, src/model/mod.rs:513-691)."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import assert_bitwise, host, max_rel, to_dev

pytestmark = pytest.mark.gpu
H, G = 16, 8


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    oracle.set_threads(8)
    return focr_hip


def rope_table(rows, seed, paired=False):
    """[rows][H][32] (cos, sin) pairs; `paired`: the temporal pairs 0..16 of
    both heads of a GQA pair agree, as the checkpoint's 2D RoPE makes them (the
    sealed cache stores that half once per pair and refuses otherwise)."""
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-3.2, 3.2, size=(rows, H, 32))
    if paired:
        ang[:, 1::2, :16] = ang[:, 0::2, :16]
    return np.ascontiguousarray(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32))


@pytest.mark.parametrize("rows,prefix_rows", [(1, 0), (5, 0), (8, 3), (300, 300), (257, 250)])
def test_qkv_rows_bitwise(fh, rows, prefix_rows):
    import torch

    x = gen.values(rows * (H * 64 + 2 * G * 64), 100 + rows, 4.0).reshape(rows, -1)
    x[0, 3], x[0, 70], x[0, 200] = 0.0, 1e-30, 3e4
    if rows > 2:
        x[2, 64:128] = 0.0  # an all-zero head: scale 1/sqrt(eps)
    rope = rope_table(rows, rows)
    want_q, want_pk, want_gk, want_v = oracle.qkv_rows(x, rows, rope, H, G, prefix_rows)
    dev = torch.device("cuda:0")
    pk = torch.full((max(prefix_rows, 1), H, 64), float("nan"), device=dev)
    gk = torch.full((max(rows - prefix_rows, 1), G, 64), float("nan"), device=dev)
    v = torch.full((rows, G, 64), float("nan"), device=dev)
    q = fh.qkv_rows(to_dev(x), rows, to_dev(rope), H, G, prefix_rows, prefix_k=pk, generated_k=gk, v=v)
    assert_bitwise(host(q), want_q, "q")
    assert_bitwise(host(pk)[:prefix_rows], want_pk, "prefix keys")
    assert_bitwise(host(gk)[:rows - prefix_rows], want_gk, "generated keys")
    assert_bitwise(host(v), want_v, "values")


@pytest.mark.parametrize("bits", [8, 16, 32])
@pytest.mark.parametrize("rows", [1, 3, 8])
def test_decode_ex_folds_row_scale_and_residual(fh, bits, rows):
    n, k = 192, 768
    if bits == 32:
        codes, scales = gen.normal((n, k), 0.02, 5), None
    else:
        lo, hi = (-127, 127) if bits == 8 else (-32767, 32767)
        codes = gen.codes_uniform((n, k), lo, hi, np.int8 if bits == 8 else np.int16, 5)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 6)
    lin = fh.Linear(bits, codes, scales, 64)
    h = gen.normal((rows, k), 1.0, 7)
    rs = oracle.row_scales(h, k)
    normalized = h * rs[:, None]  # rms_norm_row: x * scale, one rounding
    got_rs = host(fh.row_scales(to_dev(h), k))
    assert_bitwise(got_rs, rs, "row scales")
    # STORE with the row scale == linear(rms_norm(h)).
    got = host(lin.linear_ex(to_dev(h), rows, row_scale=to_dev(rs)))
    want = oracle.linear_decode(bits, codes, scales, n, k, 64, normalized, rows)
    assert_bitwise(got, want, "store")
    # ADD: residual + linear(x).
    base = gen.normal((rows, n), 1.0, 8)
    out = to_dev(base)
    lin.linear_ex(to_dev(h), rows, epilogue=fh.Epilogue.ADD, out=out)
    assert_bitwise(host(out), base + oracle.linear_decode(bits, codes, scales, n, k, 64, h, rows), "add")
    # GLU with the row scale == linear_glu(rms_norm(h)).
    got = host(lin.linear_ex(to_dev(h), rows, row_scale=to_dev(rs), epilogue=fh.Epilogue.GLU))
    want = oracle.linear_decode_glu(bits, codes, scales, n, k, 64, normalized, rows)
    assert_bitwise(got, want, "glu")
    lin.free()


@pytest.mark.parametrize("bits", [8, 16, 32])
@pytest.mark.parametrize("rows", [1, 2, 5, 8])
@pytest.mark.parametrize("k", [768, 1024])
def test_decode_ex_rms_norm_in_kernel(fh, bits, rows, k):
    # rms_norm(h) then linear / linear_glu (model/mod.rs:421-492): in the GEMV
    # for the model width 768, through focr_row_scales for other widths.
    n = 256
    if bits == 32:
        codes, scales = gen.normal((n, k), 0.02, 15), None
    else:
        lo, hi = (-127, 127) if bits == 8 else (-32767, 32767)
        codes = gen.codes_uniform((n, k), lo, hi, np.int8 if bits == 8 else np.int16, 15)
        scales = gen.uniform((n, k // 64), 1e-4, 4e-4, 16)
    lin = fh.Linear(bits, codes, scales, 64)
    h = gen.normal((rows, k), 3.0, 17)
    h[0, :64] = 0.0
    normalized = h * oracle.row_scales(h, k)[:, None]
    got = host(lin.linear_ex(to_dev(h), rows, rms_norm=True))
    assert_bitwise(got, oracle.linear_decode(bits, codes, scales, n, k, 64, normalized, rows), "rms store")
    got = host(lin.linear_ex(to_dev(h), rows, rms_norm=True, epilogue=fh.Epilogue.GLU))
    assert_bitwise(got, oracle.linear_decode_glu(bits, codes, scales, n, k, 64, normalized, rows), "rms glu")
    lin.free()


def close(got, want, tol=1e-5):
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= tol * (1.0 + np.abs(want))), float(np.max(np.abs(got - want)))
    assert max_rel(got, want) <= tol


def decode_inputs(total, prefix, rows, seed, n_kv=G, scale=0.75):
    q = gen.att_values(rows * H * 64, 41 + seed, scale).reshape(rows, H, 64)
    pk = gen.att_values(max(prefix, 1) * H * 64, 53 + seed, scale).reshape(-1, H, 64)[:prefix]
    gk = gen.att_values(max(total - prefix, 1) * n_kv * 64, 67 + seed, scale).reshape(-1, n_kv, 64)[:total - prefix]
    v = gen.att_values(total * n_kv * 64, 79 + seed, 1.0).reshape(total, n_kv, 64)
    sinks = np.array([[-1000.0, 1000.0, 0.0, 2.25][h % 4] for h in range(H)], np.float32)
    return q, pk, gk, v, sinks


def run_decode(fh, q, pk, gk, v, sinks, rows, prefix, total, offset, image, n_kv=G):
    kv = fh.CompactKv(to_dev(pk) if prefix else None, to_dev(gk) if total > prefix else None, to_dev(v), prefix,
                      total, H, n_kv, 64)
    out = fh.attention_decode(to_dev(q), kv, rows, fh.Geometry(offset, *image), to_dev(sinks))
    return host(out)


@pytest.mark.parametrize("prefix_len,tail", [(1, 0), (64, 0), (700, 2), (16320, 5)])
def test_decode_row_compact_is_bitwise_the_two_calls(fh, prefix_len, tail):
    # focr_attention_decode_row = focr_qkv_rows (one generated row) +
    # focr_attention_decode (query_len 1 at that row), bit for bit: query,
    # output and the key and value rows it appends, over three steps (the
    # third with an infinite value input, NaN in group 3's output dims).
    import torch

    dev = torch.device("cuda:0")
    cap = prefix_len + tail + 3
    image = (0, min(prefix_len, 256))
    pk = gen.normal((prefix_len, H, 64), 1.0, 71)
    gk = np.full((cap - prefix_len, G, 64), np.nan, np.float32)
    gk[:tail] = gen.normal((tail, G, 64), 1.0, 72) if tail else gk[:0]
    v = np.full((cap, G, 64), np.nan, np.float32)
    v[:prefix_len + tail] = gen.normal((prefix_len + tail, G, 64), 1.0, 73)
    caches = [(to_dev(pk), to_dev(gk), to_dev(v)) for _ in range(2)]
    sinks = to_dev(gen.uniform(H, -2.0, 2.0, 74))
    width = H * 64 + 2 * G * 64
    for step in range(3):
        pos = prefix_len + tail + step
        total = pos + 1
        qkv = gen.normal((1, width), 2.0, 75 + step)
        if step == 2:
            qkv[0, H * 64 + G * 64 + 3 * 64 + 7] = np.inf
        rope = to_dev(rope_table(1, 80 + step))
        (pk2, gk2, v2), (pk1, gk1, v1) = caches
        q2 = fh.qkv_rows(to_dev(qkv), 1, rope, H, G, 0, generated_k=gk2[pos - prefix_len: pos - prefix_len + 1],
                         v=v2[pos: pos + 1])
        kv2 = fh.CompactKv(pk2, gk2[: total - prefix_len], v2[:total], prefix_len, total, H, G, 64)
        out2 = fh.attention_decode(q2, kv2, 1, fh.Geometry(pos, *image), sinks)
        q1 = torch.empty_like(q2)
        kv1 = fh.CompactKv(pk1, gk1[: total - prefix_len], v1[:total], prefix_len, total, H, G, 64)
        out1 = fh.attention_decode_row(to_dev(qkv), rope, kv1, *image, sinks, q=q1)
        assert_bitwise(host(q1), host(q2), f"step {step} query")
        assert_bitwise(host(out1), host(out2), f"step {step} output")
        assert_bitwise(host(gk1), host(gk2), f"step {step} generated keys")
        assert_bitwise(host(v1), host(v2), f"step {step} values")
        o = host(out1)[0]
        if step < 2:
            assert np.all(np.isfinite(o))
        else:  # heads 6 and 7 read group 3's values: dim 7 not finite, every other output finite
            assert not np.any(np.isfinite(o[6:8, 7]))
            assert np.all(np.isfinite(o[:6])) and np.all(np.isfinite(o[8:])) and np.all(np.isfinite(o[6:8, :7]))
    # A row inside the prefix is not a generated row: a shape error, nothing launched.
    with pytest.raises(fh.FocrError):
        fh.attention_decode_row(to_dev(gen.normal((1, width), 1.0, 79)), rope,
                                fh.CompactKv(pk1, None, v1[:prefix_len], prefix_len, prefix_len, H, G, 64), 0, 0,
                                sinks)


# The reference's decode cases (decode64.rs tests): causal tile tails, image and
# generated boundaries, compact crossovers, GQA repeats, full-page and full-context.
CAUSAL = [1, 2, 17, 63, 64, 127, 128, 129, 143, 144, 161, 255, 256, 257, 1025]
COMPACT = [(t, p) for t in (1, 17, 127, 128, 129, 257) for p in (0, t // 2, t)]


@pytest.mark.parametrize("kv_len", CAUSAL)
def test_decode_causal_tails(fh, kv_len):
    q, pk, gk, v, sinks = decode_inputs(kv_len, kv_len, 1, kv_len)
    got = run_decode(fh, q, pk, gk, v, sinks, 1, kv_len, kv_len, kv_len - 1, (0, 0))
    close(got, oracle.attention_decode(q, pk, gk, v, 1, kv_len, kv_len, H, G, kv_len - 1, 0, 0, sinks))


@pytest.mark.parametrize("total,prefix", COMPACT)
def test_decode_compact_crossovers(fh, total, prefix):
    q, pk, gk, v, sinks = decode_inputs(total, prefix, 1, total + prefix)
    got = run_decode(fh, q, pk, gk, v, sinks, 1, prefix, total, total - 1, (0, 0))
    close(got, oracle.attention_decode(q, pk, gk, v, 1, prefix, total, H, G, total - 1, 0, 0, sinks))


@pytest.mark.parametrize("offset", [0, 1, 126, 127, 128, 129, 160])
def test_decode_image_and_generated_boundaries(fh, offset):
    total, prefix, image = 161, 129, (1, 128)
    q, pk, gk, v, sinks = decode_inputs(total, prefix, 1, offset)
    got = run_decode(fh, q, pk, gk, v, sinks, 1, prefix, total, offset, image)
    close(got, oracle.attention_decode(q, pk, gk, v, 1, prefix, total, H, G, offset, *image, sinks))


@pytest.mark.parametrize("rows", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("n_kv", [4, 8, 16])
def test_decode_verify_rows_and_gqa(fh, rows, n_kv):
    total, prefix, image = 300, 257, (1, 200)
    q, pk, gk, v, sinks = decode_inputs(total, prefix, rows, rows * n_kv, n_kv=n_kv)
    got = run_decode(fh, q, pk, gk, v, sinks, rows, prefix, total, total - rows, image, n_kv=n_kv)
    close(got, oracle.attention_decode(q, pk, gk, v, rows, prefix, total, H, n_kv, total - rows, *image, sinks))


@pytest.mark.parametrize("total,prefix", [(6544, 6544), (6545, 6544), (16384, 6544), (16384, 16320)])
def test_decode_full_page_and_context(fh, total, prefix):
    q, pk, gk, v, sinks = decode_inputs(total, prefix, 1, 3)
    got = run_decode(fh, q, pk, gk, v, sinks, 1, prefix, total, total - 1, (1, 4096))
    close(got, oracle.attention_decode(q, pk, gk, v, 1, prefix, total, H, G, total - 1, 1, 4096, sinks))


def test_decode_extreme_logits(fh):
    total, prefix = 257, 129
    q, pk, gk, v, sinks = decode_inputs(total, prefix, 1, 9, scale=100.0)
    v = v * np.float32(1e8)
    got = run_decode(fh, q, pk, gk, v, sinks, 1, prefix, total, total - 1, (1, 129))
    want = oracle.attention_decode(q, pk, gk, v, 1, prefix, total, H, G, total - 1, 1, 129, sinks)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 1e-5


# ---- one decoder layer (BASELINE config 5 in miniature) ----------------------
DIM, FFN = 768, 2304


def layer_weights(seed):
    def q8(n, k, s):
        return gen.codes_uniform((n, k), -127, 127, np.int8, s), gen.uniform((n, k // 64), 1e-4, 4e-4, s + 1)
    return {"qkv": q8(H * 64 + 2 * G * 64, DIM, seed), "wo": q8(DIM, H * 64, seed + 2),
            "w13": q8(2 * FFN, DIM, seed + 4), "w2": q8(DIM, FFN, seed + 6)}


def oracle_layer_prefill(w, h, rope, image, sinks):
    """Model::forward_layers' panel path for one layer (model/mod.rs:956-1007)."""
    rows = h.shape[0]
    h = h.copy()
    rs = oracle.row_scales(h, DIM)
    qkv = oracle.i16_gemm(h, rows, DIM, *w["qkv"], w["qkv"][0].shape[0], row_scale=rs)
    q, pk, _, v = oracle.qkv_rows(qkv, rows, rope, H, G, rows)
    attn = oracle.attention_prefill(q, pk, v, rows, rows, rows, H, G, 0, image[0], image[1], sinks)
    h = oracle.i16_gemm(attn.reshape(rows, -1), rows, H * 64, *w["wo"], DIM, epilogue=oracle.ADD, out=h)
    rs = oracle.row_scales(h, DIM)
    gated = oracle.i16_gemm(h, rows, DIM, *w["w13"], 2 * FFN, row_scale=rs, epilogue=oracle.GLU)
    h = oracle.i16_gemm(gated, rows, FFN, *w["w2"], DIM, epilogue=oracle.ADD, out=h)
    return h, q, pk, v, attn


def oracle_layer_decode(w, h, rope, cache, image, sinks):
    """project_qkv + attention_out_ffn for 1..=8 rows (model/mod.rs:421-492)."""
    rows = h.shape[0]
    pk, gk, v, prefix = cache["pk"], cache["gk"], cache["v"], cache["prefix"]
    pos = v.shape[0]
    dec = lambda name, x, glu=False: (oracle.linear_decode_glu if glu else oracle.linear_decode)(
        8, *w[name], w[name][0].shape[0], w[name][0].shape[1], 64, x, rows)
    normalized = h * oracle.row_scales(h, DIM)[:, None]
    qkv = dec("qkv", normalized)
    q, _, new_k, new_v = oracle.qkv_rows(qkv, rows, rope, H, G, 0)
    gk = np.concatenate([gk, new_k]) if gk is not None else new_k
    v = np.concatenate([v, new_v])
    cache.update(gk=gk, v=v)
    attn = oracle.attention_decode(q, pk, gk, v, rows, prefix, pos + rows, H, G, pos, image[0], image[1], sinks)
    h = h + dec("wo", attn.reshape(rows, -1))
    normalized = h * oracle.row_scales(h, DIM)[:, None]
    gated = dec("w13", normalized, glu=True)
    h = h + dec("w2", gated)
    return h, q, new_k, new_v, attn


def test_decoder_layer_prefill_and_decode(fh):
    import torch

    rows, image = 300, (0, 200)
    w = layer_weights(40)
    lins = {name: fh.QuantLinear(8, *w[name], 64) for name in w}
    sinks = gen.uniform(H, -2.0, 2.0, 47)
    layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], to_dev(sinks), capacity=rows + 16)
    h0 = gen.normal((rows, DIM), 1.0, 48)
    rope = rope_table(rows, 49)
    h = to_dev(h0)
    layer.prefill(h, to_dev(rope), *image)
    want_h, want_q, want_pk, want_v, want_attn = oracle_layer_prefill(w, h0, rope, image, sinks)
    torch.cuda.synchronize()
    # Everything before attention is bitwise; attention and after within tolerance.
    assert_bitwise(host(layer.prefix_k[:rows]), want_pk, "prefix keys")
    assert_bitwise(host(layer.v[:rows]), want_v, "values")
    close(host(layer._buf("attn", (rows, H, 64))), want_attn)
    assert max_rel(host(h), want_h) <= 1e-4
    cache = {"pk": want_pk, "gk": None, "v": want_v, "prefix": rows}
    for step, m in enumerate([1, 1, 5, 8]):
        x0 = gen.normal((m, DIM), 1.0, 60 + step)
        rope_m = rope_table(m, 70 + step)
        x = to_dev(x0)
        pos = layer.len
        layer.decode(x, to_dev(rope_m))
        want_x, _, new_k, new_v, want_attn = oracle_layer_decode(w, x0, rope_m, cache, image, sinks)
        assert_bitwise(host(layer.generated_k[pos - rows: pos - rows + m]), new_k, f"step {step} keys")
        assert_bitwise(host(layer.v[pos: pos + m]), new_v, f"step {step} values")
        close(host(layer._buf("dattn", (m, H, 64))), want_attn)
        assert max_rel(host(x), want_x) <= 1e-4, step
    for lin in lins.values():
        lin.free()


@pytest.mark.parametrize("rows", [1, 3, 5, 8])
def test_decoder_layer_short_prefill_takes_the_decode_path(fh, rows):
    """A prompt of at most 8 rows is not a panel prefill (`panel = rows > 8`,
    model/mod.rs:568): project_qkv / attention_out_ffn run the FP32 decode
    GEMVs with the separate rms_norm passes, and the attention is the online
    FP32 one whatever the plan's BF16 or static choice
    (PrefillPlan::softmaxes(false), kernels/mod.rs:148-153). Everything before
    the attention is bitwise the oracle; the attention within the FP32
    tolerance; the layer output within 1e-4 (it carries the attention's)."""
    import torch

    image = (0, max(rows - 1, 0))
    w = layer_weights(90 + rows)
    lins = {name: fh.QuantLinear(8, *w[name], 64) for name in w}
    sinks = gen.uniform(H, -2.0, 2.0, 91)
    opts = fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC, softmax=fh.Softmax.STATIC)
    layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], to_dev(sinks), capacity=rows + 2,
                            options=opts, bf16_attention=True)
    h0 = gen.normal((rows, DIM), 1.0, 92)
    rope = rope_table(rows, 93)
    h = to_dev(h0)
    layer.prefill(h, to_dev(rope), *image)
    torch.cuda.synchronize()
    dec = lambda name, x, glu=False: (oracle.linear_decode_glu if glu else oracle.linear_decode)(
        8, *w[name], w[name][0].shape[0], w[name][0].shape[1], 64, x, rows)
    qkv = dec("qkv", h0 * oracle.row_scales(h0, DIM)[:, None])
    q, pk, _, v = oracle.qkv_rows(qkv, rows, rope, H, G, rows)
    assert_bitwise(host(layer._buf("qkv", (rows, qkv.shape[1]))), qkv, "qkv GEMV")
    assert_bitwise(host(layer.prefix_k[:rows]), pk, "prefix keys")
    assert_bitwise(host(layer.v[:rows]), v, "values")
    if rows >= 4:  # the prefill tiles (attention/mod.rs:271-299), online softmax
        want_attn = oracle.attention_prefill(q, pk, v, rows, rows, rows, H, G, 0, *image, sinks)
    else:  # decode64 / online::attention
        want_attn = oracle.attention_decode(q, pk, None, v, rows, rows, rows, H, G, 0, *image, sinks)
    close(host(layer._buf("attn", (rows, H, 64))), want_attn)
    want_h = h0 + dec("wo", want_attn.reshape(rows, -1))
    gated = dec("w13", want_h * oracle.row_scales(want_h, DIM)[:, None], glu=True)
    want_h = want_h + dec("w2", gated)
    assert max_rel(host(h), want_h) <= 1e-4
    # The layer output is bitwise the decode path's on the layer's own attention.
    attn = host(layer._buf("attn", (rows, H, 64))).reshape(rows, -1)
    exact = h0 + dec("wo", attn)
    exact = exact + dec("w2", dec("w13", exact * oracle.row_scales(exact, DIM)[:, None], glu=True))
    assert_bitwise(host(h), exact, "layer output over the layer's attention")
    for lin in lins.values():
        lin.free()


@pytest.mark.parametrize("bits", [8, 16])
def test_decoder_layer_over_the_sealed_cache(fh, bits):
    """Kv::Q8 / Kv::Q16: the prefill seals the prefix after its attention
    (seal_layer, model/cache.rs:218-276); decode appends to the tail and
    attends over the records; a truncation drops rejected drafts
    (Session::truncate, model/cache.rs:281-298). The oracle runs the same
    steps over the oracle's decoded records."""
    import torch

    rows, image, cap = 200, (0, 120), 220
    w = layer_weights(50)
    lins = {name: fh.QuantLinear(8, *w[name], 64) for name in w}
    sinks = gen.uniform(H, -2.0, 2.0, 51)
    layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], to_dev(sinks), capacity=cap,
                            kv_bits=bits)
    h0 = gen.normal((rows, DIM), 1.0, 52)
    rope = rope_table(rows, 53, paired=True)
    h = to_dev(h0)
    layer.prefill(h, to_dev(rope), *image)
    want_h, _, want_pk, want_v, _ = oracle_layer_prefill(w, h0, rope, image, sinks)
    torch.cuda.synchronize()
    assert max_rel(host(h), want_h) <= 1e-4
    sealed = oracle.kv_seal(bits, want_pk, want_v, rows, H, G)
    assert not isinstance(sealed, int), sealed
    tail = oracle.kv_tail(bits, G, cap - rows)
    tail_len = 0
    assert layer.split.info()[:4] == (bits, rows, 0, cap)
    dec = lambda name, x, m, glu=False: (oracle.linear_decode_glu if glu else oracle.linear_decode)(
        8, *w[name], w[name][0].shape[0], w[name][0].shape[1], 64, x, m)
    for step, (m, drop) in enumerate([(1, 0), (5, 3), (1, 0), (8, 2), (2, 0)]):
        x0 = gen.normal((m, DIM), 1.0, 80 + step)
        rope_m = rope_table(m, 90 + step, paired=True)
        x = to_dev(x0)
        layer.decode(x, to_dev(rope_m))
        qkv = dec("qkv", x0 * oracle.row_scales(x0, DIM)[:, None], m)
        q, _, new_k, new_v = oracle.qkv_rows(qkv, m, rope_m, H, G, 0)
        for i in range(m):
            oracle.kv_push(bits, new_k[i], new_v[i], G, cap - rows, tail_len + i, tail)
        tail_len += m
        pk, vals, gk = oracle.kv_dequantize(bits, sealed, rows, H, G, tail, cap - rows, tail_len)
        total = rows + tail_len
        # default_fast_exp: fast mode gives Q8 records the fast decode exp.
        assert layer.split.fast_exp is (bits == 8)
        want_attn = oracle.attention_decode(q, pk, gk, vals, m, rows, total, H, G, total - m, image[0], image[1],
                                            sinks, exp_fast=bits == 8)
        close(host(layer._buf("dattn", (m, H, 64))), want_attn)
        want_x = x0 + dec("wo", want_attn.reshape(m, -1), m)
        gated = dec("w13", want_x * oracle.row_scales(want_x, DIM)[:, None], m, glu=True)
        want_x = want_x + dec("w2", gated, m)
        assert max_rel(host(x), want_x) <= 1e-4, step
        if drop:
            layer.truncate(layer.len - drop)
            tail_len -= drop
        assert layer.split.info()[2] == tail_len and layer.len == rows + tail_len
    with pytest.raises(fh.FocrError):
        layer.truncate(rows - 1)  # the prompt stays
    layer.free()
    for lin in lins.values():
        lin.free()


@pytest.mark.parametrize("softmax", ["static", "online"])
def test_decoder_layer_with_bf16_attention(fh, softmax):
    """Fast mode's plan: INT16 projections and BF16 prefill attention
    (PrefillAttention::Bf16Static / Bf16). The layer's attention output is
    within the BF16 tolerance of the BF16 attention oracle on the layer's own
    queries and cache."""
    import torch

    rows, image = 200, (0, 128)
    w = layer_weights(70)
    lins = {name: fh.QuantLinear(8, *w[name], 64) for name in w}
    sinks = gen.uniform(H, -2.0, 2.0, 71)
    opts = fh.PrefillOptions(softmax=fh.Softmax.STATIC if softmax == "static" else fh.Softmax.ONLINE)
    layer = fh.DecoderLayer(lins["qkv"], lins["wo"], lins["w13"], lins["w2"], to_dev(sinks), capacity=rows + 4,
                            options=opts, bf16_attention=True)
    h0 = gen.normal((rows, DIM), 1.0, 72)
    rope = rope_table(rows, 73)
    layer.prefill(to_dev(h0), to_dev(rope), *image)
    torch.cuda.synchronize()
    _, want_q, want_pk, want_v, _ = oracle_layer_prefill(w, h0, rope, image, sinks)
    want = oracle.attention_prefill_bf16(want_q, want_pk, want_v, rows, H, G, image[0], image[1], sinks,
                                         static=softmax == "static")
    got = host(layer._buf("attn", (rows, H, 64)))
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 2e-3
    for lin in lins.values():
        lin.free()
