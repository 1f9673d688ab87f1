"""One decoder layer of the Falcon-OCR runner on the `hip` backend.

`DecoderLayer` strings the C ABI's operators together the way
``Model::forward_layers`` does for one layer (src/model/mod.rs:513-691):

prefill of more than 8 rows (the panel path, mod.rs:568,956-1007)::

    row_scales(h)                          panel_qkv (rms norm folded into packing)
    qkv.prefill(h, row_scale) -> qkv        Epilogue::Store
    qkv_rows(qkv) -> q, prefix keys, values fused_prefix_rows (model/fused.rs:17-99)
    attention_with(q, cache) -> attn        LayerCache::attention (model/cache.rs:142-197)
    wo.prefill(attn) += h                   Epilogue::Add(h)
    row_scales(h); w13.prefill(h) -> gated  Epilogue::Glu
    w2.prefill(gated) += h                  Epilogue::Add(h)

decode / draft verification, and a prefill of at most 8 rows (1..=8 rows,
project_qkv + attention_out_ffn, mod.rs:421-492; a short prefill keeps the
online FP32 softmax and no BF16 attention, ``PrefillPlan::softmaxes(false)``,
src/kernels/mod.rs:148-153)::

    rms_norm(h) . qkv -> qkv                focr_linear_decode_ex, rms_norm in the GEMV
    qkv_rows -> q, generated keys, values   split_norm_rope + LayerCache::append
    attention over prefix + generated keys  (decode kernel)
    wo(attn); add_residual                  Epilogue ADD
    rms_norm(h) . w13 -> gated (GLU)
    w2(gated); add_residual

The compact cache (prefix keys per query head, generated keys and values per
KV head) lives in device memory sized for `capacity` positions, as
``Session::new`` sizes the reference's (model/cache.rs:364). With
``kv_bits`` 8 (Kv::Q8) or 16 (Kv::Q16) the prefill seals the prefix after its
attention (``seal_layer``, model/cache.rs:218-276) into a `KvSplit`, and decode
appends each step's keys and values to its tail and attends over the records
(``LayerCache::Split``); ``kv_bits`` 32 keeps the compact FP32 cache
(Kv::Compact). The sealed cache's decode exp follows ``default_fast_exp``
(kv.rs:182-184, applied in seal_layer, model/cache.rs:260-264): the fast exp
for Q8 records when ``options.exp`` is ExpMode.FAST, the exact one otherwise;
``decode_fast_exp`` overrides it as ``Tuning::decode_fast_exp`` does.
``bf16_attention`` runs the prefill attention in BF16 as the
fast mode's plan does (``PrefillAttention::Bf16`` / ``Bf16Static`` by
``options.softmax``). RoPE factors
come from the caller ([rows][n_heads][32][2] cos/sin pairs), as
``rotary_factors`` provides them to the reference's row kernels.

`clock`, if given, is called with a stage name after each stage is
enqueued, as the reference's PhaseClock marks phases (model/profile.rs:40-60).
"""
from __future__ import annotations

from typing import Optional

from . import (CompactKv, Context, Epilogue, ExpMode, FocrError, Geometry, KvSplit, PrefillOptions, PrefillProjection,
               Softmax, attention_decode_row, attention_prefill_bf16, attention_with, default_context,
               default_fast_exp, qkv_rows,
               row_scales)


class DecoderLayer:
    def __init__(self, qkv, wo, w13, w2, sinks, capacity: int, n_heads: int = 16, n_kv_heads: int = 8,
                 head_dim: int = 64, projection: PrefillProjection = PrefillProjection.I16,
                 options: PrefillOptions = PrefillOptions(), ctx: Optional[Context] = None, kv_bits: int = 32,
                 bf16_attention: bool = False, decode_fast_exp: Optional[bool] = None):
        import torch

        self.ctx = ctx or default_context()
        self.qkv, self.wo, self.w13, self.w2 = qkv, wo, w13, w2
        self.sinks = sinks
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.dim = qkv.in_dim
        qdim, kdim = n_heads * head_dim, n_kv_heads * head_dim
        if qkv.out_dim != qdim + 2 * kdim or wo.in_dim != qdim or wo.out_dim != self.dim:
            raise FocrError(-2, "layer shapes: qkv [qdim + 2 kdim][dim], wo [dim][qdim]")
        if w13.in_dim != self.dim or w2.in_dim != w13.out_dim // 2 or w2.out_dim != self.dim:
            raise FocrError(-2, "layer shapes: w13 [2 ffn][dim], w2 [dim][ffn]")
        if kv_bits not in (8, 16, 32):
            raise FocrError(-1, "kv_bits: 32 (compact FP32), 16 (Q16) or 8 (Q8)")
        self.projection, self.options = projection, options
        self.capacity = capacity
        self.kv_bits = kv_bits
        self.bf16_attention = bf16_attention
        self.decode_fast_exp = default_fast_exp(kv_bits, options.exp == ExpMode.FAST, decode_fast_exp)
        self.split: Optional[KvSplit] = None
        dev = f"cuda:{self.ctx.device}"
        f32 = torch.float32
        self.prefix_k = torch.empty((capacity, n_heads, head_dim), dtype=f32, device=dev)
        self.generated_k = torch.empty((capacity, n_kv_heads, head_dim), dtype=f32, device=dev)
        self.v = torch.empty((capacity, n_kv_heads, head_dim), dtype=f32, device=dev)
        self.len = 0
        self.prefix_len = 0
        self.image = (0, 0)
        self._work = {}

    def _buf(self, name: str, shape):
        import torch

        t = self._work.get(name)
        n = 1
        for s in shape:
            n *= s
        if t is None or t.numel() < n:
            t = torch.empty(n, dtype=torch.float32, device=f"cuda:{self.ctx.device}")
            self._work[name] = t
        return t[:n].view(*shape)

    def kv(self, total: int) -> CompactKv:
        """The cache's first `total` positions as a CompactKv."""
        p = self.prefix_len
        gen = self.generated_k[: total - p] if total > p else None
        return CompactKv(self.prefix_k[:p], gen, self.v[:total], p, total, self.n_heads, self.n_kv_heads,
                         self.head_dim)

    def prefill(self, h, rope, image_start: int, image_end: int, clock=None):
        """The whole prompt (offset 0): updates `h` [rows][dim] in place and
        fills the prefix cache."""
        rows = h.shape[0]
        if self.len != 0:
            raise FocrError(-2, "a prefill forwards the whole prefix first")
        if rows > self.capacity:
            raise FocrError(-2, "KV context exhausted")
        if not (image_start <= image_end <= rows):
            raise FocrError(-2, "attention image must be inside the prefix")
        ctx = self.ctx
        mark = clock or (lambda stage: None)
        if self.split is not None:
            self.split.free()
            self.split = None
        # The panel path takes more than 8 rows (`panel = rows > 8 && ...`,
        # model/mod.rs:568); shorter prompts run the decode step's GEMVs.
        panel = rows > 8
        if panel:
            rs = row_scales(h, self.dim, out=self._buf("rs", (rows,)), ctx=ctx)
            qkv = self.qkv.prefill(h, rows, row_scale=rs, epilogue=Epilogue.STORE, kernel=self.projection,
                                   out=self._buf("qkv", (rows, self.qkv.out_dim)))
        else:
            qkv = self.qkv.linear_ex(h, rows, rms_norm=True, out=self._buf("qkv", (rows, self.qkv.out_dim)))
        mark("qkv")
        self.prefix_len = rows
        q = qkv_rows(qkv, rows, rope, self.n_heads, self.n_kv_heads, rows, q=self._buf("q", (rows, self.n_heads, 64)),
                     prefix_k=self.prefix_k[:rows], v=self.v[:rows], ctx=ctx)
        mark("qkv_rows")
        self.image = (image_start, image_end)
        attn = self._buf("attn", (rows, self.n_heads, 64))
        geometry = Geometry(0, image_start, image_end)
        # Fast mode's BF16 attention where the plan has it; the reference's
        # `false` (a shape it does not take) falls back to the FP32 tiles
        # (Model::forward_layers, model/mod.rs:621-646 -> LayerCache::attention,
        # model/cache.rs:142-197).
        options = self.options if panel else PrefillOptions(exp=self.options.exp, fp32_softmax=Softmax.ONLINE,
                                                            softmax=self.options.softmax)
        if not (panel and self.bf16_attention and attention_prefill_bf16(q, self.kv(rows), rows, geometry,
                                                                         self.sinks, attn, options, ctx=ctx)):
            attn = attention_with(q, self.kv(rows), rows, geometry, self.sinks, options, output=attn, ctx=ctx)
        mark("attention")
        if self.kv_bits != 32:
            self.split = KvSplit.seal(self.kv_bits, self.prefix_k[:rows], self.v[:rows], rows, self.capacity,
                                      self.n_heads, self.n_kv_heads, ctx=ctx).set_fast_exp(self.decode_fast_exp)
            mark("seal")
        if panel:
            self.wo.prefill(attn, rows, epilogue=Epilogue.ADD, out=h, kernel=self.projection)
            mark("wo")
            rs = row_scales(h, self.dim, out=rs, ctx=ctx)
            gated = self.w13.prefill(h, rows, row_scale=rs, epilogue=Epilogue.GLU, kernel=self.projection,
                                     out=self._buf("gated", (rows, self.w13.out_dim // 2)))
            mark("w13")
            self.w2.prefill(gated, rows, epilogue=Epilogue.ADD, out=h, kernel=self.projection)
        else:
            self.wo.linear_ex(attn, rows, epilogue=Epilogue.ADD, out=h)
            mark("wo")
            gated = self.w13.linear_ex(h, rows, rms_norm=True, epilogue=Epilogue.GLU,
                                       out=self._buf("gated", (rows, self.w13.out_dim // 2)))
            mark("w13")
            self.w2.linear_ex(gated, rows, epilogue=Epilogue.ADD, out=h)
        mark("w2")
        self.len = rows
        return h

    def decode(self, h, rope, clock=None):
        """1..=8 rows at positions len.. (a greedy step, or the last token plus
        drafts): updates `h` [rows][dim] in place and appends to the cache."""
        rows = h.shape[0]
        if not 1 <= rows <= 8:
            raise FocrError(-2, "decode takes 1..=8 rows")
        if self.len + rows > self.capacity:
            raise FocrError(-2, "KV context exhausted")
        ctx, p, pos = self.ctx, self.prefix_len, self.len
        mark = clock or (lambda stage: None)
        qkv = self.qkv.linear_ex(h, rows, rms_norm=True, out=self._buf("dqkv", (rows, self.qkv.out_dim)))
        mark("qkv")
        total = pos + rows
        out = self._buf("dattn", (rows, self.n_heads, 64))
        if self.split is None and rows == 1:
            # The row step, the cache append and the attention in one launch.
            attn = attention_decode_row(qkv, rope, self.kv(total), *self.image, self.sinks,
                                        q=self._buf("dq", (1, self.n_heads, 64)), output=out, ctx=ctx)
        elif self.split is None:
            q = qkv_rows(qkv, rows, rope, self.n_heads, self.n_kv_heads, 0, q=self._buf("dq", (rows, self.n_heads, 64)),
                         generated_k=self.generated_k[pos - p: pos - p + rows], v=self.v[pos: pos + rows], ctx=ctx)
            mark("qkv_rows")
            attn = attention_with(q, self.kv(total), rows, Geometry(pos, *self.image), self.sinks, self.options,
                                  output=out, ctx=ctx)
        elif rows == 1:
            # The row step, the tail append and the attention in one launch.
            attn = self.split.decode_row(qkv, rope, self.sinks, q=self._buf("dq", (1, self.n_heads, 64)), out=out)
        else:
            # split_norm_rope and the tail append in one kernel.
            q = self.split.qkv_rows(qkv, rows, rope, q=self._buf("dq", (rows, self.n_heads, 64)))
            mark("qkv_rows")
            attn = self.split.attention_decode(q, rows, self.sinks, out=out)
        mark("attention")
        self.wo.linear_ex(attn, rows, epilogue=Epilogue.ADD, out=h)
        mark("wo")
        gated = self.w13.linear_ex(h, rows, rms_norm=True, epilogue=Epilogue.GLU,
                                   out=self._buf("dgated", (rows, self.w13.out_dim // 2)))
        mark("w13")
        self.w2.linear_ex(gated, rows, epilogue=Epilogue.ADD, out=h)
        mark("w2")
        self.len = total
        return h

    def truncate(self, length: int) -> None:
        """``Session::truncate`` (model/cache.rs:281-298): drop the newest
        positions so that `length` remain (rejected draft tokens); the prompt
        stays. A sealed cache forgets its tail past them; the compact cache
        overwrites them on the next decode."""
        if not (self.prefix_len <= length <= self.len) or self.len == 0:
            raise FocrError(-2, "truncation must keep the prompt")
        if self.split is not None:
            self.split.truncate_tail(length - self.prefix_len)
        self.len = length

    def free(self) -> None:
        if self.split is not None:
            self.split.free()
            self.split = None
