"""Python host mirror of the Falcon-OCR runner's operator interface, over the
``focr_hip`` C ABI (include/focr_hip.h, lib/libfocr_hip.so built for gfx950).

Names and argument meanings follow the reference (amazingvince/falcon-ocr-cpu):

  QuantLinear            src/quant/linear.rs:123-130 (codes, scales, exceptions)
    .from_parts          from_parts          (linear.rs:318-358)
    .with_exceptions     with_exceptions     (linear.rs:366-390)
    .linear              linear, 1..=8 rows  (linear.rs:497-549)
    .linear_glu          linear_glu          (linear.rs:555-625)
    .prefill             prefill             (linear.rs:634-707)
    .dequantize          dequantize_row x n  (linear.rs:246-262)
  Linear.from_f32        kernels::linear_with_simd's FP32 weights (kernels/mod.rs:387)
  Epilogue               panel::Epilogue     (kernels/panels/panel.rs:26-33)
  PrefillProjection      kernels::PrefillProjection (kernels/mod.rs:71-84), `hip` kinds
  Geometry, CompactKv    kernels::attention  (kernels/attention/mod.rs:40-196)
  PrefillOptions         (attention/mod.rs:205-221)
  attention_with         (attention/mod.rs:256-311)
  row_scales / rms_scale (model/rope.rs:147-152, kernels/mod.rs:531-533)
  argmax                 (runner/mod.rs:916-930)
  qkv_rows               fused_prefix_rows / split_norm_rope + LayerCache::append
                         (model/fused.rs:17-123, model/rope.rs:14-86, model/cache.rs:117-216)
  DecoderLayer           one layer of Model::forward_layers (model/mod.rs:513-691):
                         prefill and decode steps over a device-resident compact cache

Tensors are torch CUDA tensors (device memory and streams come from torch;
the arithmetic runs in the HIP library). Errors raise ``FocrError``, the
counterpart of the reference's ``anyhow`` errors and shape assertions. There
is no CPU fallback: without the built library or a GPU this module raises.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np

_ROOT = Path(__file__).resolve().parents[1]
LIBRARY = _ROOT / "lib" / "libfocr_hip.so"
HEADER = _ROOT.parent / "include" / "focr_hip.h"

FOCR_OK = 0
FOCR_E_UNSUPPORTED = -3
ERRORS = {-1: "FOCR_E_ARG", -2: "FOCR_E_SHAPE", -3: "FOCR_E_UNSUPPORTED", -4: "FOCR_E_HIP",
          -5: "FOCR_E_VALUE", -6: "FOCR_E_NONFINITE"}

# Every entry point of include/focr_hip.h, with its ctypes signature.
_P, _Z, _I, _F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "focr_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "focr_ctx_destroy": (_I, [_P]),
    "focr_ctx_set_stream": (_I, [_P, _P]),
    "focr_ctx_use_own_stream": (_I, [_P]),
    "focr_ctx_stream": (_P, [_P]),
    "focr_ctx_sync": (_I, [_P]),
    "focr_ctx_reserve_scratch": (_I, [_P, _Z]),
    "focr_ctx_scratch_bytes": (_I, [_P, ctypes.POINTER(_Z)]),
    "focr_last_error": (ctypes.c_char_p, []),
    "focr_malloc": (_I, [_P, _Z, ctypes.POINTER(_P)]),
    "focr_free": (_I, [_P, _P]),
    "focr_memcpy_h2d": (_I, [_P, _P, _P, _Z]),
    "focr_memcpy_d2h": (_I, [_P, _P, _P, _Z]),
    "focr_linear_upload": (_I, [_P, _I, _Z, _Z, _Z, _P, _P, _P, _P, _Z, ctypes.POINTER(_P)]),
    "focr_linear_free": (_I, [_P]),
    "focr_linear_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_Z), ctypes.POINTER(_Z),
                              ctypes.POINTER(_Z), ctypes.POINTER(_Z), ctypes.POINTER(_Z)]),
    "focr_linear_dequantize": (_I, [_P, _P, _P]),
    "focr_linear_decode": (_I, [_P, _P, _P, _Z, _P]),
    "focr_linear_decode_glu": (_I, [_P, _P, _P, _Z, _P]),
    "focr_linear_decode_ex": (_I, [_P, _P, _P, _Z, _P, _I, _I, _P]),
    "focr_linear_prefill": (_I, [_P, _P, _P, _Z, _P, _I, _I, _P]),
    "focr_row_scales": (_I, [_P, _P, _Z, _Z, _F, _P]),
    "focr_attention_prefill": (_I, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _P]),
    "focr_attention_prefill_split": (_I, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _P]),
    "focr_attention_prefill_bf16": (_I, [_P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _P]),
    "focr_argmax": (_I, [_P, _P, _Z, _Z, _P]),
    "focr_kv_seal": (_I, [_P, _I, _P, _P, _Z, _Z, _Z, _Z, _Z, ctypes.POINTER(_P)]),
    "focr_kv_append": (_I, [_P, _P, _P, _P, _Z]),
    "focr_kv_attention_decode": (_I, [_P, _P, _P, _Z, _P, _P]),
    "focr_kv_attention_decode_noalloc": (_I, [_P, _P, _P, _Z, _P, _P]),
    "focr_kv_dequantize": (_I, [_P, _P, _P, _P, _P]),
    "focr_kv_truncate_tail": (_I, [_P, _Z]),
    "focr_kv_set_fast_exp": (_I, [_P, _I]),
    "focr_kv_fast_exp": (_I, [_P, _P]),
    "focr_kv_qkv_rows": (_I, [_P, _P, _P, _Z, _P, _P]),
    "focr_kv_decode_row": (_I, [_P, _P, _P, _P, _P, _P, _P]),
    "focr_kv_info": (_I, [_P, _P, _P, _P, _P, _P]),
    "focr_kv_free": (_I, [_P]),
    "focr_screen_build": (_I, [_P, _P, _Z, _Z, ctypes.POINTER(_P)]),
    "focr_screen_upload": (_I, [_P, _P, _P, _Z, _Z, ctypes.c_float, ctypes.c_float, ctypes.POINTER(_P)]),
    "focr_screen_free": (_I, [_P]),
    "focr_screen_constants": (_I, [_P, _P, _P]),
    "focr_screen_bounds": (_I, [_P, _Z, _P]),
    "focr_screen_select": (_I, [_P, _P, _P, _P, _Z, _P, _P]),
    "focr_qkv_rows": (_I, [_P, _P, _Z, _P, _Z, _Z, _Z, _Z, _P, _P, _P, _P]),
    "focr_attention_decode": (_I, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _P]),
    "focr_attention_decode_row": (_I, [_P] * 6 + [_Z] * 7 + [_P] * 3),
}


class FocrError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, code)}: {message}")
        self.code = code


def load_library(path: Path = LIBRARY) -> ctypes.CDLL:
    """Load lib/libfocr_hip.so and bind every declared symbol (raises if absent)."""
    if not path.exists():
        raise FocrError(-3, f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def _check(rc: int) -> None:
    if rc != FOCR_OK:
        raise FocrError(rc, lib().focr_last_error().decode())


def _torch():
    import torch

    return torch


def _dev(t) -> Optional[int]:
    """Device pointer of a CUDA tensor (None passes NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise FocrError(-1, "expected a CUDA tensor")
    if not t.is_contiguous():
        raise FocrError(-2, "expected a contiguous tensor")
    return t.data_ptr()


class Context:
    """A focr_ctx bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0):
        torch = _torch()
        handle = ctypes.c_void_p()
        _check(lib().focr_ctx_create(device, ctypes.byref(handle)))
        self.handle = handle
        self.device = device
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
        _check(lib().focr_ctx_set_stream(self.handle, ctypes.c_void_p(stream.cuda_stream)))

    def use_stream(self, stream) -> None:
        """Run on a torch stream (None: the context's own stream)."""
        if stream is None:
            _check(lib().focr_ctx_use_own_stream(self.handle))
        else:
            _check(lib().focr_ctx_set_stream(self.handle, ctypes.c_void_p(stream.cuda_stream)))

    def sync(self) -> None:
        _check(lib().focr_ctx_sync(self.handle))

    def reserve_scratch(self, nbytes: int) -> None:
        """Grow the context scratch now (before a HIP graph capture)."""
        _check(lib().focr_ctx_reserve_scratch(self.handle, int(nbytes)))

    def scratch_bytes(self) -> int:
        out = ctypes.c_size_t()
        _check(lib().focr_ctx_scratch_bytes(self.handle, ctypes.byref(out)))
        return out.value

    def close(self) -> None:
        if self.handle:
            _check(lib().focr_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default: Optional[Context] = None


def default_context() -> Context:
    global _default
    if _default is None:
        _default = Context(0)
    return _default


class Epilogue(enum.IntEnum):
    """Where a finished tile goes (panel.rs:26-33)."""

    STORE = 0
    GLU = 1
    ADD = 2


class PrefillProjection(enum.IntEnum):
    """The `hip` backend's prefill projection kernels."""

    F32_MFMA = 0  # FP32 matrix cores, within FP32 tolerance of the panels
    F32_CHAIN = 1  # bitwise the FP32 panels (PanelAvx2)
    I16 = 2  # bitwise the INT16 panels (PanelI16Vnni / PanelI16Avx2)
    F32_SPLIT = 3  # FP32 weights: power-of-two scaled FP16 pairs on the FP16 matrix cores, FP32 tolerance


class Linear:
    """A device-resident matrix (focr_linear): 8/16-bit codes or FP32 weights."""

    def __init__(self, bits, codes, scales, group, exc_cols=None, exc_vals=None, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()
        codes = np.ascontiguousarray(codes)
        n, k = codes.shape
        dtype = {8: np.int8, 16: np.int16, 32: np.float32}[bits]
        codes = codes.astype(dtype, copy=False)
        sc = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)
        cols = vals = None
        n_exc = 0
        if exc_cols is not None and len(exc_cols):
            cols = np.ascontiguousarray(exc_cols, dtype=np.int32)
            vals = np.ascontiguousarray(exc_vals, dtype=np.float32)
            n_exc = len(cols)
        handle = ctypes.c_void_p()
        ptr = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
        _check(lib().focr_linear_upload(self.ctx.handle, bits, n, k, group if bits != 32 else 0, ptr(codes), ptr(sc),
                                        ptr(cols), ptr(vals), n_exc, ctypes.byref(handle)))
        self.handle = handle
        self.out_dim, self.in_dim, self.group, self._bits, self.n_exc = n, k, group, bits, n_exc

    @classmethod
    def from_f32(cls, weights, ctx: Optional[Context] = None) -> "Linear":
        return cls(32, np.asarray(weights, dtype=np.float32), None, 32, ctx=ctx)

    def dimensions(self):
        return self.out_dim, self.in_dim

    def bits(self) -> int:
        return self._bits

    def device_bytes(self) -> int:
        out = ctypes.c_size_t()
        _check(lib().focr_linear_info(self.handle, None, None, None, None, None, ctypes.byref(out)))
        return out.value

    def free(self) -> None:
        if getattr(self, "handle", None):
            _check(lib().focr_linear_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    # -- operators ---------------------------------------------------------
    def dequantize(self):
        torch = _torch()
        out = torch.empty((self.out_dim, self.in_dim), dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        _check(lib().focr_linear_dequantize(self.ctx.handle, self.handle, _dev(out)))
        return out

    def linear(self, input, rows: int, output=None):
        """`QuantLinear::linear` for 1..=8 rows: returns [rows][out]."""
        torch = _torch()
        if input.numel() != rows * self.in_dim:
            raise FocrError(-2, "W8 input shape")
        if output is None:
            output = torch.empty((rows, self.out_dim), dtype=torch.float32, device=input.device)
        elif output.numel() != rows * self.out_dim:
            raise FocrError(-2, "W8 output shape")
        _check(lib().focr_linear_decode(self.ctx.handle, self.handle, _dev(input), rows, _dev(output)))
        return output

    def linear_glu(self, input, rows: int, gated=None):
        """`QuantLinear::linear_glu`: squared-ReLU GLU of interleaved gate/up rows."""
        torch = _torch()
        if input.numel() != rows * self.in_dim:
            raise FocrError(-2, "W8 input shape")
        if gated is None:
            gated = torch.empty((rows, self.out_dim // 2), dtype=torch.float32, device=input.device)
        _check(lib().focr_linear_decode_glu(self.ctx.handle, self.handle, _dev(input), rows, _dev(gated)))
        return gated

    def linear_ex(self, input, rows: int, row_scale=None, epilogue: Epilogue = Epilogue.STORE, out=None,
                  rms_norm: bool = False):
        """The decode step's projection with its neighbours folded in
        (Model::project_qkv / attention_out_ffn, model/mod.rs:421-492):
        input rows rms-normalized (`rms_norm=True`, computed in the kernel)
        or times a precomputed `row_scale`, then `linear` (STORE),
        `linear_glu` (GLU) or `linear` + `add_residual` into `out` (ADD)."""
        torch = _torch()
        if input.numel() != rows * self.in_dim:
            raise FocrError(-2, "W8 input shape")
        width = self.out_dim // 2 if epilogue == Epilogue.GLU else self.out_dim
        if out is None:
            if epilogue == Epilogue.ADD:
                raise FocrError(-1, "Epilogue.ADD needs the residual `out`")
            out = torch.empty((rows, width), dtype=torch.float32, device=input.device)
        elif out.numel() != rows * width:
            raise FocrError(-2, "W8 output shape")
        _check(lib().focr_linear_decode_ex(self.ctx.handle, self.handle, _dev(input), rows, _dev(row_scale),
                                           int(bool(rms_norm)), int(epilogue), _dev(out)))
        return out

    def prefill(self, input, rows: int, row_scale=None, epilogue: Epilogue = Epilogue.STORE, out=None,
                kernel: PrefillProjection = PrefillProjection.F32_MFMA):
        """`QuantLinear::prefill`: out = epilogue(A' W^T), A' = input * row_scale per row.

        For Epilogue.ADD, `out` holds the residual and is updated in place."""
        torch = _torch()
        if input.numel() != rows * self.in_dim:
            raise FocrError(-2, "prefill input shape")
        width = self.out_dim // 2 if epilogue == Epilogue.GLU else self.out_dim
        if out is None:
            if epilogue == Epilogue.ADD:
                raise FocrError(-1, "Epilogue.ADD needs the residual `out`")
            out = torch.empty((rows, width), dtype=torch.float32, device=input.device)
        _check(lib().focr_linear_prefill(self.ctx.handle, self.handle, _dev(input), rows, _dev(row_scale),
                                         int(epilogue), int(kernel), _dev(out)))
        return out


class QuantLinear(Linear):
    """A quantized matrix with 8- or 16-bit codes (src/quant/linear.rs:123-130)."""

    @classmethod
    def from_parts(cls, out_dim, in_dim, group_size, codes, scales, ctx: Optional[Context] = None) -> "QuantLinear":
        codes = np.asarray(codes).reshape(out_dim, in_dim)
        bits = 8 if codes.dtype == np.int8 else 16
        return cls(bits, codes, np.asarray(scales, dtype=np.float32).reshape(out_dim, -1), group_size, ctx=ctx)

    def with_exceptions(self, columns, values) -> "QuantLinear":
        raise FocrError(-3, "pass exc_cols/exc_vals to the constructor (the device copy is immutable)")


@dataclass(frozen=True)
class Geometry:
    """Masking geometry (attention/mod.rs:40-76)."""

    query_offset: int
    image_start: int
    image_end: int


@dataclass
class CompactKv:
    """Compact KV cache (attention/mod.rs:78-151); tensors on the GPU."""

    prefix_k: object
    generated_k: object
    v: object
    prefix_len: int
    total_len: int
    n_heads: int
    n_kv_heads: int
    head_dim: int

    @classmethod
    def prefill(cls, k, v, total, n_heads, n_kv_heads, head_dim=64) -> "CompactKv":
        return cls(k, None, v, total, total, n_heads, n_kv_heads, head_dim)


class Softmax(enum.IntEnum):
    ONLINE = 0
    STATIC = 1


class ExpMode(enum.IntEnum):
    FAST = 0
    EXACT = 1


@dataclass(frozen=True)
class PrefillOptions:
    """attention/mod.rs:205-221: `softmax` is the BF16 kernels' softmax
    (static shift by default, as the reference's PrefillSoftmax), and
    `fp32_softmax` the FP32 tiles' one. `split_products` (a `hip` choice,
    no reference counterpart) forms the FP32 tiles' products on the FP16
    matrix cores from power-of-two scaled FP16 pairs on a pure prefill
    (focr_attention_prefill_split); False keeps the FP32 matrix cores
    everywhere."""

    exp: ExpMode = ExpMode.FAST
    fp32_softmax: Softmax = Softmax.ONLINE
    softmax: Softmax = Softmax.STATIC
    split_products: bool = True


def attention_with(q, kv: CompactKv, query_len: int, geometry: Geometry, sinks, options: PrefillOptions = PrefillOptions(),
                   output=None, ctx: Optional[Context] = None):
    """`kernels::attention_with`: returns [query_len][n_heads][64].

    As the reference dispatches (attention/mod.rs:271-311): fewer than 4
    queries, or up to 8 over a cache with generated keys (decode and draft
    verification), take the decode kernel; the rest the prefill tiles (their
    products from FP16 pairs on a pure prefill unless
    `options.split_products` is False)."""
    torch = _torch()
    ctx = ctx or default_context()
    if output is None:
        output = torch.empty_like(q)
    if query_len < 4 or (query_len <= 8 and kv.total_len > kv.prefix_len):
        return attention_decode(q, kv, query_len, geometry, sinks, output=output, ctx=ctx)
    pure = geometry.query_offset == 0 and query_len == kv.prefix_len == kv.total_len
    fn = lib().focr_attention_prefill_split if options.split_products and pure else lib().focr_attention_prefill
    _check(fn(ctx.handle, _dev(q), _dev(kv.prefix_k), _dev(kv.generated_k), _dev(kv.v), query_len, kv.prefix_len,
              kv.total_len, kv.n_heads, kv.n_kv_heads, kv.head_dim, geometry.query_offset, geometry.image_start,
              geometry.image_end, _dev(sinks), int(options.fp32_softmax), int(options.exp), _dev(output)))
    return output


def attention_decode(q, kv: CompactKv, query_len: int, geometry: Geometry, sinks, output=None,
                     ctx: Optional[Context] = None):
    """Decode / draft-verify attention of 1..=8 query rows (online::head,
    attention/online.rs:96-150, split over many waves): [query_len][n_heads][64]."""
    torch = _torch()
    ctx = ctx or default_context()
    if output is None:
        output = torch.empty_like(q)
    _check(lib().focr_attention_decode(ctx.handle, _dev(q), _dev(kv.prefix_k), _dev(kv.generated_k), _dev(kv.v),
                                       query_len, kv.prefix_len, kv.total_len, kv.n_heads, kv.n_kv_heads,
                                       kv.head_dim, geometry.query_offset, geometry.image_start, geometry.image_end,
                                       _dev(sinks), _dev(output)))
    return output


def attention_decode_row(qkv, rope, kv: CompactKv, image_start: int, image_end: int, sinks, q=None, output=None,
                         ctx: Optional[Context] = None):
    """One greedy step in one launch: `qkv_rows` for the generated row at
    position kv.total_len - 1 (its key and value written to the cache kv
    views, which must include that row), then `attention_decode` of that row
    over kv (bitwise the two calls). Returns output [1][n_heads][64]; `q`
    [1][n_heads][64], if given, receives the rotated query."""
    torch = _torch()
    ctx = ctx or default_context()
    if output is None:
        output = torch.empty((1, kv.n_heads, kv.head_dim), dtype=torch.float32, device=qkv.device)
    _check(lib().focr_attention_decode_row(ctx.handle, _dev(qkv), _dev(rope), _dev(kv.prefix_k), _dev(kv.generated_k),
                                           _dev(kv.v), kv.prefix_len, kv.total_len, kv.n_heads, kv.n_kv_heads,
                                           kv.head_dim, image_start, image_end, _dev(sinks), _dev(q),
                                           _dev(output)))
    return output


def qkv_rows(qkv, rows: int, rope, n_heads: int, n_kv_heads: int, prefix_rows: int, q=None, prefix_k=None,
             generated_k=None, v=None, head_dim: int = 64, ctx: Optional[Context] = None):
    """Split, per-head RMS norm, RoPE and cache append of `rows` QKV rows
    (fused_prefix_rows for the first `prefix_rows`, split_norm_rope +
    LayerCache::append after them). `prefix_k`, `generated_k` and `v` are the
    cache slots of the first row; returns q [rows][n_heads][64]."""
    torch = _torch()
    ctx = ctx or default_context()
    if q is None:
        q = torch.empty((rows, n_heads, head_dim), dtype=torch.float32, device=qkv.device)
    _check(lib().focr_qkv_rows(ctx.handle, _dev(qkv), rows, _dev(rope), n_heads, n_kv_heads, head_dim, prefix_rows,
                               _dev(q), _dev(prefix_k), _dev(generated_k), _dev(v)))
    return q


def attention_prefill_bf16(q, kv: CompactKv, query_len: int, geometry: Geometry, sinks, output,
                           options: PrefillOptions = PrefillOptions(), ctx: Optional[Context] = None) -> bool:
    """`kernels::attention_prefill_bf16` (attention/mod.rs:320-352): the BF16
    prefill into `output`; False (nothing written) where the reference's
    returns false: not a pure prefill, fewer than 4 queries, head_dim != 64."""
    ctx = ctx or default_context()
    if geometry.query_offset != 0 or kv.prefix_len != kv.total_len or query_len != kv.total_len:
        return False
    rc = lib().focr_attention_prefill_bf16(ctx.handle, _dev(q), _dev(kv.prefix_k), _dev(kv.v), query_len, kv.n_heads,
                                           kv.n_kv_heads, kv.head_dim, geometry.image_start, geometry.image_end,
                                           _dev(sinks), int(options.softmax), int(options.exp), _dev(output))
    if rc == FOCR_E_UNSUPPORTED:
        return False
    _check(rc)
    return True


F32_EPSILON = float(np.finfo(np.float32).eps)


def row_scales(h, width: int, eps: float = F32_EPSILON, out=None, ctx: Optional[Context] = None):
    """`rms_norm`'s factor of every width-wide row (eps f32::EPSILON by default)."""
    torch = _torch()
    ctx = ctx or default_context()
    rows = h.numel() // width
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=h.device)
    _check(lib().focr_row_scales(ctx.handle, _dev(h), rows, width, eps, _dev(out)))
    return out


def argmax(logits, rows: int, vocab: int, ctx: Optional[Context] = None):
    """Greedy tokens of `rows` rows; FocrError(FOCR_E_NONFINITE) on NaN/inf."""
    ctx = ctx or default_context()
    tokens = (ctypes.c_uint32 * rows)()
    _check(lib().focr_argmax(ctx.handle, _dev(logits), rows, vocab, ctypes.cast(tokens, ctypes.c_void_p)))
    return list(tokens)


def default_fast_exp(kv_bits: int, fast_exps: bool, requested: Optional[bool] = None) -> bool:
    """`default_fast_exp` (src/quant/kv.rs:176-184): the fast decode exp for
    8-bit records when the run allows fast exps (ExpMode::FAST), the exact one
    otherwise; `requested` (`Tuning::decode_fast_exp`) overrides it."""
    if requested is not None:
        return bool(requested)
    return bool(fast_exps) and kv_bits == 8


class KvSplit:
    """`SplitPrefix` (src/quant/kv.rs) for `Kv::Q8` (bits 8) and `Kv::Q16`
    (bits 16): the sealed prefix records and the generated tail, on the device."""

    def __init__(self, handle, bits: int, n_heads: int, n_kv_heads: int, ctx: Context):
        self.handle, self.bits, self.n_heads, self.n_kv_heads, self.ctx = handle, bits, n_heads, n_kv_heads, ctx

    @classmethod
    def seal(cls, bits: int, prefix_k, v, prefix_len: int, capacity: int, n_heads: int = 16, n_kv_heads: int = 8,
             ctx: Optional[Context] = None) -> "KvSplit":
        """`SplitPrefix::from_compact` of a compact prefix (device tensors)."""
        ctx = ctx or default_context()
        handle = ctypes.c_void_p()
        _check(lib().focr_kv_seal(ctx.handle, bits, _dev(prefix_k), _dev(v), prefix_len, capacity, n_heads,
                                  n_kv_heads, 64, ctypes.byref(handle)))
        return cls(handle, bits, n_heads, n_kv_heads, ctx)

    def append(self, k, v, rows: int) -> None:
        """`push_unique` of `rows` positions: k, v [rows][n_kv_heads][64]."""
        _check(lib().focr_kv_append(self.ctx.handle, self.handle, _dev(k), _dev(v), rows))

    def qkv_rows(self, qkv, rows: int, rope, q=None):
        """The decode row step fused with the append: queries [rows][n_heads][64]
        out, the rows' unique keys and values coded into the tail."""
        torch = _torch()
        if q is None:
            q = torch.empty((rows, self.n_heads, 64), dtype=torch.float32, device=qkv.device)
        _check(lib().focr_kv_qkv_rows(self.ctx.handle, self.handle, _dev(qkv), rows, _dev(rope), _dev(q)))
        return q

    def decode_row(self, qkv, rope, sinks, q=None, out=None):
        """One greedy step in one launch: the row step and append of
        `qkv_rows` for one row, then `attention_decode` of that row over the
        cache including it (bitwise the two calls). Returns out [1][n_heads][64];
        `q` [1][n_heads][64], if given, receives the rotated query."""
        torch = _torch()
        if out is None:
            out = torch.empty((1, self.n_heads, 64), dtype=torch.float32, device=qkv.device)
        _check(lib().focr_kv_decode_row(self.ctx.handle, self.handle, _dev(qkv), _dev(rope), _dev(sinks), _dev(q),
                                        _dev(out)))
        return out

    def attention_decode(self, q, rows: int, sinks, out=None):
        """`attention_decode_rows`: [rows][n_heads][64] for the last `rows` positions."""
        torch = _torch()
        if out is None:
            out = torch.empty((rows, self.n_heads, 64), dtype=torch.float32, device=q.device)
        _check(lib().focr_kv_attention_decode(self.ctx.handle, self.handle, _dev(q), rows, _dev(sinks), _dev(out)))
        return out

    def attention_decode_noalloc(self, q, rows: int, sinks, out):
        """`attention_decode_rows` through the entry point that allocates
        nothing (a fixed per-GPU array holds the partial states; calls that
        overlap on one GPU race). `out` [rows][n_heads][64] is required."""
        _check(lib().focr_kv_attention_decode_noalloc(self.ctx.handle, self.handle, _dev(q), rows, _dev(sinks),
                                                      _dev(out)))
        return out

    def set_fast_exp(self, fast: bool) -> "KvSplit":
        """`with_fast_exp` (kv.rs:423): the decode softmax's per-key
        probabilities use the hardware exp2 (the reference's polynomial exp)."""
        _check(lib().focr_kv_set_fast_exp(self.handle, int(bool(fast))))
        return self

    @property
    def fast_exp(self) -> bool:
        """`SplitPrefix::fast_exp` (kv/record_bits.rs:6-8)."""
        f = ctypes.c_int()
        _check(lib().focr_kv_fast_exp(self.handle, ctypes.byref(f)))
        return bool(f.value)

    def truncate_tail(self, tail_len: int) -> None:
        """`truncate_tail`: forget the generated positions past `tail_len`."""
        _check(lib().focr_kv_truncate_tail(self.handle, tail_len))

    def info(self):
        """(bits, prefix_len, tail_len, capacity, device_bytes)."""
        b, p, t, c, n = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(lib().focr_kv_info(self.handle, ctypes.byref(b), ctypes.byref(p), ctypes.byref(t), ctypes.byref(c),
                                  ctypes.byref(n)))
        return b.value, p.value, t.value, c.value, n.value

    def dequantize(self):
        """(prefix_k [P][n_heads][64], values [P + tail][n_kv][64], generated_k [tail][n_kv][64])."""
        torch = _torch()
        _, p, t, _, _ = self.info()
        dev = f"cuda:{self.ctx.device}"
        pk = torch.empty((p, self.n_heads, 64), dtype=torch.float32, device=dev)
        vals = torch.empty((p + t, self.n_kv_heads, 64), dtype=torch.float32, device=dev)
        gk = torch.empty((max(t, 1), self.n_kv_heads, 64), dtype=torch.float32, device=dev)
        _check(lib().focr_kv_dequantize(self.ctx.handle, self.handle, _dev(pk), _dev(vals), _dev(gk)))
        return pk, vals, gk[:t]

    def free(self) -> None:
        if getattr(self, "handle", None):
            _check(lib().focr_kv_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


SCREEN_LIMIT = 1024  # CANDIDATE_LIMIT (src/head_screen.rs:29)


class ScreenedHead:
    """`ScreenedHead` (src/head_screen.rs): an INT8 screen of the FP32
    vocabulary head whose `select` returns the exact FP32 greedy token."""

    def __init__(self, handle, vocab: int, dim: int, ctx: Context):
        self.handle, self.vocab, self.dim, self.ctx = handle, vocab, dim, ctx

    @classmethod
    def build(cls, weights, ctx: Optional[Context] = None) -> "ScreenedHead":
        """`ScreenedHead::build` from host FP32 weights [vocab][dim]."""
        ctx = ctx or default_context()
        w = np.ascontiguousarray(weights, dtype=np.float32)
        vocab, dim = w.shape
        handle = ctypes.c_void_p()
        _check(lib().focr_screen_build(ctx.handle, w.ctypes.data_as(ctypes.c_void_p), vocab, dim, ctypes.byref(handle)))
        return cls(handle, vocab, dim, ctx)

    @classmethod
    def from_parts(cls, codes, scales, weight_abs_max: float, kappa: float, ctx: Optional[Context] = None):
        """`ScreenedHead::from_mapped`: a stored screen and its constants."""
        ctx = ctx or default_context()
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        vocab, dim = codes.shape
        handle = ctypes.c_void_p()
        _check(lib().focr_screen_upload(ctx.handle, codes.ctypes.data_as(ctypes.c_void_p),
                                        scales.ctypes.data_as(ctypes.c_void_p), vocab, dim, weight_abs_max, kappa,
                                        ctypes.byref(handle)))
        return cls(handle, vocab, dim, ctx)

    def constants(self):
        """(weight_abs_max, kappa)."""
        wmax, kappa = ctypes.c_float(), ctypes.c_float()
        _check(lib().focr_screen_constants(self.handle, ctypes.byref(wmax), ctypes.byref(kappa)))
        return float(wmax.value), float(kappa.value)

    def bounds(self, rows: int) -> np.ndarray:
        """q + B [rows][vocab] of the last `select` (HeadScratch::upper)."""
        out = np.empty((rows, self.vocab), dtype=np.float32)
        _check(lib().focr_screen_bounds(self.handle, rows, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def select(self, x, rows: int, head: "Linear"):
        """`select_rows`: per input row, (token, candidates) for Screened::Token
        or (None, candidates) for Screened::Fallback."""
        if x.numel() != rows * self.dim:
            raise FocrError(-2, "screened head input shape")
        tokens = (ctypes.c_int32 * rows)()
        cands = (ctypes.c_uint32 * rows)()
        _check(lib().focr_screen_select(self.ctx.handle, self.handle, head.handle, _dev(x), rows,
                                        ctypes.cast(tokens, ctypes.c_void_p), ctypes.cast(cands, ctypes.c_void_p)))
        return [(None if t < 0 else int(t), int(c)) for t, c in zip(tokens, cands)]

    def free(self) -> None:
        if getattr(self, "handle", None):
            _check(lib().focr_screen_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


from .layer import DecoderLayer  # noqa: E402,F401
