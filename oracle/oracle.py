"""ctypes loader for the C oracle (oracle/focr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by bench.py's ``cpu_baseline`` leg. The product library
never loads it. Each wrapper names the reference function its C body follows
(see the C file for file:line citations).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_BUILD = _HERE / "_build"

STORE, GLU, ADD = 0, 1, 2


def cpu_flags() -> set:
    try:
        return set(Path("/proc/cpuinfo").read_text().split("flags", 2)[1].split("\n", 1)[0].split(":", 1)[1].split())
    except (OSError, IndexError):
        return set()


V3_FLAGS = ("avx2", "fma", "bmi2", "movbe")
V4_FLAGS = V3_FLAGS + ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")


def variant() -> str:
    """The widest oracle build the host CPU runs: v4 (AVX-512), v3 (AVX2) or generic."""
    flags = cpu_flags()
    if all(f in flags for f in V4_FLAGS):
        return "v4"
    if all(f in flags for f in V3_FLAGS):
        return "v3"
    return "generic"


def build() -> None:
    """Compile the oracle (gcc, oracle/Makefile)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _load() -> ctypes.CDLL:
    name = f"liboracle_{variant()}.so"
    path = _BUILD / name
    if not path.exists():
        build()
    return ctypes.CDLL(str(path))


_lib = _load()
_P = ctypes.c_void_p
_Z = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float


def _sig(name, restype, *args):
    fn = getattr(_lib, name)
    fn.restype = restype
    fn.argtypes = list(args)
    return fn


_sig("orc_exp_poly", _F, _F)
_sig("orc_exp_poly_unchecked", _F, _F)
_sig("orc_squared_relu_glu", _F, _F, _F)
_sig("orc_quantize_bits", _I, _P, _Z, _Z, _Z, _I, _P, _P)
_sig("orc_dequantize", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _P)
_sig("orc_validate_w8", _I, _Z, _Z, _Z, _P, _P)
_sig("orc_dot", _F, _P, _P, _Z)
_sig("orc_dot_q", _F, _I, _P, _P, _P, _Z, _Z)
_sig("orc_linear_decode", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _P, _Z, _P)
_sig("orc_linear_decode_fast", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _P, _Z, _P)
_sig("orc_linear_decode_glu_fast", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _P, _Z, _P)
_sig("orc_linear_decode_glu", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _P, _Z, _P)
_sig("orc_rms_scale", _F, _P, _Z, _F)
_sig("orc_row_scales", None, _P, _Z, _Z, _F, _P)
_sig("orc_panel_gemm", None, _P, _Z, _Z, _P, _Z, _P, _I, _P)
_sig("orc_panel_gemm_fast", None, _P, _Z, _Z, _P, _Z, _P, _I, _P)
_sig("orc_attention_prefill_fast", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _Z, _Z, _P)
_sig("orc_i16_quantize_group", _F, _P, _P)
_sig("orc_i16_quantize_rows", None, _P, _Z, _Z, _P, _Z, _P, _P, _P, _P)
_sig("orc_i16_gemm", None, _P, _Z, _Z, _P, _P, _Z, _P, _P, _Z, _P, _I, _P)
_sig("orc_i16_panels_pack", _P, _Z, _Z, _P, _P, _P, _P, _Z)
_sig("orc_i16_panels_free", None, _P)
_sig("orc_i16_gemm_fast", _I, _P, _P, _Z, _P, _I, _P)
_sig("orc_attention_prefill", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _P)
_sig("orc_attention_prefill_tiles", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _Z, _Z, _P)
_sig("orc_attention_prefill_bf16_tiles", None, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _P, _I, _I, _Z, _Z, _P)
_sig("orc_exp2_minimax", _F, _F)
_sig("orc_bf16_round", _F, _F)
_sig("orc_argmax", _I, _P, _Z, _P)
_sig("orc_screen_kappa", _F, _Z)
_sig("orc_screen_build", _I, _P, _Z, _Z, _P, _P, _P, _P)
_sig("orc_screen_prepare", _I, _P, _Z, _F, _P)
_sig("orc_screen_row", None, _P, _P, _P, _P, _Z, _P, _P)
_sig("orc_screen_select", _I, _P, _P, _P, _P, _Z, _Z, _F, _F, _P, _P, _P)
_sig("orc_bf16_up", ctypes.c_uint16, _F)
_sig("orc_bf16_f32", _F, ctypes.c_uint16)
_sig("orc_kv_seal", _I, _I, _P, _P, _Z, _Z, _Z, _P, _P)
_sig("orc_kv_push", None, _I, _P, _P, _Z, _Z, _Z, _P, _P)
_sig("orc_kv_dequantize", None, _I, _P, _P, _Z, _Z, _Z, _P, _P, _Z, _Z, _P, _P, _P)
_sig("orc_qkv_rows", None, _P, _Z, _P, _Z, _Z, _Z, _P, _P, _P, _P)
_sig("orc_attention_decode", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _P)
_sig("orc_attention_decode_ex", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _I, _P)
_sig("orc_attention_decode_fast", None, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _Z, _P, _P)
_sig("orc_set_threads", None, _I)
_sig("orc_get_threads", _I)


def _ptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    _lib.orc_set_threads(int(n))


def threads() -> int:
    return _lib.orc_get_threads()


set_threads(1)


def exp_poly(x: float) -> float:
    return _lib.orc_exp_poly(x)


def exp_poly_unchecked(x: float) -> float:
    return _lib.orc_exp_poly_unchecked(x)


def squared_relu_glu(gate: float, up: float) -> float:
    return _lib.orc_squared_relu_glu(gate, up)


def quantize_bits(w, n, k, group, bits):
    """QuantLinear::quantize_bits (src/quant/linear.rs:140-201) -> (codes, scales) or error code."""
    w = _f32(w)
    codes = np.zeros(n * k, dtype=np.int8 if bits == 8 else np.int16)
    scales = np.zeros(n * ((k + group - 1) // group), dtype=np.float32)
    rc = _lib.orc_quantize_bits(_ptr(w), n, k, group, bits, _ptr(codes), _ptr(scales))
    if rc != 0:
        return rc
    return codes.reshape(n, k), scales.reshape(n, -1)


def _exc(exc_cols, exc_vals):
    if exc_cols is None or len(exc_cols) == 0:
        return None, None, 0
    cols = np.ascontiguousarray(exc_cols, dtype=np.int32)
    vals = _f32(exc_vals)
    return cols, vals, len(cols)


def dequantize(bits, codes, scales, n, k, group, exc_cols=None, exc_vals=None):
    """dequantize_row for every row (src/quant/linear.rs:246-262)."""
    codes = np.ascontiguousarray(codes)
    scales = _f32(scales)
    cols, vals, ne = _exc(exc_cols, exc_vals)
    out = np.zeros((n, k), dtype=np.float32)
    _lib.orc_dequantize(bits, _ptr(codes), _ptr(scales), n, k, group, _ptr(cols), _ptr(vals), ne, _ptr(out))
    return out


def validate_w8(n, k, group, codes, scales) -> int:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = _f32(scales)
    return _lib.orc_validate_w8(n, k, group, _ptr(codes), _ptr(scales))


def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return _lib.orc_dot(_ptr(a), _ptr(b), a.size)


def dot_q(bits, x, codes, scales, group) -> float:
    x, scales, codes = _f32(x), _f32(scales), np.ascontiguousarray(codes)
    return _lib.orc_dot_q(bits, _ptr(x), _ptr(codes), _ptr(scales), x.size, group)


def linear_decode(bits, codes, scales, n, k, group, x, rows, exc_cols=None, exc_vals=None, fast=False):
    """QuantLinear::linear small-M (bits 8/16) or linear_with_simd rows<=8 (bits 32).
    fast: the reference's AVX2 dot_q restated (oracle/focr_cpu_gemv.c), the
    same bits at CPU-baseline speed."""
    codes = np.ascontiguousarray(codes)
    scales = _f32(scales) if scales is not None else np.zeros(1, np.float32)
    x = _f32(x)
    cols, vals, ne = _exc(exc_cols, exc_vals)
    out = np.zeros((rows, n), dtype=np.float32)
    (_lib.orc_linear_decode_fast if fast else _lib.orc_linear_decode)(bits, _ptr(codes), _ptr(scales), n, k, group, _ptr(cols), _ptr(vals), ne, _ptr(x), rows, _ptr(out))
    return out


def linear_decode_glu(bits, codes, scales, n, k, group, x, rows, exc_cols=None, exc_vals=None, fast=False):
    codes = np.ascontiguousarray(codes)
    scales = _f32(scales) if scales is not None else np.zeros(1, np.float32)
    x = _f32(x)
    cols, vals, ne = _exc(exc_cols, exc_vals)
    out = np.zeros((rows, n // 2), dtype=np.float32)
    (_lib.orc_linear_decode_glu_fast if fast else _lib.orc_linear_decode_glu)(bits, _ptr(codes), _ptr(scales), n, k, group, _ptr(cols), _ptr(vals), ne, _ptr(x), rows, _ptr(out))
    return out


def rms_scale(row, eps=float(np.finfo(np.float32).eps)) -> float:
    row = _f32(row)
    return _lib.orc_rms_scale(_ptr(row), row.size, eps)


def row_scales(h, width, eps=float(np.finfo(np.float32).eps)):
    h = _f32(h)
    rows = h.size // width
    out = np.zeros(rows, dtype=np.float32)
    _lib.orc_row_scales(_ptr(h), rows, width, eps, _ptr(out))
    return out


def panel_gemm(a, m, k, w, n, row_scale=None, epilogue=STORE, out=None):
    """FP32 panel GEMM (src/kernels/panels/panel.rs:118-172) on dequantized w [n][k]."""
    a, w = _f32(a), _f32(w)
    rs = _f32(row_scale) if row_scale is not None else None
    width = n // 2 if epilogue == GLU else n
    if out is None:
        out = np.zeros((m, width), dtype=np.float32)
    else:
        out = _f32(out).copy()
    _lib.orc_panel_gemm(_ptr(a), m, k, _ptr(w), n, _ptr(rs), epilogue, _ptr(out))
    return out


def panel_gemm_fast(a, m, k, w, n, row_scale=None, epilogue=STORE, out=None):
    """The FP32 panel GEMM with the reference's AVX2 6x16 micro-kernel
    (oracle/focr_cpu_panels.c): bitwise panel_gemm, CPU-baseline speed."""
    a, w = _f32(a), _f32(w)
    rs = _f32(row_scale) if row_scale is not None else None
    width = n // 2 if epilogue == GLU else n
    if out is None:
        out = np.zeros((m, width), dtype=np.float32)
    else:
        out = _f32(out).copy()
    _lib.orc_panel_gemm_fast(_ptr(a), m, k, _ptr(w), n, _ptr(rs), epilogue, _ptr(out))
    return out


def i16_quantize_group(x):
    x = _f32(x)
    assert x.size == 64
    q = np.zeros(64, dtype=np.int16)
    step = _lib.orc_i16_quantize_group(_ptr(x), _ptr(q))
    return np.float32(step), q


def i16_quantize_rows(a, m, k, row_scale=None, exc_cols=None):
    a = _f32(a)
    rs = _f32(row_scale) if row_scale is not None else None
    cols = np.ascontiguousarray(exc_cols, dtype=np.int32) if exc_cols is not None and len(exc_cols) else None
    ne = 0 if cols is None else len(cols)
    codes = np.zeros((m, k), dtype=np.int16)
    steps = np.zeros((m, k // 64), dtype=np.float32)
    xe = np.zeros((m, max(ne, 1)), dtype=np.float32)
    _lib.orc_i16_quantize_rows(_ptr(a), m, k, _ptr(cols), ne, _ptr(rs), _ptr(codes), _ptr(steps), _ptr(xe))
    return codes, steps, xe[:, :ne]


def i16_gemm(a, m, k, codes, scales, n, row_scale=None, epilogue=STORE, exc_cols=None, exc_vals=None, out=None):
    """INT16-activation panel GEMM (src/kernels/panels/panel_i16.rs:133-369)."""
    a = _f32(a)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = _f32(scales)
    rs = _f32(row_scale) if row_scale is not None else None
    cols, vals, ne = _exc(exc_cols, exc_vals)
    width = n // 2 if epilogue == GLU else n
    if out is None:
        out = np.zeros((m, width), dtype=np.float32)
    else:
        out = _f32(out).copy()
    _lib.orc_i16_gemm(_ptr(a), m, k, _ptr(codes), _ptr(scales), n, _ptr(cols), _ptr(vals), ne, _ptr(rs), epilogue, _ptr(out))
    return out


class I16Panels:
    """INT8 codes packed once into the reference's VNNI panels
    (oracle/focr_cpu_panels_i16.c; panel_i16::pack at load). gemm() is
    bitwise i16_gemm at CPU-baseline speed; it returns None on a CPU
    without AVX-512 VNNI."""

    def __init__(self, codes, scales, n, k, exc_cols=None, exc_vals=None):
        self.n, self.k = n, k
        self._codes = np.ascontiguousarray(codes, dtype=np.int8)
        self._scales = _f32(scales)
        cols, vals, ne = _exc(exc_cols, exc_vals)
        self.handle = _lib.orc_i16_panels_pack(n, k, _ptr(self._codes), _ptr(self._scales), _ptr(cols), _ptr(vals), ne)
        if not self.handle:
            raise ValueError("VNNI panels need n a multiple of 32 and k of 64")

    def gemm(self, a, m, row_scale=None, epilogue=STORE, out=None):
        a = _f32(a)
        rs = _f32(row_scale) if row_scale is not None else None
        width = self.n // 2 if epilogue == GLU else self.n
        if out is None:
            out = np.zeros((m, width), dtype=np.float32)
        else:
            out = _f32(out).copy()
        rc = _lib.orc_i16_gemm_fast(self.handle, _ptr(a), m, _ptr(rs), epilogue, _ptr(out))
        return None if rc == -1 else out

    def free(self):
        if self.handle:
            _lib.orc_i16_panels_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def attention_prefill(q, prefix_k, v, query_len, prefix_len, total_len, n_heads, n_kv_heads,
                      query_offset, image_start, image_end, sinks, static=False, exp_fast=True,
                      generated_k=None, tiles=None):
    """compact_prefill (src/kernels/attention/prefill64.rs:149-480), head_dim 64."""
    q, prefix_k, v, sinks = _f32(q), _f32(prefix_k), _f32(v), _f32(sinks)
    gk = _f32(generated_k) if generated_k is not None else None
    out = np.zeros(query_len * n_heads * 64, dtype=np.float32)
    if tiles is None:
        _lib.orc_attention_prefill(_ptr(q), _ptr(prefix_k), _ptr(gk), _ptr(v), query_len, prefix_len, total_len,
                                   n_heads, n_kv_heads, query_offset, image_start, image_end, _ptr(sinks),
                                   int(static), int(exp_fast), _ptr(out))
    else:
        _lib.orc_attention_prefill_tiles(_ptr(q), _ptr(prefix_k), _ptr(gk), _ptr(v), query_len, prefix_len,
                                         total_len, n_heads, n_kv_heads, query_offset, image_start, image_end,
                                         _ptr(sinks), int(static), int(exp_fast), tiles[0], tiles[1], _ptr(out))
    return out.reshape(query_len, n_heads, 64)


def attention_prefill_fast(q, prefix_k, v, query_len, prefix_len, total_len, n_heads, n_kv_heads, query_offset,
                           image_start, image_end, sinks, static=False, generated_k=None, tiles=None, out=None):
    """attention_prefill (Fast exp or static) vectorized over the query lanes:
    bitwise the same outputs, at CPU-baseline speed (oracle/focr_cpu_attention.c)."""
    q, prefix_k, v, sinks = _f32(q), _f32(prefix_k), _f32(v), _f32(sinks)
    gk = _f32(generated_k) if generated_k is not None else None
    if out is None:
        out = np.zeros(query_len * n_heads * 64, dtype=np.float32)
    lo, hi = (0, (query_len + 31) // 32) if tiles is None else tiles
    _lib.orc_attention_prefill_fast(_ptr(q), _ptr(prefix_k), _ptr(gk), _ptr(v), query_len, prefix_len, total_len,
                                    n_heads, n_kv_heads, query_offset, image_start, image_end, _ptr(sinks),
                                    int(static), lo, hi, _ptr(out))
    return out.reshape(query_len, n_heads, 64)


def attention_prefill_bf16(q, k, v, query_len, n_heads, n_kv_heads, image_start, image_end, sinks,
                           static=False, exp_fast=True, tiles=None):
    """BF16 compact_prefill (src/kernels/attention/prefill64/bf16.rs:70-175), pure prefill."""
    q, k, v, sinks = _f32(q), _f32(k), _f32(v), _f32(sinks)
    out = np.zeros(query_len * n_heads * 64, dtype=np.float32)
    lo, hi = (0, (query_len + 31) // 32) if tiles is None else tiles
    _lib.orc_attention_prefill_bf16_tiles(_ptr(q), _ptr(k), _ptr(v), query_len, n_heads, n_kv_heads, image_start,
                                          image_end, _ptr(sinks), int(static), int(exp_fast), lo, hi, _ptr(out))
    return out.reshape(query_len, n_heads, 64)


def exp2_minimax(t):
    return np.float32(_lib.orc_exp2_minimax(float(t)))


def bf16_round(x):
    """half::bf16::from_f32(x).to_f32(), elementwise."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7fffffff) > 0x7f800000
    r = ((u + 0x7fff + ((u >> 16) & 1)) & 0xffff0000).astype(np.uint32)
    r = np.where(nan, (u.astype(np.uint32) | 0x00400000) & 0xffff0000, r).astype(np.uint32)
    return r.view(np.float32)


def qkv_rows(qkv, rows, rope, n_heads, n_kv_heads, prefix_rows):
    """fused_row / split_norm_rope + append_unique_heads (src/model/fused.rs:101-123,
    src/model/rope.rs:14-86, src/model/cache.rs:202-216): returns
    (q [rows][n_heads][64], prefix_k [prefix_rows][n_heads][64],
    generated_k [rows - prefix_rows][n_kv_heads][64], v [rows][n_kv_heads][64])."""
    qkv, rope = _f32(qkv), _f32(rope)
    q = np.zeros((rows, n_heads, 64), dtype=np.float32)
    pk = np.zeros((prefix_rows, n_heads, 64), dtype=np.float32)
    gk = np.zeros((rows - prefix_rows, n_kv_heads, 64), dtype=np.float32)
    v = np.zeros((rows, n_kv_heads, 64), dtype=np.float32)
    _lib.orc_qkv_rows(_ptr(qkv), rows, _ptr(rope), n_heads, n_kv_heads, prefix_rows, _ptr(q), _ptr(pk), _ptr(gk),
                      _ptr(v))
    return q, pk, gk, v


def attention_decode(q, prefix_k, generated_k, v, query_len, prefix_len, total_len, n_heads, n_kv_heads,
                     query_offset, image_start, image_end, sinks, exp_fast=False, fast=False):
    """online::head (src/kernels/attention/online.rs:96-150) for every (query, head).
    exp_fast: the per-key probabilities by exp_poly, as the sealed cache's
    decode with SplitPrefix::fast_exp (src/quant/kv/decode.rs:346-347).
    fast: the same bits with the reference's AVX2 dot and axpy
    (oracle/focr_cpu_gemv.c), CPU-baseline speed (platform exp only)."""
    q, v, sinks = _f32(q), _f32(v), _f32(sinks)
    pk = _f32(prefix_k) if prefix_len else None
    gk = _f32(generated_k) if total_len > prefix_len else None
    out = np.zeros(query_len * n_heads * 64, dtype=np.float32)
    if fast and not exp_fast:
        _lib.orc_attention_decode_fast(_ptr(q), _ptr(pk), _ptr(gk), _ptr(v), query_len, prefix_len, total_len,
                                       n_heads, n_kv_heads, query_offset, image_start, image_end, _ptr(sinks),
                                       _ptr(out))
        return out.reshape(query_len, n_heads, 64)
    _lib.orc_attention_decode_ex(_ptr(q), _ptr(pk), _ptr(gk), _ptr(v), query_len, prefix_len, total_len, n_heads,
                                 n_kv_heads, query_offset, image_start, image_end, _ptr(sinks), int(exp_fast),
                                 _ptr(out))
    return out.reshape(query_len, n_heads, 64)


def argmax(logits):
    logits = _f32(logits)
    out = ctypes.c_uint32(0)
    rc = _lib.orc_argmax(_ptr(logits), logits.size, ctypes.byref(out))
    if rc != 0:
        raise ValueError("nonfinite or empty logits")
    return int(out.value)


# ---- INT8 screened vocabulary head (src/head_screen.rs) -------------------
SCREEN_LIMIT = 1024


def screen_build(w, vocab, dim):
    """ScreenedHead::build: (codes int8 [vocab][dim], scales [vocab][dim/64],
    weight_abs_max, kappa); raises ValueError where the reference errors."""
    w = _f32(w)
    codes = np.zeros((vocab, dim), dtype=np.int8)
    scales = np.zeros((vocab, max(dim // 64, 1)), dtype=np.float32)
    wmax, kappa = ctypes.c_float(0), ctypes.c_float(0)
    rc = _lib.orc_screen_build(_ptr(w), vocab, dim, _ptr(codes), _ptr(scales), ctypes.byref(wmax), ctypes.byref(kappa))
    if rc != 0:
        raise ValueError("screened head build rejected the weights")
    return codes, scales, float(wmax.value), float(kappa.value)


def screen_kappa(dim):
    return float(_lib.orc_screen_kappa(dim))


def screen_prepare(x, dim, weight_abs_max):
    """(ok, norms) of prepare."""
    x = _f32(x)
    norms = np.zeros(max(dim // 64, 1), dtype=np.float32)
    ok = _lib.orc_screen_prepare(_ptr(x), dim, weight_abs_max, _ptr(norms))
    return bool(ok), norms


def screen_row(x, codes, scales, norms, dim):
    """(q, S) of screen_row for one screen row."""
    x, scales, norms = _f32(x), _f32(scales), _f32(norms)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    q, s = ctypes.c_float(0), ctypes.c_float(0)
    _lib.orc_screen_row(_ptr(x), _ptr(codes), _ptr(scales), _ptr(norms), dim, ctypes.byref(q), ctypes.byref(s))
    return float(q.value), float(s.value)


def screen_select(x, fp32, codes, scales, vocab, dim, weight_abs_max, kappa):
    """ScreenedHead::select: (token or None for Fallback, candidates, upper [vocab])."""
    x, fp32, scales = _f32(x), _f32(fp32), _f32(scales)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    upper = np.zeros(vocab, dtype=np.float32)
    token, cand = ctypes.c_uint32(0), ctypes.c_uint32(0)
    ok = _lib.orc_screen_select(_ptr(x), _ptr(fp32), _ptr(codes), _ptr(scales), vocab, dim, weight_abs_max, kappa,
                                _ptr(upper), ctypes.byref(token), ctypes.byref(cand))
    return (int(token.value) if ok else None), int(cand.value), upper


# ---- Sealed split KV cache, Kv::Q8 / Kv::Q16 (src/quant/kv.rs) -------------
def bf16_up(scale: float) -> int:
    return int(_lib.orc_bf16_up(scale))


def bf16_f32(bits: int) -> float:
    return float(_lib.orc_bf16_f32(bits))


def kv_seal(bits, prefix_k, v, prefix_len, n_heads, n_kv):
    """SplitPrefix::seal: (codes [n_kv][P][160], steps [n_kv][P][5] as uint16)
    or the error code (-1 pair, -2 non-finite, -3 overflow, -4 shape)."""
    prefix_k, v = _f32(prefix_k), _f32(v)
    codes = np.zeros((n_kv, prefix_len, 160), dtype=np.int8 if bits == 8 else np.int16)
    scales = np.zeros((n_kv, prefix_len, 5), dtype=np.uint16)
    rc = _lib.orc_kv_seal(bits, _ptr(prefix_k), _ptr(v), prefix_len, n_heads, n_kv, _ptr(codes), _ptr(scales))
    return rc if rc != 0 else (codes, scales)


def kv_tail(bits, n_kv, capacity):
    """An empty tail: (codes [n_kv][capacity][128], steps [n_kv][capacity][4])."""
    return (np.zeros((n_kv, capacity, 128), dtype=np.int8 if bits == 8 else np.int16),
            np.zeros((n_kv, capacity, 4), dtype=np.uint16))


def kv_push(bits, k, v, n_kv, capacity, index, tail):
    """push_unique of one generated position (keys, values [n_kv][64]) into `tail`."""
    k, v = _f32(k), _f32(v)
    codes, scales = tail
    _lib.orc_kv_push(bits, _ptr(k), _ptr(v), n_kv, capacity, index, _ptr(codes), _ptr(scales))


def kv_dequantize(bits, sealed, prefix_len, n_heads, n_kv, tail, capacity, tail_len):
    """(prefix_k [P][n_heads][64], values [P + tail_len][n_kv][64],
    generated_k [tail_len][n_kv][64]) decoded from the records."""
    codes, scales = sealed
    tcodes, tscales = tail
    pk = np.zeros((prefix_len, n_heads, 64), dtype=np.float32)
    vals = np.zeros((prefix_len + tail_len, n_kv, 64), dtype=np.float32)
    gk = np.zeros((max(tail_len, 1), n_kv, 64), dtype=np.float32)
    _lib.orc_kv_dequantize(bits, _ptr(codes), _ptr(scales), prefix_len, n_heads, n_kv, _ptr(tcodes), _ptr(tscales),
                           capacity, tail_len, _ptr(pk), _ptr(vals), _ptr(gk))
    return pk, vals, gk[:tail_len]
