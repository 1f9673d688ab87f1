"""Kernel-ready model files on the `hip` backend: map a packed safetensors
file and upload its matrices and screen into device handles.

Mirrors ``src/model/packed.rs``: the format tags and body tensor names
(packed.rs:27-41), ``write_packed`` (packed.rs:54-179), ``load_packed``
(packed.rs:190-310), the header-only inspection (``packed_profile``,
``packed_facts``, ``safetensors_header``: packed.rs:182-188,486-515), the
matrix mapping with exception columns (``map_matrix``, packed.rs:400-465;
``QuantLinear::with_mapped_exceptions``, src/quant/linear.rs:386-426), the
digest order (``packed_order``, packed.rs:536-565) and the tensor digest
(``packed_digest``, packed.rs:567-577).

What the reference maps in place and computes with on the CPU is here mapped
(numpy ``memmap``, no copy) and handed to the upload entry points as it is:
body matrices to ``focr_linear_upload`` (codes bytes unchanged), the INT8
screen to ``focr_screen_upload`` with its stored constants, the FP32 head to
``focr_linear_upload(bits 32)``, the sinks to device tensors. The
embedding, image projector, final norm and golden RoPE table stay host
memmaps (their consumers are outside the accelerated path).

Safetensors layout (the format the reference reads through the
``safetensors 0.8.0`` crate): an 8-byte little-endian header length, the
JSON header (``__metadata__`` string map plus ``{dtype, shape,
data_offsets}`` per tensor, offsets relative to the end of the header), then
the tensor bytes.
"""
from __future__ import annotations

import enum
import hashlib
import json
import math
import re
import struct
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from . import FocrError, Linear, QuantLinear, ScreenedHead, default_context

# Format tags and names (packed.rs:27-41), the checkpoint pins
# (src/config.rs:10-12). A file must carry these exact strings.
PACKED_FORMAT = "falcon-ocr-kernel-v1"
PACKED_FORMAT_EXCEPTIONS = "falcon-ocr-kernel-v2"
PACKED_FORMAT_FP32 = "falcon-ocr-kernel-fp32-v1"
BODY = ("attention.wqkv", "attention.wo", "feed_forward.w13", "feed_forward.w2")
EXCEPTION_SUFFIXES = (".__exc_cols", ".__exc_vals")
MODEL_REVISION = "fe757d59ecd79d4d68760162306a70a015761ad9"
WEIGHTS_SHA256 = "3df91e403dc48794bf1c48511e75c3508b1cc52df599dcc15f1080d46101ab16"
HEADER_LIMIT = 64 << 20  # safetensors_header's cap (packed.rs:494)

DTYPES = {"F32": np.dtype("<f4"), "I8": np.dtype("i1"), "I16": np.dtype("<i2"), "I32": np.dtype("<i4"),
          "I64": np.dtype("<i8"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"), "U8": np.dtype("u1")}


def _err(msg: str) -> FocrError:
    return FocrError(-5, msg)


def _ensure(cond: bool, msg: str) -> None:
    if not cond:
        raise _err(msg)


# ---- model config (src/config.rs:92-165) -------------------------------------
@dataclass(frozen=True)
class ModelConfig:
    dim: int
    n_layers: int
    n_heads: int
    head_dim: int
    n_kv_heads: int
    vocab_size: int
    ffn_dim: int
    norm_eps: float
    max_seq_len: int
    rope_theta: float
    channel_size: int
    spatial_patch_size: int
    temporal_patch_size: int
    eos_id: int
    img_id: int
    image_cls_token_id: int
    image_reg_1_token_id: int
    image_reg_2_token_id: int
    image_reg_3_token_id: int
    image_reg_4_token_id: int
    img_end_id: int

    @classmethod
    def from_json(cls, text: str) -> "ModelConfig":
        """serde's reading: the struct's fields (unknown keys ignored), f32
        fields rounded to f32."""
        raw = json.loads(text)
        try:
            values = {f.name: raw[f.name] for f in fields(cls)}
        except KeyError as e:
            raise _err(f"model config field {e.args[0]} missing") from None
        for f in fields(cls):
            if f.name in ("norm_eps", "rope_theta"):
                values[f.name] = float(np.float32(values[f.name]))
            elif not isinstance(values[f.name], int) or values[f.name] < 0:
                raise _err(f"model config field {f.name}")
        return cls(**values)

    def to_json(self) -> str:
        return json.dumps({f.name: getattr(self, f.name) for f in fields(self)}, separators=(",", ":"))

    def validate(self) -> None:
        """ModelConfig::validate (config.rs:123-156): only the pinned
        Falcon-OCR v1.5 architecture."""
        _ensure((self.dim, self.n_layers, self.n_heads, self.head_dim, self.n_kv_heads, self.ffn_dim,
                 self.vocab_size) == (768, 22, 16, 64, 8, 2304, 65536),
                "unsupported architecture: expected Falcon-OCR v1.5 dimensions")
        _ensure((self.channel_size, self.spatial_patch_size, self.temporal_patch_size) == (3, 16, 1),
                "unsupported patch configuration")
        _ensure(self.max_seq_len == 16384 and np.float32(self.rope_theta) == np.float32(10000.0)
                and np.float32(self.norm_eps) == np.float32(1e-5),
                "unsupported positional/normalization configuration")
        _ensure([self.eos_id, self.img_id, self.image_cls_token_id, self.image_reg_1_token_id,
                 self.image_reg_2_token_id, self.image_reg_3_token_id, self.image_reg_4_token_id,
                 self.img_end_id] == [11, 227, 244, 245, 246, 247, 248, 230],
                "unsupported special token configuration")

    def query_dim(self) -> int:
        return self.n_heads * self.head_dim

    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def patch_dim(self) -> int:
        return self.channel_size * self.spatial_patch_size ** 2


# ---- storage profiles (src/quant/mod.rs:18-160) ------------------------------
WEIGHTS = ("f32", "int16", "int8")
KVS = ("compact", "f32-split", "q16", "q8", "q8r", "q4r")
_PROFILE_LABELS = {
    ("f32", "compact"): "reference", ("f32", "f32-split"): "split-f32", ("f32", "q16"): "kv-q16",
    ("f32", "q8"): "kv-q8", ("f32", "q8r"): "kv-q8r", ("f32", "q4r"): "kv-q4r",
    ("int16", "compact"): "w16-body-compact", ("int16", "f32-split"): "w16-body",
    ("int16", "q16"): "w16-body-kv-q16", ("int16", "q8"): "w16-body-kv-q8", ("int16", "q8r"): "w16-body-kv-q8r",
    ("int16", "q4r"): "w16-body-kv-q4r",
    ("int8", "compact"): "w8-body", ("int8", "f32-split"): "w8-body-split-f32", ("int8", "q16"): "w8-body-kv-q16",
    ("int8", "q8"): "w8-body-kv-q8", ("int8", "q8r"): "w8-body-kv-q8r", ("int8", "q4r"): "w8-body-kv-q4r",
}


@dataclass(frozen=True)
class Profile:
    """A weight and KV storage pair; labels are the strings packed files record
    (Profile::label, quant/mod.rs:122-142)."""

    weights: str
    kv: str

    def label(self) -> str:
        return _PROFILE_LABELS[(self.weights, self.kv)]

    @staticmethod
    def parse(label: str) -> Optional["Profile"]:
        for (w, kv), name in _PROFILE_LABELS.items():
            if name == label:
                return Profile(w, kv)
        return None

    def weight_bits(self) -> int:
        return {"f32": 32, "int16": 16, "int8": 8}[self.weights]

    def quantizes_body(self) -> bool:
        return self.weights != "f32"

    def kv_bits(self) -> Optional[int]:
        """The sealed record width this profile's cache uses on the `hip`
        backend: 8 (Q8), 16 (Q16), 32 (compact FP32), None where the format is
        not built here (F32 split, rotated Q8 / Q4)."""
        return {"compact": 32, "q16": 16, "q8": 8}.get(self.kv)


ALL_PROFILES = [Profile(w, kv) for w in WEIGHTS for kv in KVS]


class PackedFormat(enum.Enum):
    FP32 = PACKED_FORMAT_FP32
    QUANTIZED = PACKED_FORMAT
    QUANTIZED_EXCEPTIONS = PACKED_FORMAT_EXCEPTIONS

    @property
    def tag(self) -> str:
        return self.value

    @property
    def quantized(self) -> bool:
        return self is not PackedFormat.FP32


def packed_format(meta: Dict[str, str]) -> Optional[PackedFormat]:
    """The body layout a file's `format` tag names (packed.rs:333-341)."""
    try:
        return PackedFormat(meta.get("format"))
    except ValueError:
        return None


def packed_profile_of(meta: Dict[str, str], fmt: PackedFormat) -> Profile:
    """The stored profile, FP32 weights required for the FP32 format
    (packed.rs:343-353)."""
    label = meta.get("profile")
    _ensure(label is not None, "packed metadata profile missing")
    profile = Profile.parse(label)
    _ensure(profile is not None, f"packed profile: invalid value '{label}'")
    _ensure(fmt is not PackedFormat.FP32 or profile.weights == "f32", "packed weight format")
    return profile


def validate_weight_format(meta: Dict[str, str], fmt: PackedFormat, profile: Profile) -> None:
    """The weight bits and group metadata agree with the format (packed.rs:355-370)."""
    bits = meta.get("weight_bits")
    _ensure(bits is not None, "packed metadata weight_bits missing")
    try:
        bits = int(bits)
    except ValueError:
        raise _err("packed metadata weight_bits") from None
    if fmt is PackedFormat.FP32:
        matches = profile.weights == "f32" and "group_size" not in meta
    else:
        matches = profile.quantizes_body() and meta.get("group_size") == "64"
    _ensure(bits == profile.weight_bits() and matches, "packed weight format")


def body_shapes(c: ModelConfig) -> List[Tuple[int, int]]:
    """(out, in) of each matrix in BODY (packed.rs:372-380)."""
    return [(c.query_dim() + 2 * c.kv_dim(), c.dim), (c.dim, c.query_dim()), (2 * c.ffn_dim, c.dim),
            (c.dim, c.ffn_dim)]


def packed_order(c: ModelConfig, fmt: PackedFormat, exceptions: Callable[[str], bool]) -> List[str]:
    """Tensor names in the order write_packed hashes them (packed.rs:536-565)."""
    names = ["tok_embeddings.weight", "img_projector.weight", "norm.weight", "output.weight", "freqs_cis_golden"]
    for i in range(c.n_layers):
        names.append(f"layers.{i}.attention.sinks")
        for name in BODY:
            prefix = f"layers.{i}.{name}"
            if fmt is PackedFormat.FP32:
                names.append(f"{prefix}.weight")
                continue
            names += [f"{prefix}.__codes", f"{prefix}.__scales"]
            if exceptions(prefix):
                names += [prefix + s for s in EXCEPTION_SUFFIXES]
    return names + ["output.__screen_codes", "output.__screen_scales"]


def _byte_view(data) -> memoryview:
    """The bytes of a bytes-like object or a numpy array, without a copy."""
    if isinstance(data, np.ndarray):
        return memoryview(np.ascontiguousarray(data).reshape(-1).view(np.uint8))
    return memoryview(data).cast("B")


def packed_digest(tensors: Iterable[Tuple[str, bytes]]) -> str:
    """SHA-256 over each tensor's name and bytes, each preceded by its length
    as a little-endian u64, in the given order (packed.rs:567-577)."""
    h = hashlib.sha256()
    for name, data in tensors:
        raw = name.encode()
        mv = _byte_view(data)
        h.update(struct.pack("<Q", len(raw)))
        h.update(raw)
        h.update(struct.pack("<Q", mv.nbytes))
        h.update(mv)
    return h.hexdigest()


# ---- safetensors -------------------------------------------------------------
def safetensors_header(path) -> dict:
    """The header JSON, read without touching the tensors (packed.rs:486-499)."""
    with open(path, "rb") as f:
        prefix = f.read(8)
        _ensure(len(prefix) == 8, "safetensors header length missing")
        length = struct.unpack("<Q", prefix)[0]
        _ensure(length <= HEADER_LIMIT, f"safetensors header of {length} bytes")
        raw = f.read(length)
        _ensure(len(raw) == length, "safetensors header truncated")
    try:
        header = json.loads(raw)
    except ValueError as e:
        raise _err(f"safetensors header: {e}") from None
    _ensure(isinstance(header, dict), "safetensors header is not an object")
    return header


def header_metadata(header: dict) -> Dict[str, str]:
    meta = header.get("__metadata__") or {}
    _ensure(isinstance(meta, dict) and all(isinstance(v, str) for v in meta.values()), "safetensors metadata")
    return dict(meta)


@dataclass(frozen=True)
class TensorInfo:
    dtype: str
    shape: Tuple[int, ...]
    start: int  # absolute file offset
    end: int


class SafeTensorsFile:
    """A safetensors file mapped read-only; tensors are numpy views of the
    mapping (no copy). Checks what the reference's deserializer checks:
    known dtypes, byte sizes that match the shapes, offsets inside the file,
    tensors that neither overlap nor leave gaps."""

    def __init__(self, path):
        self.path = Path(path)
        self.header = safetensors_header(self.path)
        self.metadata = header_metadata(self.header)
        size = self.path.stat().st_size
        with open(self.path, "rb") as f:
            base = 8 + struct.unpack("<Q", f.read(8))[0]
        infos: Dict[str, TensorInfo] = {}
        spans = []
        for name, entry in self.header.items():
            if name == "__metadata__":
                continue
            try:
                dtype, shape, (lo, hi) = entry["dtype"], tuple(int(s) for s in entry["shape"]), entry["data_offsets"]
            except (KeyError, TypeError, ValueError):
                raise _err(f"safetensors entry {name}") from None
            _ensure(dtype in DTYPES, f"safetensors dtype {dtype} of {name}")
            _ensure(0 <= lo <= hi and base + hi <= size, f"safetensors offsets of {name}")
            _ensure(hi - lo == math.prod(shape) * DTYPES[dtype].itemsize, f"safetensors size of {name}")
            infos[name] = TensorInfo(dtype, shape, base + lo, base + hi)
            spans.append((lo, hi))
        spans.sort()
        at = 0
        for lo, hi in spans:
            _ensure(lo == at, "safetensors tensors overlap or leave gaps")
            at = hi
        self.infos = infos
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r") if size > base else np.zeros(0, np.uint8)

    def names(self) -> List[str]:
        return list(self.infos)

    def has(self, name: str) -> bool:
        return name in self.infos

    def raw(self, name: str) -> np.ndarray:
        info = self.infos[name]
        return self._map[info.start:info.end]

    def tensor(self, name: str, dtype: str, shape: Sequence[int]) -> np.ndarray:
        """tensor_range (packed.rs:382-398): the named tensor, which must have
        `dtype` and `shape`, as a view of the mapping."""
        info = self.infos.get(name)
        _ensure(info is not None, f"packed tensor {name} missing")
        _ensure(info.dtype == dtype and info.shape == tuple(shape),
                f"packed tensor {name}: {info.dtype} {list(info.shape)}")
        return self.raw(name).view(DTYPES[dtype]).reshape(info.shape)


def serialize(tensors: Sequence[Tuple[str, str, Sequence[int], np.ndarray]], metadata: Optional[Dict[str, str]],
              path) -> None:
    """Write a safetensors file. Tensors are laid out by element size
    (largest first), then name, so every tensor is aligned to its element
    size; the header is padded with spaces to a multiple of 8 bytes."""
    order = sorted(tensors, key=lambda t: (-DTYPES[t[1]].itemsize, t[0]))
    header: dict = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    at = 0
    blobs = []
    for name, dtype, shape, data in order:
        arr = np.ascontiguousarray(data)
        nbytes = arr.nbytes
        _ensure(nbytes == math.prod(shape) * DTYPES[dtype].itemsize, f"tensor {name} size")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [at, at + nbytes]}
        blobs.append(arr)
        at += nbytes
    raw = json.dumps(header, separators=(",", ":")).encode()
    raw += b" " * (-len(raw) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        for arr in blobs:
            f.write(_byte_view(arr))


# ---- body matrices -----------------------------------------------------------
@dataclass
class MappedMatrix:
    """One body matrix as the file holds it: codes [out][in] (int8 / int16)
    or FP32 weights, scales [out][in/64], optional exception columns and their
    values [out][count]; all views of the mapping."""

    prefix: str
    bits: int
    codes: np.ndarray
    scales: Optional[np.ndarray] = None
    exc_cols: Optional[np.ndarray] = None
    exc_vals: Optional[np.ndarray] = None

    def upload(self, ctx=None) -> Linear:
        if self.bits == 32:
            return Linear(32, self.codes, None, 32, ctx=ctx)
        return QuantLinear(self.bits, self.codes, self.scales, 64, exc_cols=self.exc_cols, exc_vals=self.exc_vals,
                           ctx=ctx)


def check_exception_columns(columns: np.ndarray, in_dim: int) -> None:
    """QuantLinear::check_exception_columns (src/quant/linear.rs:408-421)."""
    _ensure(len(columns) > 0, "empty exception column set")
    c = columns.astype(np.int64)
    _ensure(bool(np.all(c[1:] > c[:-1])), "exception columns must be sorted and unique")
    _ensure(c[0] >= 0 and c[-1] < in_dim, f"exception column outside the {in_dim} inputs")


def map_matrix(st: SafeTensorsFile, prefix: str, shape: Tuple[int, int], bits: int, exceptions: bool) -> MappedMatrix:
    """map_matrix (packed.rs:425-465): codes and scales of `prefix`, with its
    exception columns when the file has any (format v2 only)."""
    out, inp = shape
    code_dtype = "I8" if bits == 8 else "I16"
    codes = st.tensor(f"{prefix}.__codes", code_dtype, (out, inp))
    _ensure(inp % 64 == 0, f"packed matrix {prefix}: inputs not a multiple of the group")
    scales = st.tensor(f"{prefix}.__scales", "F32", (out, inp // 64))
    cols_name, vals_name = (prefix + s for s in EXCEPTION_SUFFIXES)
    m = MappedMatrix(prefix, bits, codes, scales)
    if not st.has(cols_name):
        _ensure(not st.has(vals_name), f"packed tensor {vals_name} without {cols_name}")
        return m
    _ensure(exceptions, f"packed tensor {cols_name} needs the format {PACKED_FORMAT_EXCEPTIONS}")
    info = st.infos[cols_name]
    count = info.shape[0] if len(info.shape) >= 1 else 0
    cols = st.tensor(cols_name, "I32", (count,))
    check_exception_columns(cols, inp)
    vals = st.tensor(vals_name, "F32", (out, count))
    _ensure(bool(np.all(np.isfinite(vals))), "nonfinite exception value")
    m.exc_cols, m.exc_vals = cols, vals
    return m


# ---- the model file ----------------------------------------------------------
@dataclass
class PackedLayer:
    qkv: object
    wo: object
    w13: object
    w2: object
    sinks: object  # device tensor [n_heads] (host view before upload)


@dataclass
class PackedModel:
    """A kernel-ready file mapped and uploaded: the hot path's matrices,
    sinks, FP32 head and INT8 screen on the device; the rest host views."""

    path: Path
    config: ModelConfig
    profile: Profile
    format: PackedFormat
    layers: List[PackedLayer]
    head: object  # Linear (bits 32) or the host view
    screen: object  # ScreenedHead or (codes, scales, weight_abs_max, kappa)
    embedding: np.ndarray
    projector: np.ndarray
    norm: np.ndarray
    golden: np.ndarray
    overlay_sha256: Optional[str]
    file: SafeTensorsFile

    def body_bits(self) -> Optional[int]:
        return None if self.format is PackedFormat.FP32 else self.profile.weight_bits()

    def free(self) -> None:
        for layer in self.layers:
            for lin in (layer.qkv, layer.wo, layer.w13, layer.w2):
                if hasattr(lin, "free"):
                    lin.free()
        for obj in (self.head, self.screen):
            if hasattr(obj, "free"):
                obj.free()


def packed_profile(path) -> Profile:
    """Model::packed_profile (packed.rs:182-188): the profile from the header
    alone."""
    meta = header_metadata(safetensors_header(path))
    fmt = packed_format(meta)
    _ensure(fmt is not None, f"{path} is not a kernel-ready file")
    return packed_profile_of(meta, fmt)


def packed_facts(path) -> Tuple[ModelConfig, Optional[str], int]:
    """packed_facts (packed.rs:471-480): config, overlay digest and the bytes
    of exception tensors, from the header alone."""
    header = safetensors_header(path)
    meta = header_metadata(header)
    _ensure("config" in meta, "packed metadata config missing")
    config = ModelConfig.from_json(meta["config"])
    config.validate()
    exc = 0
    for name, info in header.items():
        if name != "__metadata__" and any(name.endswith(s) for s in EXCEPTION_SUFFIXES):
            lo, hi = info.get("data_offsets", [0, 0])
            exc += max(0, hi - lo)
    return config, meta.get("w8_artifact_sha256"), exc


def load_packed(path, verify: bool = False, upload: bool = True, ctx=None) -> PackedModel:
    """Model::load_packed (packed.rs:190-310) for the `hip` backend: every
    check of the reference, then (with `upload`) one upload per matrix, the
    screen and the FP32 head. `verify` recomputes the tensor digest."""
    st = SafeTensorsFile(path)
    meta = st.metadata
    _ensure(bool(meta), "packed model metadata missing")

    def get(key: str) -> str:
        _ensure(key in meta, f"packed metadata {key} missing")
        return meta[key]

    fmt = packed_format(meta)
    _ensure(fmt is not None, "not a kernel-ready file")
    _ensure(get("source_sha256") == WEIGHTS_SHA256, "packed file comes from another checkpoint")
    _ensure(get("model_revision") == MODEL_REVISION, "packed file comes from another revision")
    config = ModelConfig.from_json(get("config"))
    config.validate()
    profile = packed_profile_of(meta, fmt)
    validate_weight_format(meta, fmt, profile)
    bits = profile.weight_bits()

    def constant(key: str) -> float:
        # f32::from_bits(u32::from_str_radix(value, 16)): up to 8 hex digits.
        text = get(key)
        _ensure(re.fullmatch(r"\+?[0-9a-fA-F]{1,8}", text) is not None, f"packed metadata {key}")
        return float(np.array([int(text, 16)], dtype=np.uint32).view(np.float32)[0])

    c = config
    embedding = st.tensor("tok_embeddings.weight", "F32", (c.vocab_size, c.dim))
    projector = st.tensor("img_projector.weight", "F32", (c.dim, c.patch_dim()))
    norm = st.tensor("norm.weight", "F32", (c.dim,))
    output = st.tensor("output.weight", "F32", (c.vocab_size, c.dim))
    golden = st.tensor("freqs_cis_golden", "F32", (c.n_heads, c.head_dim // 4, 2))
    mapped = []
    for i in range(c.n_layers):
        body = []
        for name, shape in zip(BODY, body_shapes(c)):
            prefix = f"layers.{i}.{name}"
            if fmt is PackedFormat.FP32:
                body.append(MappedMatrix(prefix, 32, st.tensor(f"{prefix}.weight", "F32", shape)))
            else:
                body.append(map_matrix(st, prefix, shape, bits, fmt is PackedFormat.QUANTIZED_EXCEPTIONS))
        mapped.append((body, st.tensor(f"layers.{i}.attention.sinks", "F32", (c.n_heads,))))
    screen_codes = st.tensor("output.__screen_codes", "I8", (c.vocab_size, c.dim))
    screen_scales = st.tensor("output.__screen_scales", "F32", (c.vocab_size, c.dim // 64))
    wmax, kappa = constant("screen_weight_abs_max"), constant("screen_kappa")
    if verify:
        names = st.names()
        order = packed_order(c, fmt, lambda m: any(n == m + EXCEPTION_SUFFIXES[0] for n in names))
        _ensure(len(names) == len(order), "packed file has unexpected tensors")
        digest = packed_digest((n, st.raw(n) if st.has(n) else b"") for n in order)
        _ensure(digest == get("tensors_sha256"), "packed tensor digest mismatch")
    layers: List[PackedLayer] = []
    if not upload:
        layers = [PackedLayer(*body, sinks) for body, sinks in mapped]
        return PackedModel(Path(path), config, profile, fmt, layers, output,
                           (screen_codes, screen_scales, wmax, kappa), embedding, projector, norm, golden,
                           meta.get("w8_artifact_sha256"), st)
    import torch

    ctx = ctx or default_context()
    dev = f"cuda:{ctx.device}"
    model = PackedModel(Path(path), config, profile, fmt, layers, None, None, embedding, projector, norm, golden,
                        meta.get("w8_artifact_sha256"), st)
    try:
        for body, sinks in mapped:
            ups = [m.upload(ctx) for m in body]
            layers.append(PackedLayer(*ups, torch.from_numpy(np.array(sinks)).to(dev)))
        model.screen = ScreenedHead.from_parts(screen_codes, screen_scales, wmax, kappa, ctx=ctx)
        model.head = Linear(32, output, None, 32, ctx=ctx)
    except Exception:
        model.free()
        raise
    return model


def _fp32_bits_hex(x: float) -> str:
    return "%08x" % int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def write_packed(path, config: ModelConfig, profile: Profile, embedding, projector, norm, output, golden,
                 layers: Sequence[dict], screen: Tuple[np.ndarray, np.ndarray, float, float],
                 weights_sha256: str = WEIGHTS_SHA256, overlay_sha256: Optional[str] = None) -> str:
    """Model::write_packed (packed.rs:54-179) from host arrays: `layers[i]`
    holds `sinks` and, per BODY name, either an FP32 [out][in] array (FP32
    profile) or a dict {codes, scales[, exc_cols, exc_vals]}; `screen` is
    (codes, scales, weight_abs_max, kappa) as ScreenedHead::raw_parts.
    Returns the tensor digest it records."""
    c = config
    fp32 = profile.weights == "f32"
    has_exc = (not fp32) and any(
        isinstance(layer[name], dict) and layer[name].get("exc_cols") is not None for layer in layers for name in BODY)
    fmt = PackedFormat.FP32 if fp32 else (PackedFormat.QUANTIZED_EXCEPTIONS if has_exc else PackedFormat.QUANTIZED)
    tensors: List[Tuple[str, str, Tuple[int, ...], np.ndarray]] = [
        ("tok_embeddings.weight", "F32", (c.vocab_size, c.dim), embedding),
        ("img_projector.weight", "F32", (c.dim, c.patch_dim()), projector),
        ("norm.weight", "F32", (c.dim,), norm),
        ("output.weight", "F32", (c.vocab_size, c.dim), output),
        ("freqs_cis_golden", "F32", (c.n_heads, c.head_dim // 4, 2), golden),
    ]
    bits = None
    _ensure(len(layers) == c.n_layers, "one entry per layer")
    for i, layer in enumerate(layers):
        tensors.append((f"layers.{i}.attention.sinks", "F32", (c.n_heads,), layer["sinks"]))
        for name, (out, inp) in zip(BODY, body_shapes(c)):
            prefix = f"layers.{i}.{name}"
            w = layer[name]
            if fp32:
                tensors.append((f"{prefix}.weight", "F32", (out, inp), w))
                continue
            _ensure(isinstance(w, dict), f"layer {i} {name} is not quantized")
            codes = np.asarray(w["codes"])
            b = 8 if codes.dtype == np.int8 else 16
            bits = bits or b
            _ensure(b == bits, "mixed packing formats")
            tensors.append((f"{prefix}.__codes", "I8" if b == 8 else "I16", (out, inp), codes))
            tensors.append((f"{prefix}.__scales", "F32", (out, inp // 64), w["scales"]))
            if w.get("exc_cols") is not None:
                cols = np.asarray(w["exc_cols"], dtype=np.int32)
                tensors.append((prefix + EXCEPTION_SUFFIXES[0], "I32", (len(cols),), cols))
                tensors.append((prefix + EXCEPTION_SUFFIXES[1], "F32", (out, len(cols)), w["exc_vals"]))
    codes, scales, wmax, kappa = screen
    tensors.append(("output.__screen_codes", "I8", (c.vocab_size, c.dim), codes))
    tensors.append(("output.__screen_scales", "F32", (c.vocab_size, c.dim // 64), scales))
    arrays = [(n, d, s, np.ascontiguousarray(a, dtype=DTYPES[d])) for n, d, s, a in tensors]
    metadata = {"format": fmt.tag, "profile": profile.label(),
                "weight_bits": str(32 if fp32 else (bits or 8)),
                "source_sha256": weights_sha256, "model_revision": MODEL_REVISION, "config": c.to_json(),
                "screen_weight_abs_max": _fp32_bits_hex(wmax), "screen_kappa": _fp32_bits_hex(kappa)}
    if not fp32:
        metadata["group_size"] = "64"
    if overlay_sha256 is not None:
        metadata["w8_artifact_sha256"] = overlay_sha256
    digest = packed_digest((n, a) for n, _, _, a in arrays)
    metadata["tensors_sha256"] = digest
    serialize(arrays, metadata, path)
    return digest
