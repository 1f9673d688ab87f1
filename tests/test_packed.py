"""The packed model file on the host (focr_hip.packed): the reference's own
packed.rs tests restated (formats and digest order, header-only profiles,
FP32 tensor mapping and the digest's inputs, malformed exception columns,
body matrices with and without exception columns), the safetensors layout
cross-checked with the independent `safetensors` package, and a whole
22-layer file written, mapped and verified. No GPU: nothing is uploaded."""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import gen
from focr_hip import FocrError
from focr_hip import packed as pk

CONFIG_JSON = json.dumps({  # tests/fixtures/model-config.json's values
    "architectures": ["FalconOCRForCausalLM"], "model_type": "falcon_ocr", "torch_dtype": "float32",
    "dim": 768, "n_layers": 22, "n_heads": 16, "head_dim": 64, "n_kv_heads": 8, "vocab_size": 65536,
    "ffn_dim": 2304, "norm_eps": 1e-05, "max_seq_len": 16384, "rope_theta": 10000, "channel_size": 3,
    "spatial_patch_size": 16, "temporal_patch_size": 1, "eos_id": 11, "img_id": 227, "image_cls_token_id": 244,
    "image_reg_1_token_id": 245, "image_reg_2_token_id": 246, "image_reg_3_token_id": 247,
    "image_reg_4_token_id": 248, "img_end_id": 230})


def config():
    c = pk.ModelConfig.from_json(CONFIG_JSON)
    c.validate()
    return c


def test_config_validation_and_round_trip():
    c = config()
    assert pk.ModelConfig.from_json(c.to_json()) == c
    assert (c.query_dim(), c.kv_dim(), c.patch_dim()) == (1024, 512, 768)
    bad = json.loads(CONFIG_JSON)
    bad["n_layers"] = 12
    with pytest.raises(FocrError, match="unsupported architecture"):
        pk.ModelConfig.from_json(json.dumps(bad)).validate()
    bad = json.loads(CONFIG_JSON)
    bad["img_end_id"] = 231
    with pytest.raises(FocrError, match="special token"):
        pk.ModelConfig.from_json(json.dumps(bad)).validate()
    del bad["dim"]
    with pytest.raises(FocrError, match="dim missing"):
        pk.ModelConfig.from_json(json.dumps(bad))


def test_profile_labels_round_trip():
    # Profile::label / parse (quant/mod.rs:122-147, tests 214-226).
    labels = [p.label() for p in pk.ALL_PROFILES]
    assert len(set(labels)) == 18
    for p in pk.ALL_PROFILES:
        assert pk.Profile.parse(p.label()) == p
    assert pk.Profile.parse("reference") == pk.Profile("f32", "compact")
    assert pk.Profile.parse("w8-body-kv-q8").weight_bits() == 8 and pk.Profile.parse("w8-body-kv-q8").kv_bits() == 8
    assert pk.Profile.parse("w16-body").kv_bits() is None
    assert pk.Profile.parse("nope") is None


def test_formats_and_the_digest_order_follow_the_exception_columns():
    # packed.rs:739-797.
    fmt = lambda v: pk.packed_format({"format": v})
    assert fmt(pk.PACKED_FORMAT) is pk.PackedFormat.QUANTIZED
    assert fmt(pk.PACKED_FORMAT_EXCEPTIONS) is pk.PackedFormat.QUANTIZED_EXCEPTIONS
    assert fmt(pk.PACKED_FORMAT_FP32) is pk.PackedFormat.FP32
    assert fmt("falcon-ocr-kernel-v3") is None
    c = config()
    v1 = pk.packed_order(c, pk.PackedFormat.QUANTIZED, lambda _: False)
    assert len(v1) == 5 + 22 * 9 + 2
    assert v1[5:8] == ["layers.0.attention.sinks", "layers.0.attention.wqkv.__codes",
                       "layers.0.attention.wqkv.__scales"]
    v2 = pk.packed_order(c, pk.PackedFormat.QUANTIZED_EXCEPTIONS, lambda m: m == "layers.3.feed_forward.w2")
    assert len(v2) == len(v1) + 2
    at = v2.index("layers.3.feed_forward.w2.__scales")
    assert v2[at + 1:at + 4] == ["layers.3.feed_forward.w2.__exc_cols", "layers.3.feed_forward.w2.__exc_vals",
                                 "layers.4.attention.sinks"]
    fp32 = pk.packed_order(c, pk.PackedFormat.FP32, lambda _: pytest.fail("FP32 has no exception columns"))
    assert len(fp32) == 5 + 22 * 5 + 2
    assert fp32[5:11] == ["layers.0.attention.sinks", "layers.0.attention.wqkv.weight", "layers.0.attention.wo.weight",
                          "layers.0.feed_forward.w13.weight", "layers.0.feed_forward.w2.weight",
                          "layers.1.attention.sinks"]
    assert fp32[-2:] == ["output.__screen_codes", "output.__screen_scales"]


def write_header(path, meta):
    raw = json.dumps({"__metadata__": meta}).encode()
    path.write_bytes(struct.pack("<Q", len(raw)) + raw)


def test_fp32_header_profiles_require_fp32_body_metadata(tmp_path):
    # packed.rs:800-841.
    path = tmp_path / "header.safetensors"
    for profile in pk.ALL_PROFILES:
        write_header(path, {"format": pk.PACKED_FORMAT_FP32, "profile": profile.label(),
                            "weight_bits": str(profile.weight_bits()), "config": CONFIG_JSON})
        if profile.weights == "f32":
            assert pk.packed_profile(path) == profile
            assert pk.packed_facts(path)[2] == 0
        else:
            with pytest.raises(FocrError):
                pk.packed_profile(path)
    meta = {"profile": "reference", "weight_bits": "32"}
    assert pk.packed_profile_of(meta, pk.PackedFormat.FP32) == pk.Profile("f32", "compact")
    with pytest.raises(FocrError):
        pk.validate_weight_format(meta, pk.PackedFormat.QUANTIZED, pk.Profile("f32", "compact"))
    with pytest.raises(FocrError):
        pk.validate_weight_format({**meta, "weight_bits": "16"}, pk.PackedFormat.FP32, pk.Profile("f32", "compact"))
    with pytest.raises(FocrError):
        pk.validate_weight_format({**meta, "group_size": "64"}, pk.PackedFormat.FP32, pk.Profile("f32", "compact"))
    assert pk.packed_profile_of({"profile": "w16-body-kv-q16"}, pk.PackedFormat.QUANTIZED) == \
        pk.Profile("int16", "q16")
    # The header-length cap and truncation.
    path.write_bytes(struct.pack("<Q", (64 << 20) + 1))
    with pytest.raises(FocrError, match="header of"):
        pk.safetensors_header(path)
    path.write_bytes(struct.pack("<Q", 100) + b"{}")
    with pytest.raises(FocrError, match="truncated"):
        pk.safetensors_header(path)


def test_fp32_body_tensor_mapping_preserves_bits_and_digest(tmp_path):
    # packed.rs:843-878: bits survive the mapping; name, payload and order all
    # enter the digest.
    name = "layers.0.attention.wo.weight"
    data = np.array([0, 0x80000000, 0x7FC00123, 0x7F800000, 0x3F800000, 0xBF800000], np.uint32).view(np.float32)
    path = tmp_path / "one.safetensors"
    pk.serialize([(name, "F32", (2, 3), data.reshape(2, 3))], None, path)
    st = pk.SafeTensorsFile(path)
    got = st.tensor(name, "F32", (2, 3))
    assert got.view(np.uint32).tobytes() == data.view(np.uint32).tobytes()
    with pytest.raises(FocrError):
        st.tensor(name, "I16", (2, 3))
    with pytest.raises(FocrError):
        st.tensor(name, "F32", (3, 2))
    raw = data.tobytes()
    digest = pk.packed_digest([(name, raw)])
    assert digest == pk.packed_digest([(name, st.raw(name))])
    assert digest != pk.packed_digest([("layers.0.attention.wo.__codes", raw)])
    changed = bytearray(raw)
    changed[0] ^= 1
    assert digest != pk.packed_digest([(name, bytes(changed))])
    assert pk.packed_digest([(name, raw), ("norm.weight", bytes(changed))]) != \
        pk.packed_digest([("norm.weight", bytes(changed)), (name, raw)])
    # Moving a byte from the name to the payload changes the digest (lengths are hashed).
    assert pk.packed_digest([("ab", b"c")]) != pk.packed_digest([("a", b"bc")])


def test_safetensors_layout_agrees_with_the_safetensors_package(tmp_path):
    st_np = pytest.importorskip("safetensors.numpy")
    arrays = {"a.f32": gen.normal((3, 5), 1.0, 1), "b.i8": np.arange(-7, 7, dtype=np.int8).reshape(2, 7),
              "c.i16": np.arange(12, dtype=np.int16).reshape(3, 4), "d.i32": np.array([5, 64], np.int32)}
    dt = {np.float32: "F32", np.int8: "I8", np.int16: "I16", np.int32: "I32"}
    ours = tmp_path / "ours.safetensors"
    pk.serialize([(k, dt[v.dtype.type], v.shape, v) for k, v in arrays.items()], {"format": "x"}, ours)
    back = st_np.load_file(str(ours))
    for k, v in arrays.items():
        assert back[k].dtype == v.dtype and np.array_equal(back[k], v)
    theirs = tmp_path / "theirs.safetensors"
    st_np.save_file(arrays, str(theirs), metadata={"format": "y"})
    f = pk.SafeTensorsFile(theirs)
    assert f.metadata == {"format": "y"}
    for k, v in arrays.items():
        assert np.array_equal(f.tensor(k, dt[v.dtype.type], v.shape), v)
    # Every tensor of our layout is aligned to its element size.
    for k, info in pk.SafeTensorsFile(ours).infos.items():
        assert info.start % pk.DTYPES[info.dtype].itemsize == 0, k


def quantize_rows(w):
    """RTN W8 group-64 codes and scales (absmax / 127 in f64, ties to even):
    test data only."""
    out, inp = w.shape
    g = w.reshape(out, inp // 64, 64).astype(np.float64)
    amax = np.abs(g).max(-1)
    scale = (amax / 127.0).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        codes = np.where(scale[..., None] > 0, np.rint(g / scale[..., None].astype(np.float64)), 0)
    return np.clip(codes, -127, 127).astype(np.int8).reshape(out, inp), scale


def matrix_file(path, prefix, codes, scales, columns=None, values=None):
    out, inp = codes.shape
    tensors = [(f"{prefix}.__codes", "I8", (out, inp), codes), (f"{prefix}.__scales", "F32", scales.shape, scales)]
    if columns is not None:
        tensors.append((prefix + ".__exc_cols",) + columns)
    if values is not None:
        tensors.append((prefix + ".__exc_vals",) + values)
    pk.serialize(tensors, None, path)
    return pk.SafeTensorsFile(path)


def test_malformed_exception_columns_are_refused(tmp_path):
    # packed.rs:656-737.
    out, inp = 16, 128
    w = ((np.arange(out * inp) * 7919 % 2003).astype(np.float32) - 1001.0) / 977.0
    codes, scales = quantize_rows(w.reshape(out, inp))
    prefix = "layers.0.feed_forward.w2"
    cols = lambda v: ("I32", (len(v),), np.array(v, dtype=np.int64).astype(np.int32))
    vals = lambda r, k: ("F32", (r, k), (np.arange(r * k, dtype=np.float32) * 0.5).reshape(r, k))
    cases = [
        ("valid", cols([5, 64]), vals(out, 2), True),
        ("unsorted", cols([64, 5]), vals(out, 2), False),
        ("duplicate", cols([5, 5]), vals(out, 2), False),
        ("negative", cols([-1, 5]), vals(out, 2), False),
        ("out of range", cols([5, 128]), vals(out, 2), False),
        ("i32 max", cols([5, 2 ** 31 - 1]), vals(out, 2), False),
        ("empty", cols([]), vals(out, 0), False),
        ("more than the inputs", cols(list(range(129))), vals(out, 129), False),
        ("values k", cols([5, 64]), vals(out, 3), False),
        ("values rows", cols([5, 64]), vals(out + 1, 2), False),
        ("values 1-d", cols([5, 64]), ("F32", (out * 2,), np.zeros(out * 2, np.float32)), False),
        ("values F16", cols([5, 64]), ("F16", (out, 2), np.zeros((out, 2), np.float16)), False),
        ("values missing", cols([5, 64]), None, False),
        ("columns missing", None, vals(out, 2), False),
        ("columns I64", ("I64", (2,), np.array([5, 64], np.int64)), vals(out, 2), False),
        ("columns 2-d", ("I32", (1, 2), np.array([[5, 64]], np.int32)), vals(out, 2), False),
        ("columns 0-d", ("I32", (), np.array(5, np.int32)), vals(out, 1), False),
    ]
    for i, (label, c, v, ok) in enumerate(cases):
        st = matrix_file(tmp_path / f"m{i}.safetensors", prefix, codes, scales, c, v)
        if ok:
            m = pk.map_matrix(st, prefix, (out, inp), 8, True)
            assert m.exc_cols.tolist() == [5, 64]
        else:
            with pytest.raises(FocrError):
                pk.map_matrix(st, prefix, (out, inp), 8, True)
    # Format v1 refuses exception columns; shapes are checked.
    st = matrix_file(tmp_path / "v1.safetensors", prefix, codes, scales, cols([5, 64]), vals(out, 2))
    with pytest.raises(FocrError, match=pk.PACKED_FORMAT_EXCEPTIONS):
        pk.map_matrix(st, prefix, (out, inp), 8, False)
    with pytest.raises(FocrError):
        pk.map_matrix(st, prefix, (out, 2 * inp), 8, True)
    plain = matrix_file(tmp_path / "plain.safetensors", prefix, codes, scales)
    m = pk.map_matrix(plain, prefix, (out, inp), 8, False)
    assert m.exc_cols is None and np.array_equal(m.codes, codes) and np.array_equal(m.scales, scales)


def small_model(seed=0, exceptions=False):
    """Every tensor of a 22-layer INT8 model at checkpoint shapes, cheap
    deterministic contents (host arrays; about 640 MB)."""
    c = config()
    rng = np.random.default_rng(seed)
    shapes = pk.body_shapes(c)
    layers = []
    for i in range(c.n_layers):
        layer = {"sinks": rng.uniform(-2, 2, c.n_heads).astype(np.float32)}
        for name, (out, inp) in zip(pk.BODY, shapes):
            codes = rng.integers(-127, 128, (out, inp), dtype=np.int8)
            entry = {"codes": codes, "scales": rng.uniform(1e-4, 4e-4, (out, inp // 64)).astype(np.float32)}
            if exceptions and i == 3 and name == "feed_forward.w2":
                entry["codes"] = codes.copy()
                entry["codes"][:, [5, 700]] = 0
                entry["exc_cols"] = np.array([5, 700], np.int32)
                entry["exc_vals"] = rng.normal(0, 0.1, (out, 2)).astype(np.float32)
            layer[name] = entry
        layers.append(layer)
    emb = np.full((c.vocab_size, c.dim), 0.25, np.float32)
    out = rng.normal(0, 0.02, (c.vocab_size, c.dim)).astype(np.float32)
    screen = (rng.integers(-127, 128, (c.vocab_size, c.dim), dtype=np.int8),
              rng.uniform(1e-5, 2e-4, (c.vocab_size, c.dim // 64)).astype(np.float32), 0.125, 0.0078125)
    return dict(config=c, profile=pk.Profile("int8", "q8"), embedding=emb,
                projector=np.ones((c.dim, c.patch_dim()), np.float32), norm=np.ones(c.dim, np.float32),
                output=out, golden=np.zeros((c.n_heads, c.head_dim // 4, 2), np.float32), layers=layers,
                screen=screen)


@pytest.fixture(scope="module")
def packed_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("packed") / "model.safetensors"
    parts = small_model(1, exceptions=True)
    digest = pk.write_packed(path, **parts)
    return path, parts, digest


def test_whole_file_maps_in_place_and_verifies(packed_file):
    path, parts, digest = packed_file
    assert pk.packed_profile(path) == pk.Profile("int8", "q8")
    cfg, overlay, exc_bytes = pk.packed_facts(path)
    assert cfg == parts["config"] and overlay is None and exc_bytes == 2 * 4 + 768 * 2 * 4
    model = pk.load_packed(path, verify=True, upload=False)
    assert model.format is pk.PackedFormat.QUANTIZED_EXCEPTIONS and model.body_bits() == 8
    assert model.file.metadata["tensors_sha256"] == digest
    layer = model.layers[3]
    src = parts["layers"][3]
    assert np.array_equal(layer.w2.codes, src["feed_forward.w2"]["codes"])
    assert layer.w2.exc_cols.tolist() == [5, 700]
    assert np.array_equal(layer.w2.exc_vals, src["feed_forward.w2"]["exc_vals"])
    assert layer.qkv.exc_cols is None
    assert np.array_equal(layer.sinks, src["sinks"])
    codes, scales, wmax, kappa = model.screen
    assert (wmax, kappa) == (0.125, 0.0078125)
    assert np.array_equal(codes, parts["screen"][0])
    # The mapping is the file: no copy.
    assert isinstance(layer.qkv.codes.base, np.memmap) or layer.qkv.codes.base is not None


def test_digest_and_metadata_refusals(packed_file, tmp_path):
    import shutil

    path, parts, _ = packed_file
    st = pk.SafeTensorsFile(path)
    at = st.infos["layers.21.feed_forward.w13.__codes"].start + 12345
    bad = tmp_path / "bad.safetensors"
    shutil.copyfile(path, bad)
    with open(bad, "r+b") as f:
        f.seek(at)
        byte = f.read(1)
        f.seek(at)
        f.write(bytes([byte[0] ^ 1]))
    pk.load_packed(bad, verify=False, upload=False)  # mapped without a check
    with pytest.raises(FocrError, match="digest mismatch"):
        pk.load_packed(bad, verify=True, upload=False)
    with open(path, "rb") as f:
        length = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(length))

    def with_meta(**changes):
        h = json.loads(json.dumps(header))
        h["__metadata__"].update({k: v for k, v in changes.items() if v is not None})
        for k in [k for k, v in changes.items() if v is None]:
            del h["__metadata__"][k]
        text = json.dumps(h, separators=(",", ":")).encode()
        text += b" " * (-len(text) % 8)
        with open(path, "rb") as src, open(bad, "wb") as dst:
            dst.write(struct.pack("<Q", len(text)) + text)
            src.seek(8 + length)
            shutil.copyfileobj(src, dst, 1 << 24)
        return bad

    for changes, msg in [({"source_sha256": "0" * 64}, "another checkpoint"),
                         ({"model_revision": "x"}, "another revision"),
                         ({"format": pk.PACKED_FORMAT}, "needs the format"),
                         ({"format": "falcon-ocr-kernel-v3"}, "not a kernel-ready file"),
                         ({"weight_bits": "16"}, "packed weight format"),
                         ({"group_size": None}, "packed weight format"),
                         ({"profile": "kv-q8"}, "packed weight format"),
                         ({"screen_kappa": "xyz"}, "screen_kappa"),
                         ({"tensors_sha256": None}, "tensors_sha256 missing")]:
        with pytest.raises(FocrError, match=msg):
            pk.load_packed(with_meta(**changes), verify=True, upload=False)
    # Rewritten with the original metadata: loads and verifies.
    pk.load_packed(with_meta(), verify=True, upload=False)


def test_hip_prefill_plan_follows_the_reference_predicates():
    # prefill_plan (kernels/mod.rs:203-259) with the `hip` kernels, and the
    # labels a page record stores (kernels/mod.rs:156-180).
    from focr_hip import PrefillProjection, Softmax
    from focr_hip.plan import HipPrefillPlan, hip_prefill_plan

    fast = hip_prefill_plan(8, False)  # fast mode: INT16 panels, BF16 static attention
    assert fast.labels() == {"projection": "hip-i16", "attention": "hip-bf16-static"}
    assert fast.bf16() and fast.softmax() == Softmax.STATIC
    assert hip_prefill_plan(8, False, prefill_softmax="online").attention == "hip-bf16"
    assert hip_prefill_plan(8, True).projection == PrefillProjection.F32_CHAIN  # misfit: FP32 panels
    assert hip_prefill_plan(8, False, prefill_projections="fp32").projection == PrefillProjection.F32_CHAIN
    assert hip_prefill_plan(8, False, prefill_bf16=False).attention == "hip"  # 8-bit FP32 tiles: online
    assert hip_prefill_plan(8, False, prefill_bf16=False, prefill_softmax_fp32="static").attention == "hip-static"
    near = hip_prefill_plan(16, False)  # near-exact: FP32 panels, static FP32 tiles
    assert near.labels() == {"projection": "hip-f32-chain", "attention": "hip-static"}
    assert hip_prefill_plan(16, False, prefill_softmax_fp32="online").attention == "hip"
    exact = hip_prefill_plan(None, False, prefill_softmax_fp32="static")  # FP32 bodies keep online
    assert exact.labels() == {"projection": "hip-f32-split", "attention": "hip"}
    mfma = HipPrefillPlan(PrefillProjection.F32_MFMA, "hip")
    assert mfma.labels() == {"projection": "hip-f32-mfma", "attention": "hip"}
    for plan in (fast, near, exact, mfma):
        assert HipPrefillPlan.from_labels(plan.labels()) == plan
    with pytest.raises(FocrError):
        HipPrefillPlan.from_labels({"projection": "panel-avx2", "attention": "avx2"})
    with pytest.raises(FocrError):
        hip_prefill_plan(8, False, prefill_softmax="fast")
