"""The C ABI without a GPU: the library loads, exports every entry point that
include/focr_hip.h declares, the Python binding covers exactly those, and
argument checks that precede any device work return their error codes."""
import ctypes
import re
from pathlib import Path

import pytest

import focr_hip

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "focr_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(focr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("focr_linear_upload", "focr_linear_decode", "focr_linear_decode_glu", "focr_linear_prefill",
                     "focr_linear_dequantize", "focr_row_scales", "focr_attention_prefill", "focr_argmax",
                     "focr_linear_decode_ex", "focr_qkv_rows", "focr_attention_decode", "focr_screen_build",
                     "focr_screen_upload", "focr_screen_select", "focr_screen_free", "focr_screen_constants",
                     "focr_kv_seal", "focr_kv_append", "focr_kv_attention_decode", "focr_kv_dequantize"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(focr_hip.LIBRARY))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing


def test_binding_signatures_match_the_header():
    assert sorted(focr_hip.SIGNATURES) == declared_functions()
    focr_hip.load_library()  # binds every signature


def test_null_arguments_are_errors_not_crashes():
    lib = focr_hip.lib()
    assert lib.focr_ctx_sync(None) == -1
    assert "null" in lib.focr_last_error().decode()
    assert lib.focr_linear_info(None, None, None, None, None, None, None) == -1
    assert lib.focr_linear_decode(None, None, None, 1, None) == -1
    assert lib.focr_linear_prefill(None, None, None, 1, None, 0, 0, None) == -1
    assert lib.focr_attention_prefill(None, *([None] * 4), *([0] * 9), None, 0, 0, None) == -1
    assert lib.focr_linear_decode_ex(None, None, None, 1, None, 0, 0, None) == -1
    assert lib.focr_qkv_rows(None, None, 1, None, 16, 8, 64, 0, None, None, None, None) == -1
    assert lib.focr_attention_decode(None, *([None] * 4), *([0] * 9), None, None) == -1
    assert lib.focr_screen_build(None, None, 1, 64, None) == -1
    assert lib.focr_screen_upload(None, None, None, 1, 64, 1.0, 0.5, None) == -1
    assert lib.focr_screen_select(None, None, None, None, 1, None, None) == -1
    assert lib.focr_screen_constants(None, None, None) == -1
    assert lib.focr_ctx_destroy(None) == 0
    assert lib.focr_linear_free(None) == 0
    assert lib.focr_screen_free(None) == 0
    assert lib.focr_kv_seal(None, 8, None, None, 1, 1, 16, 8, 64, None) == -1
    assert lib.focr_kv_append(None, None, None, None, 1) == -1
    assert lib.focr_kv_attention_decode(None, None, None, 1, None, None) == -1
    assert lib.focr_kv_dequantize(None, None, None, None, None) == -1
    assert lib.focr_kv_info(None, None, None, None, None, None) == -1
    assert lib.focr_kv_truncate_tail(None, 0) == -1
    assert lib.focr_kv_set_fast_exp(None, 1) == -1
    assert lib.focr_kv_fast_exp(None, None) == -1
    assert lib.focr_kv_qkv_rows(None, None, None, 1, None, None) == -1
    assert lib.focr_kv_decode_row(None, None, None, None, None, None, None) == -1
    assert lib.focr_attention_decode_row(None, *([None] * 5), *([0] * 7), None, None, None) == -1
    assert lib.focr_kv_free(None) == 0
    assert lib.focr_ctx_reserve_scratch(None, 1) == -1
    assert lib.focr_ctx_scratch_bytes(None, None) == -1


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(focr_hip.FocrError):
        focr_hip.load_library(tmp_path / "libfocr_hip.so")
