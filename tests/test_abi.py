"""The drop-in boundary without a GPU: libjepa.so loads, exports every function include/jepa.h and
include/jepa_amd.h declare, and fails cleanly (NULL / -1 plus jepa_error_text) on bad inputs that are
rejected before any device work (reference tests/test-errors.cpp covers the same error paths)."""
import ctypes as C
import os
import re
import struct

import pytest

from jepa_amd import _lib, forge

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("jepa.h", "jepa_amd.h")]
DECL = re.compile(r"^[A-Za-z_][\w \t\*]*?\b(jepa_\w+)\s*\(", re.M)


def declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in DECL.finditer(text):
            line = text[m.start():text.find("\n", m.start())]
            if line.lstrip().startswith(("typedef", "#")):
                continue
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_headers_declare_the_reference_api():
    names = declared()
    assert len(names) > 110
    for fn in ("jepa_model_load", "jepa_context_new", "jepa_encode", "jepa_free", "jepa_model_load_ex",
               "jepa_error_text", "jepa_amd_encode_device", "jepa_amd_matmul"):
        assert fn in names


def test_library_exports_every_declared_function(L):
    missing = [fn for fn in sorted(declared()) if not hasattr(L, fn)]
    assert not missing, missing


def _load(L, path):
    L.jepa_model_load.restype = C.c_void_p
    L.jepa_model_load.argtypes = [C.c_char_p, C.c_bool]
    return L.jepa_model_load(path.encode(), False)


def test_missing_file_is_rejected(L, tmp_path):
    assert _load(L, str(tmp_path / "nope.gguf")) is None
    assert "nope.gguf" in _lib.error_text()


@pytest.mark.parametrize("blob", [b"", b"GGUF", b"XXXX" + b"\0" * 60,
                                  b"GGUF" + struct.pack("<IQQ", 3, 1 << 40, 0),     # absurd tensor count
                                  b"GGUF" + struct.pack("<IQQ", 9, 0, 0)])          # unknown version
def test_malformed_gguf_is_rejected(L, tmp_path, blob):
    p = tmp_path / "bad.gguf"
    p.write_bytes(blob)
    assert _load(L, str(p)) is None
    assert _lib.error_text().strip()


def test_truncated_model_is_rejected(L, tmp_path):
    src = forge.cached_model(forge.tiny("vjepa2", "q8_0"), str(tmp_path))
    data = open(src, "rb").read()
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[: len(data) // 2])
    assert _load(L, str(p)) is None


def test_null_arguments(L):
    L.jepa_encode.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    assert L.jepa_encode(None, None, None) == -1
    L.jepa_context_new.restype = C.c_void_p
    assert L.jepa_context_new(None, _lib.ContextParams()) is None
    L.jepa_model_free(None)          # accepted, like free(NULL)
    L.jepa_context_free(None)


def test_out_of_scope_entry_points_report_and_fail(L):
    """Everything beyond the encoder path is exported but returns its failure value with a message."""
    L.jepa_predict.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    L.jepa_predict.restype = C.c_int
    assert L.jepa_predict(None, None, None, 0, None, 0, None) == -1


def test_versions_and_defaults(L):
    L.jepa_version.restype = C.c_char_p
    assert L.jepa_version()
    L.jepa_model_default_params.restype = _lib.ModelParams
    p = L.jepa_model_default_params()
    assert p.device >= -1


def test_gemm_tile_hook_is_host_only(L):
    assert L.jepa_amd_gemm_tile(99) == -1
    assert L.jepa_amd_gemm_tile(-1) == 0
