"""Host-side entry points of include/jepa.h that need no GPU: the classifier helpers (jepa_softmax,
jepa_top_k, contract include/jepa.h:146-150), the per-thread diagnostics capture (jepa_error_reset /
jepa_error_text, include/jepa.h:596-610 and the thread-safety notes at 612-647), and the drop-in
claim itself: the reference's own tools/jepa-bench.cpp, which includes only jepa.h and jepa-args.h,
compiles against this repository's header and links against libjepa.so unchanged."""
import ctypes as C
import os
import shutil
import subprocess
import threading

import numpy as np
import pytest

from jepa_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE_TOOLS = "/root/reference/tools"


@pytest.fixture(scope="module")
def L():
    L = _lib.lib()
    L.jepa_softmax.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    L.jepa_softmax.restype = None
    L.jepa_top_k.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    L.jepa_top_k.restype = C.c_int
    return L


def _softmax(L, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    p = np.zeros_like(x)
    L.jepa_softmax(x.ctypes.data, x.size, p.ctypes.data)
    return p


@pytest.mark.parametrize("n,scale", [(1, 1.0), (7, 1.0), (174, 8.0), (1000, 30.0)])
def test_softmax_against_float64(L, n, scale):
    x = (np.random.default_rng(n).standard_normal(n) * scale).astype(np.float32)
    got = _softmax(L, x)
    e = np.exp(x.astype(np.float64) - x.max())
    want = e / e.sum()
    assert np.abs(got - want).max() <= 2e-7 * max(1.0, want.max()) + 1e-12
    assert abs(got.astype(np.float64).sum() - 1.0) < 1e-5
    assert int(np.argmax(got)) == int(np.argmax(x))


def test_softmax_is_shift_invariant_and_survives_large_logits(L):
    x = np.array([1000.0, 999.0, 998.0, -1000.0], np.float32)
    got = _softmax(L, x)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, _softmax(L, x - 1000.0), rtol=0, atol=0)


def test_softmax_degenerate_calls_are_no_ops(L):
    p = np.full(3, 7.0, np.float32)
    L.jepa_softmax(None, 3, p.ctypes.data)
    L.jepa_softmax(p.ctypes.data, 0, p.ctypes.data)
    assert np.all(p == 7.0)


def _top_k(L, x, k):
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.full(max(k, 1), -1, np.int32)
    n = L.jepa_top_k(x.ctypes.data, x.size, k, idx.ctypes.data)
    return idx[:n]


@pytest.mark.parametrize("n,k", [(10, 3), (174, 5), (1000, 1000), (5, 9)])
def test_top_k_order_with_ties(L, n, k):
    rng = np.random.default_rng(n + k)
    x = rng.integers(-4, 5, n).astype(np.float32)           # many exact ties
    got = _top_k(L, x, k)
    want = np.lexsort((np.arange(n), -x))[: min(k, n)]       # larger first, then the smaller index
    assert got.tolist() == want.tolist()


def test_top_k_nan_ranks_last_and_bad_calls_return_zero(L):
    x = np.array([np.nan, 1.0, np.nan, 3.0], np.float32)
    assert _top_k(L, x, 4).tolist() == [3, 1, 0, 2]
    idx = np.zeros(4, np.int32)
    assert L.jepa_top_k(x.ctypes.data, 4, 0, idx.ctypes.data) == 0
    assert L.jepa_top_k(None, 4, 2, idx.ctypes.data) == 0
    assert L.jepa_top_k(x.ctypes.data, 0, 2, idx.ctypes.data) == 0


def _fail_once(L, tag):
    L.jepa_model_load.restype = C.c_void_p
    L.jepa_model_load.argtypes = [C.c_char_p, C.c_bool]
    assert L.jepa_model_load(f"/nonexistent/{tag}.gguf".encode(), False) is None


def test_error_capture_reset_and_accumulate(L):
    L.jepa_error_reset()
    assert _lib.error_text() == ""
    _fail_once(L, "first")
    _fail_once(L, "second")
    text = _lib.error_text()
    assert "first.gguf" in text and "second.gguf" in text and text.index("first") < text.index("second")
    L.jepa_error_reset()
    assert _lib.error_text() == ""


def test_error_capture_is_bounded(L):
    L.jepa_error_reset()
    for i in range(400):
        _fail_once(L, f"{i:04d}" + "x" * 40)
    text = _lib.error_text()
    assert 4096 < len(text.encode()) <= 8192
    assert "0000" in text                # the earliest lines are kept, later ones dropped
    L.jepa_error_reset()


def test_error_capture_is_per_thread(L):
    """A capture holds only the calling thread's lines (include/jepa.h:630-631)."""
    L.jepa_error_reset()
    seen = {}

    def worker(tag):
        L.jepa_error_reset()
        _fail_once(L, tag)
        seen[tag] = _lib.error_text()

    threads = [threading.Thread(target=worker, args=(f"thread{i}",)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for tag, text in seen.items():
        assert tag in text
        assert all(other not in text for other in seen if other != tag)
    assert _lib.error_text() == ""       # this thread logged nothing


@pytest.mark.skipif(not os.path.isfile(os.path.join(REFERENCE_TOOLS, "jepa-bench.cpp")) or shutil.which("g++") is None,
                    reason="the reference tree (tools/jepa-bench.cpp) is not present")
def test_reference_jepa_bench_links_unchanged(L, tmp_path):
    """tools/jepa-bench.cpp of the reference, compiled as it lies against include/jepa.h of this
    repository and linked against libjepa.so: every symbol it references resolves, and the program
    runs (its usage text needs no model and no GPU)."""
    exe = tmp_path / "jepa-bench"
    lib_dir = os.path.join(ROOT, "jepa.cpp_amd")
    cmd = ["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), os.path.join(REFERENCE_TOOLS, "jepa-bench.cpp"),
           "-L", lib_dir, "-ljepa", f"-Wl,-rpath,{lib_dir}", "-Wl,--no-undefined", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe), "--help"], capture_output=True, text=True, timeout=60)
    assert "usage" in (r.stdout + r.stderr).lower()


@pytest.mark.skipif(not os.path.isfile(os.path.join(REFERENCE_TOOLS, "jepa-bench.cpp")) or shutil.which("g++") is None,
                    reason="the reference tree (tools/jepa-bench.cpp) is not present")
@pytest.mark.parametrize("shape", [(1, 1, 224, 224, 1234), (2, 3, 16, 24, 0), (1, 2, 32, 32, 987654321)])
def test_synthetic_input_equals_reference_make_input(L, tmp_path, shape):
    """jepa_amd.inputs.make_input against the reference's own make_input (tools/jepa-bench.cpp:124-149),
    compiled from the reference file as it lies (its main renamed by the harness) and linked against
    libjepa.so for jepa_preprocess_default_params (NULL model: the ImageNet defaults both use): every
    float bit for bit, including seed 0 (the generator's fixed replacement seed)."""
    B, T, H, W, seed = shape
    src = tmp_path / "make_input_harness.cpp"
    src.write_text(
        "#define main jepa_bench_main\n"
        f'#include "{os.path.join(REFERENCE_TOOLS, "jepa-bench.cpp")}"\n'
        "#undef main\n"
        "int main(int argc, char ** argv) {\n"
        "    const std::vector<float> x = make_input(nullptr, atoi(argv[1]), atoi(argv[2]), atoi(argv[3]), atoi(argv[4]),\n"
        "                                            strtoull(argv[5], nullptr, 10));\n"
        "    return fwrite(x.data(), sizeof(float), x.size(), stdout) == x.size() ? 0 : 1;\n"
        "}\n")
    exe = tmp_path / "make_input_harness"
    lib_dir = os.path.join(ROOT, "jepa.cpp_amd")
    cmd = ["g++", "-std=c++17", "-O1", "-w", "-I", os.path.join(ROOT, "include"), "-I", REFERENCE_TOOLS, str(src),
           "-L", lib_dir, "-ljepa", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe), str(B), str(T), str(H), str(W), str(seed)], capture_output=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    want = np.frombuffer(r.stdout, dtype=np.float32).reshape(B, 3, T, H, W)
    from jepa_amd import inputs
    got = inputs.make_input(B, T, H, W, seed=seed)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


REFERENCE_ROOT = os.path.dirname(REFERENCE_TOOLS)


@pytest.mark.skipif(not os.path.isfile(os.path.join(REFERENCE_TOOLS, "jepa-embed.cpp")) or shutil.which("g++") is None,
                    reason="the reference tree (tools/jepa-embed.cpp) is not present")
@pytest.mark.parametrize("tool", ["jepa-embed", "jepa-classify"])
def test_reference_embed_tools_link_unchanged(L, tmp_path, tool):
    """tools/jepa-embed.cpp and tools/jepa-classify.cpp of the reference, each with tools/video-decode.cpp
    (the reference's own tool recipe, CMakeLists.txt:90-102: include paths src/ and third_party/ for
    npy.h and the stb headers), compiled as they lie against include/jepa.h of this repository and
    linked against libjepa.so with --no-undefined: every entry point they call (preprocessing, image
    loading, pooling, the head, device queries) resolves to this library, and the program runs its
    usage text (no model, no GPU)."""
    exe = tmp_path / tool
    lib_dir = os.path.join(ROOT, "jepa.cpp_amd")
    cmd = ["g++", "-std=c++17", "-O1", "-w", "-I", os.path.join(ROOT, "include"), "-I", REFERENCE_TOOLS,
           "-I", os.path.join(REFERENCE_ROOT, "src"), "-I", os.path.join(REFERENCE_ROOT, "third_party"),
           os.path.join(REFERENCE_TOOLS, f"{tool}.cpp"), os.path.join(REFERENCE_TOOLS, "video-decode.cpp"),
           "-L", lib_dir, "-ljepa", f"-Wl,-rpath,{lib_dir}", "-Wl,--no-undefined", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe), "--help"], capture_output=True, text=True, timeout=60)
    assert "usage" in (r.stdout + r.stderr).lower()
