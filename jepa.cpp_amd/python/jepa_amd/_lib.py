"""ctypes binding of libjepa.so (the role of the reference's python/src/jepa_cpp/_lib.py + _api.py).

Loads the in-tree library built by `make -C jepa.cpp_amd`; there is no fallback: if the library is
missing, every call fails loudly."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(PKG_DIR, "..", ".."))       # jepa.cpp_amd/
LIB_PATH = os.path.join(ROOT, "libjepa.so")

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q8_K = 0, 1, 2, 8, 12, 15


class ContextParams(C.Structure):
    _fields_ = [("n_threads", C.c_int), ("use_flash_attn", C.c_bool), ("verbose", C.c_bool), ("flash_kv", C.c_int)]


class Input(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("n_batch", C.c_int), ("n_chans", C.c_int), ("n_frames", C.c_int),
                ("height", C.c_int), ("width", C.c_int)]


class Output(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("n_tokens", C.c_int64), ("dim", C.c_int64)]


class ModelParams(C.Structure):
    _fields_ = [("verbose", C.c_bool), ("device", C.c_int)]


class PreprocessParams(C.Structure):
    _fields_ = [("mean", C.c_float * 3), ("std", C.c_float * 3), ("resize_short", C.c_int), ("crop", C.c_int),
                ("resample", C.c_int), ("resize_mode", C.c_int), ("rescale", C.c_float), ("fused_norm", C.c_bool)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {ROOT}` (or __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    vp, i64, cp = C.c_void_p, C.c_int64, C.c_char_p
    sig = {
        "jepa_version": (cp, []),
        "jepa_error_reset": (None, []),
        "jepa_error_text": (cp, []),
        "jepa_context_default_params": (ContextParams, []),
        "jepa_model_default_params": (ModelParams, []),
        "jepa_model_load": (vp, [cp, C.c_bool]),
        "jepa_model_load_ex": (vp, [cp, C.POINTER(ModelParams)]),
        "jepa_model_free": (None, [vp]),
        "jepa_context_new": (vp, [vp, ContextParams]),
        "jepa_context_free": (None, [vp]),
        "jepa_context_last_compute_ms": (C.c_double, [vp]),
        "jepa_context_set_max_batch": (None, [vp, C.c_int]),
        "jepa_context_last_batch": (C.c_int, [vp]),
        "jepa_encode": (C.c_int, [vp, C.POINTER(Input), C.POINTER(Output)]),
        "jepa_free": (None, [vp]),
        "jepa_token_grid": (i64, [vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_model_embed_dim": (C.c_int, [vp]),
        "jepa_model_n_layer": (C.c_int, [vp]),
        "jepa_model_n_head": (C.c_int, [vp]),
        "jepa_model_family": (cp, [vp]),
        "jepa_model_name": (cp, [vp]),
        "jepa_model_file_type": (C.c_int, [vp]),
        "jepa_model_file_type_name": (cp, [vp]),
        "jepa_model_n_bytes": (C.c_size_t, [vp]),
        "jepa_model_has_cls": (C.c_bool, [vp]),
        "jepa_model_n_prefix_tokens": (C.c_int, [vp]),
        "jepa_model_device": (C.c_int, [vp]),
        "jepa_model_device_name": (cp, [vp]),
        "jepa_device_count": (C.c_int, []),
        "jepa_device_name": (cp, [C.c_int]),
        "jepa_device_description": (cp, [C.c_int]),
        "jepa_preprocess_default_params": (PreprocessParams, [vp]),
        "jepa_preprocess_frames_rgb_ex": (C.POINTER(C.c_float), [C.POINTER(PreprocessParams), C.POINTER(C.c_void_p), C.c_int, C.c_int,
                                                                 C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_preprocess_image_rgb_ex": (C.POINTER(C.c_float), [C.POINTER(PreprocessParams), vp, C.c_int, C.c_int,
                                                                C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_preprocess_image_file": (C.POINTER(C.c_float), [vp, cp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_load_image_rgb": (C.POINTER(C.c_uint8), [cp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_resize_antialias_u8": (None, [vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, C.c_int, C.c_int]),
        "jepa_amd_preprocess_frames_device": (C.c_int, [C.c_int, C.POINTER(PreprocessParams), vp, C.c_int, C.c_int, C.c_int, vp, i64,
                                                        C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "jepa_amd_preprocess_frames_device_noalloc": (C.c_int, [C.c_int, C.POINTER(PreprocessParams), vp, C.c_int, C.c_int, C.c_int, vp,
                                                                i64, C.POINTER(C.c_int), C.POINTER(C.c_int), vp]),
        "jepa_pool_mean": (C.c_int, [vp, C.POINTER(Output), C.POINTER(Output)]),
        "jepa_pool_cls": (C.c_int, [vp, C.POINTER(Output), C.POINTER(Output)]),
        "jepa_softmax": (None, [vp, C.c_int, vp]),
        "jepa_top_k": (C.c_int, [vp, C.c_int, C.c_int, vp]),
        "jepa_head": (C.c_int, [vp, C.POINTER(Output), C.POINTER(Output)]),
        "jepa_head_ex": (C.c_int, [vp, C.POINTER(Output), C.POINTER(Output), C.POINTER(Output)]),
        "jepa_model_has_head": (C.c_bool, [vp]),
        "jepa_model_n_classes": (C.c_int, [vp]),
        "jepa_model_label": (cp, [vp, C.c_int]),
        "jepa_amd_head_device": (C.c_int, [vp, vp, i64, vp, vp]),
        "jepa_model_has_predictor": (C.c_bool, [vp]),
        "jepa_amd_quantize_file": (C.c_int, [cp, cp, cp, C.POINTER(cp), C.c_int, C.c_bool, C.c_int, C.c_bool]),
        "jepa_amd_quantize_rows": (C.c_int, [C.c_int, C.c_int, vp, i64, vp]),
        "jepa_predict": (C.c_int, [vp, C.POINTER(Output), vp, C.c_int, vp, C.c_int, C.POINTER(Output)]),
        "jepa_predict_ex": (C.c_int, [vp, C.POINTER(Output), vp, C.c_int, vp, C.c_int, C.c_int, C.POINTER(Output)]),
        "jepa_predict_mod": (C.c_int, [vp, C.POINTER(Output), vp, C.c_int, vp, C.c_int, C.c_int, C.c_int, C.POINTER(Output)]),
        # jepa_amd.h
        "jepa_amd_encode_device": (i64, [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, i64]),
        "jepa_amd_encode_trace": (i64, [vp, C.POINTER(Input), vp, i64, vp, i64]),
        "jepa_amd_context_set_kernel_timing": (None, [vp, C.c_bool]),
        "jepa_amd_context_kernel_stats": (C.c_int, [vp, cp, C.POINTER(i64), C.POINTER(C.c_double)]),
        "jepa_amd_context_reset_kernel_stats": (None, [vp]),
        "jepa_amd_context_set_graph": (None, [vp, C.c_bool]),
        "jepa_amd_context_stream": (vp, [vp]),
        "jepa_amd_dequantize": (C.c_int, [C.c_int, C.c_int, vp, i64, i64, vp]),
        "jepa_amd_rownorm": (C.c_int, [C.c_int, vp, i64, i64, vp, vp, C.c_float, C.c_int, C.c_int, vp]),
        "jepa_amd_matmul": (C.c_int, [C.c_int, C.c_int, vp, i64, i64, vp, vp, i64, vp, C.c_int, C.POINTER(C.c_double)]),
        "jepa_amd_matmul_gelu": (C.c_int, [C.c_int, C.c_int, vp, i64, i64, vp, vp, i64, C.c_int, vp, C.c_int, C.POINTER(C.c_double)]),
        "jepa_amd_attention": (C.c_int, [C.c_int, vp, i64, i64, C.c_int, C.c_int, vp, vp, C.c_int, i64, C.c_int, vp]),
        "jepa_amd_mfma_probe": (C.c_int, [C.c_int, vp, vp, vp]),
        "jepa_amd_copy": (C.c_int, [C.c_int, vp, vp, i64, C.c_int, C.POINTER(C.c_double)]),
        "jepa_amd_gemm_step_probe": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]),
        "jepa_amd_gemm_tile": (C.c_int, [C.c_int]),
        "jepa_amd_gemm_split": (C.c_int, [C.c_int]),
        "jepa_amd_gemm_split_of": (C.c_int, [C.c_int, i64, i64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def error_text() -> str:
    return (lib().jepa_error_text() or b"").decode(errors="replace")


def check(rc, what: str):
    if rc is None or (isinstance(rc, int) and rc < 0):
        raise RuntimeError(f"{what} failed: {error_text().strip()}")
    return rc


def fptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Model:
    def __init__(self, path: str, device: int = 0, verbose: bool = False):
        L = lib()
        L.jepa_error_reset()
        p = ModelParams(verbose, device)
        self.ptr = L.jepa_model_load_ex(path.encode(), C.byref(p))
        if not self.ptr:
            raise RuntimeError(f"jepa_model_load_ex({path}) failed: {error_text().strip()}")
        self.dim = L.jepa_model_embed_dim(self.ptr)
        self.n_layer = L.jepa_model_n_layer(self.ptr)
        self.has_head = bool(L.jepa_model_has_head(self.ptr))
        self.has_predictor = bool(L.jepa_model_has_predictor(self.ptr))
        self.n_classes = int(L.jepa_model_n_classes(self.ptr))

    def label(self, i: int):
        r = lib().jepa_model_label(self.ptr, i)
        return None if r is None else r.decode()

    def _pool(self, fn, rows: np.ndarray) -> np.ndarray:
        L = lib()
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        enc = Output(C.cast(rows.ctypes.data, C.POINTER(C.c_float)), rows.shape[0], rows.shape[1])
        out = Output()
        L.jepa_error_reset()
        check(fn(self.ptr, C.byref(enc), C.byref(out)), fn.__name__)
        y = np.ctypeslib.as_array(out.data, shape=(out.dim,)).copy()
        L.jepa_free(C.cast(out.data, C.c_void_p))
        return y

    def pool_mean(self, rows: np.ndarray) -> np.ndarray:
        """jepa_pool_mean over one item's encoder rows [N, dim] (prefix rows left out)."""
        return self._pool(lib().jepa_pool_mean, rows)

    def pool_cls(self, rows: np.ndarray) -> np.ndarray:
        """jepa_pool_cls: row 0 of one item's encoder rows (models with a CLS token)."""
        return self._pool(lib().jepa_pool_cls, rows)

    def token_grid(self, n_frames, h, w) -> int:
        return int(lib().jepa_token_grid(self.ptr, n_frames, h, w, None, None, None))

    def close(self):
        if self.ptr:
            lib().jepa_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    def __init__(self, model: Model):
        L = lib()
        self.model = model
        self.ptr = L.jepa_context_new(model.ptr, L.jepa_context_default_params())
        if not self.ptr:
            raise RuntimeError(f"jepa_context_new failed: {error_text().strip()}")

    def encode(self, x: np.ndarray) -> np.ndarray:
        """x: NCTHW float32 -> [rows, dim] float32 (jepa_encode)."""
        L = lib()
        x = np.ascontiguousarray(x, dtype=np.float32)
        B, Cc, T, H, W = x.shape
        inp = Input(fptr(x), B, Cc, T, H, W)
        out = Output()
        L.jepa_error_reset()
        check(L.jepa_encode(self.ptr, C.byref(inp), C.byref(out)), "jepa_encode")
        y = np.ctypeslib.as_array(out.data, shape=(out.n_tokens, out.dim)).copy()
        L.jepa_free(C.cast(out.data, C.c_void_p))
        return y

    def head(self, rows: np.ndarray, pooled: bool = True, logits: bool = True):
        """Attentive-pool head on encoder rows [N, dim] (jepa_head_ex) -> (pooled [dim] | None, logits | None)."""
        L = lib()
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        enc = Output(C.cast(rows.ctypes.data, C.POINTER(C.c_float)), rows.shape[0], rows.shape[1])
        po, lo = Output(), Output()
        L.jepa_error_reset()
        check(L.jepa_head_ex(self.ptr, C.byref(enc), C.byref(po) if pooled else None, C.byref(lo) if logits else None), "jepa_head_ex")
        res = []
        for want, o in ((pooled, po), (logits, lo)):
            if not want:
                res.append(None)
                continue
            res.append(np.ctypeslib.as_array(o.data, shape=(o.dim,)).copy())
            L.jepa_free(C.cast(o.data, C.c_void_p))
        return tuple(res)

    def predict(self, enc: np.ndarray, ctx_ids, tgt_ids, mask_index: int = 1, modality: int = 1) -> np.ndarray:
        """Masked predictor (jepa_predict_mod): encoder rows [N, dim], context / target token ids."""
        L = lib()
        enc = np.ascontiguousarray(enc, dtype=np.float32)
        e = Output(C.cast(enc.ctypes.data, C.POINTER(C.c_float)), enc.shape[0], enc.shape[1])
        ci = None if ctx_ids is None else np.ascontiguousarray(ctx_ids, dtype=np.int32)
        ti = None if tgt_ids is None else np.ascontiguousarray(tgt_ids, dtype=np.int32)
        out = Output()
        L.jepa_error_reset()
        check(L.jepa_predict_mod(self.ptr, C.byref(e), None if ci is None else ci.ctypes.data, 0 if ci is None else len(ci),
                                 None if ti is None else ti.ctypes.data, 0 if ti is None else len(ti), mask_index, modality,
                                 C.byref(out)), "jepa_predict_mod")
        y = np.ctypeslib.as_array(out.data, shape=(out.n_tokens, out.dim)).copy()
        L.jepa_free(C.cast(out.data, C.c_void_p))
        return y

    def head_device(self, x_ptr: int, n_tokens: int, pooled_ptr: int, logits_ptr: int) -> int:
        return check(lib().jepa_amd_head_device(self.ptr, x_ptr, n_tokens, pooled_ptr, logits_ptr), "jepa_amd_head_device")

    def encode_trace(self, x: np.ndarray, n_items: int, rows: int):
        L = lib()
        x = np.ascontiguousarray(x, dtype=np.float32)
        B, Cc, T, H, W = x.shape
        D, nl = self.model.dim, self.model.n_layer
        out = np.zeros((n_items * rows, D), np.float32)
        tr = np.zeros((n_items, nl + 1, rows, D), np.float32)
        inp = Input(fptr(x), B, Cc, T, H, W)
        L.jepa_error_reset()
        check(L.jepa_amd_encode_trace(self.ptr, C.byref(inp), out.ctypes.data, out.size, tr.ctypes.data, tr.size), "jepa_amd_encode_trace")
        return out, tr

    def encode_device(self, in_ptr: int, shape, out_ptr: int, out_cap: int) -> int:
        B, Cc, T, H, W = shape
        return check(lib().jepa_amd_encode_device(self.ptr, in_ptr, B, Cc, T, H, W, out_ptr, out_cap), "jepa_amd_encode_device")

    @property
    def last_compute_ms(self) -> float:
        return float(lib().jepa_context_last_compute_ms(self.ptr))

    def set_kernel_timing(self, on: bool):
        lib().jepa_amd_context_set_kernel_timing(self.ptr, on)

    def kernel_stats(self, cls: str):
        n = C.c_int64(0)
        ms = C.c_double(0)
        lib().jepa_amd_context_kernel_stats(self.ptr, cls.encode(), C.byref(n), C.byref(ms))
        return int(n.value), float(ms.value)

    def reset_kernel_stats(self):
        lib().jepa_amd_context_reset_kernel_stats(self.ptr)

    def set_graph(self, on: bool):
        lib().jepa_amd_context_set_graph(self.ptr, on)

    def close(self):
        if self.ptr:
            lib().jepa_context_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------------------------------------
# preprocessing helpers (host functions of include/jepa.h; numpy in, numpy out)
# ------------------------------------------------------------------------------------------------
def resize_u8(img: np.ndarray, out_h: int, out_w: int, resample: int = 0) -> np.ndarray:
    """jepa_resize_antialias_u8 on an HWC uint8 array"""
    img = np.ascontiguousarray(img, dtype=np.uint8)
    h, w, c = img.shape
    out = np.zeros((out_h, out_w, c), np.uint8)
    lib().jepa_resize_antialias_u8(img.ctypes.data, h, w, c, out.ctypes.data, out_h, out_w, resample)
    return out


def preprocess_frames(params: PreprocessParams, frames) -> np.ndarray:
    """jepa_preprocess_frames_rgb_ex on a list of equal HWC uint8 frames -> [3][T][crop][crop] float32"""
    frames = [np.ascontiguousarray(f, dtype=np.uint8) for f in frames]
    h, w, _ = frames[0].shape
    ptrs = (C.c_void_p * len(frames))(*[f.ctypes.data for f in frames])
    oh, ow = C.c_int(0), C.c_int(0)
    L = lib()
    r = L.jepa_preprocess_frames_rgb_ex(C.byref(params), ptrs, len(frames), h, w, C.byref(oh), C.byref(ow))
    if not r:
        raise RuntimeError(f"jepa_preprocess_frames_rgb_ex failed: {error_text().strip()}")
    n = 3 * len(frames) * oh.value * ow.value
    out = np.ctypeslib.as_array(r, shape=(n,)).copy().reshape(3, len(frames), oh.value, ow.value)
    L.jepa_free(C.cast(r, C.c_void_p))
    return out


def load_image(path: str) -> np.ndarray:
    """jepa_load_image_rgb -> HWC uint8"""
    h, w = C.c_int(0), C.c_int(0)
    L = lib()
    r = L.jepa_load_image_rgb(path.encode(), C.byref(h), C.byref(w))
    if not r:
        raise RuntimeError(f"jepa_load_image_rgb({path}) failed: {error_text().strip()}")
    out = np.ctypeslib.as_array(r, shape=(h.value * w.value * 3,)).copy().reshape(h.value, w.value, 3)
    L.jepa_free(C.cast(r, C.c_void_p))
    return out


def quantize_file(in_path: str, out_path: str, qtype: str, keep=(), allow_requant: bool = False, device: int = 0,
                  verbose: bool = False) -> None:
    """jepa_amd_quantize_file: re-type the weights of a jepa GGUF (the reference's jepa-quantize)."""
    L = lib()
    arr = (C.c_char_p * max(len(keep), 1))(*[k.encode() for k in keep])
    L.jepa_error_reset()
    check(L.jepa_amd_quantize_file(in_path.encode(), out_path.encode(), qtype.encode(), arr, len(keep), allow_requant, device,
                                   verbose), "jepa_amd_quantize_file")
