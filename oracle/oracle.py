"""ctypes wrapper of liboracle.so (test infrastructure only: imported by tests/, smoke() and the
cpu_baseline leg of bench.py, never by the product path)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OR_F32, OR_F16, OR_Q4_0, OR_Q8_0, OR_Q4_K, OR_Q8_K = 0, 1, 2, 8, 12, 15


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, f32p = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.or_fp32_to_fp16.restype = C.c_uint16
        L.or_fp32_to_fp16.argtypes = [C.c_float]
        L.or_fp16_to_fp32.restype = C.c_float
        L.or_fp16_to_fp32.argtypes = [C.c_uint16]
        L.or_row_size.restype = C.c_size_t
        L.or_row_size.argtypes = [C.c_int, i64]
        for fn in ("or_quantize_q8_0_ref", "or_quantize_q4_0_ref", "or_quantize_q4_K",
                   "or_quantize_q8_0_act", "or_quantize_q8_K_act"):
            getattr(L, fn).argtypes = [vp, vp, i64]
            getattr(L, fn).restype = None
        L.or_dequantize.argtypes = [C.c_int, vp, vp, i64]
        L.or_dequantize.restype = None
        L.or_vec_dot.argtypes = [C.c_int, i64, vp, vp]
        L.or_vec_dot.restype = C.c_float
        L.or_mul_mat.argtypes = [C.c_int, vp, i64, i64, vp, i64, vp, vp, C.c_int]
        L.or_mul_mat.restype = C.c_int
        L.or_layer_norm.argtypes = [vp, i64, i64, vp, vp, C.c_float, vp]
        L.or_layer_norm.restype = None
        L.or_gelu_erf.argtypes = [C.c_float]
        L.or_gelu_erf.restype = C.c_float
        L.or_gelu_erf_n.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.or_gelu_erf_n.restype = None
        L.or_rope_tables.argtypes = [vp, vp, i64, vp, vp, C.c_int]
        L.or_rope_tables.restype = None
        L.or_rope_apply.argtypes = [vp, i64, C.c_int, C.c_int, vp, vp]
        L.or_rope_apply.restype = None
        L.or_attention.argtypes = [vp, vp, vp, i64, i64, C.c_int, C.c_int, C.c_float, C.c_int, vp, vp, C.c_int]
        L.or_attention.restype = None
        L.or_block_causal_mask.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, vp]
        L.or_block_causal_mask.restype = None
        L.or_encode_file.argtypes = [C.c_char_p, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, i64,
                                     vp, i64, C.c_int, C.c_int]
        L.or_encode_file.restype = i64
        L.or_head_file.argtypes = [C.c_char_p, vp, i64, vp, vp, i64, C.c_int]
        L.or_head_file.restype = i64
        L.or_predict_file.argtypes = [C.c_char_p, vp, i64, vp, C.c_int, vp, C.c_int, C.c_int, C.c_int, vp, i64, C.c_int]
        L.or_predict_file.restype = i64
        for fn in ("or_fp32_to_fp16_row", "or_fp16_to_fp32_row"):
            getattr(L, fn).argtypes = [vp, vp, i64]
            getattr(L, fn).restype = None
        L.or_make_qkx2_quants.argtypes = [C.c_int, C.c_int, vp, vp, vp, vp, C.c_float, C.c_float, C.c_int]
        L.or_make_qkx2_quants.restype = C.c_float
        L.or_set_first_block.argtypes = [C.c_int]
        L.or_set_first_block.restype = None
        L.or_set_ggml_lanes.argtypes = [C.c_int]
        L.or_set_ggml_lanes.restype = None
        L.or_get_ggml_lanes.argtypes = []
        L.or_get_ggml_lanes.restype = C.c_int
        L.or_set_reverse_block_order.argtypes = [C.c_int]
        L.or_set_reverse_block_order.restype = None
        L.or_set_k_split.argtypes = [C.c_int]
        L.or_set_k_split.restype = None
        L.or_set_attn_f16.argtypes = [C.c_int]
        L.or_set_attn_f16.restype = None
        L.or_set_rounding.argtypes = [C.c_int]
        L.or_set_rounding.restype = None
        L.or_get_rounding.argtypes = []
        L.or_get_rounding.restype = C.c_int
        L.or_set_teacher.argtypes = [C.c_void_p, C.c_int64]
        L.or_set_teacher.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class RopeParams(C.Structure):
    _fields_ = [("grid_t", C.c_int), ("grid_h", C.c_int), ("grid_w", C.c_int), ("head_dim", C.c_int),
                ("theta", C.c_float), ("interpolate", C.c_int), ("train_grid_h", C.c_int),
                ("train_grid_w", C.c_int), ("variant", C.c_int)]


def threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1))


def row_size(t: int, n: int) -> int:
    return int(lib().or_row_size(t, n))


def quantize(fn: str, x: np.ndarray, block_type: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.zeros((rows, row_size(block_type, n)), dtype=np.uint8)
    for r in range(rows):
        getattr(lib(), fn)(_p(x.reshape(rows, n)[r]), _p(out[r]), n)
    return out.reshape(*x.shape[:-1], -1)


def quantize_weight(t: int, x: np.ndarray) -> np.ndarray:
    fn = {OR_Q8_0: "or_quantize_q8_0_ref", OR_Q4_0: "or_quantize_q4_0_ref", OR_Q4_K: "or_quantize_q4_K"}[t]
    return quantize(fn, x, t)


def make_qkx2_quants(x: np.ndarray, w: np.ndarray, nmax: int = 15, rmin: float = -1.0, rdelta: float = 0.1,
                     nstep: int = 20):
    """One asymmetric fit of the values x with weights w: (scale, min, levels) with x ~ scale * L + min."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    L = np.zeros(x.size, np.uint8)
    the_min = C.c_float(0)
    s = lib().or_make_qkx2_quants(x.size, nmax, x.ctypes.data, w.ctypes.data, L.ctypes.data, C.addressof(the_min),
                                  rmin, rdelta, nstep)
    return float(s), -the_min.value, L


def quantize_act(t: int, x: np.ndarray) -> np.ndarray:
    fn = {OR_Q8_0: "or_quantize_q8_0_act", OR_Q8_K: "or_quantize_q8_K_act"}[t]
    return quantize(fn, x, t)


def dequantize(t: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    rows = raw.size // row_size(t, n)
    out = np.zeros((rows, n), dtype=np.float32)
    r2 = raw.reshape(rows, -1)
    for r in range(rows):
        lib().or_dequantize(t, _p(r2[r]), _p(out[r]), n)
    return out


def mul_mat(wtype: int, w_raw: np.ndarray, n_out: int, n_in: int, x: np.ndarray, bias=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
    w_raw = np.ascontiguousarray(w_raw, dtype=np.uint8)
    y = np.zeros((x.shape[0], n_out), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().or_mul_mat(wtype, _p(w_raw), n_out, n_in, _p(x), x.shape[0], None if b is None else _p(b), _p(y), threads())
    assert rc == 0
    return y


def layer_norm(x, w, b, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    d = x.shape[-1]
    lib().or_layer_norm(_p(x), x.size // d, d, None if w is None else _p(np.ascontiguousarray(w, np.float32)),
                        None if b is None else _p(np.ascontiguousarray(b, np.float32)), eps, _p(y))
    return y


def rope_tables(grid, head_dim, variant=0, interpolate=0, train=(0, 0), ids=None, signed=True, theta=10000.0):
    p = RopeParams(grid[0], grid[1], grid[2], head_dim, theta, interpolate, train[0], train[1], variant)
    n = len(ids) if ids is not None else grid[0] * grid[1] * grid[2]
    c = np.zeros((n, head_dim), np.float32)
    s = np.zeros((n, head_dim), np.float32)
    idp = None
    if ids is not None:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        idp = _p(ids)
    lib().or_rope_tables(C.byref(p), idp, n, _p(c), _p(s), 1 if signed else 0)
    return c, s


def rope_apply(x, cos_t, sin_t):
    """x [n_tok, n_head, hd] f32 -> rotated copy"""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    n, h, d = x.shape
    lib().or_rope_apply(_p(x), n, h, d, _p(np.ascontiguousarray(cos_t, np.float32)), _p(np.ascontiguousarray(sin_t, np.float32)))
    return x


def attention(q, k, v, n_head, scale=None, kv_f16=True, mask=None):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    n_q, row = q.shape
    hd = row // n_head
    out = np.zeros_like(q)
    sc = scale if scale is not None else 1.0 / np.sqrt(hd)
    mp = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, np.float32)
        assert mask.shape == (n_q, k.shape[0])
        mp = _p(mask)
    lib().or_attention(_p(q), _p(k), _p(v), n_q, k.shape[0], n_head, hd, sc, 1 if kv_f16 else 0, mp, _p(out), threads())
    return out


def block_causal_mask(gt, gh, gw, n_prefix):
    """[N][N] float32 additive mask (0 visible / -inf), N = n_prefix + gt*gh*gw"""
    n = n_prefix + gt * gh * gw
    out = np.zeros((n, n), np.float32)
    lib().or_block_causal_mask(gt, gh, gw, n_prefix, _p(out))
    return out


def encode_file(path: str, x: np.ndarray, rows_per_item: int, dim: int, n_layers: int = 0, trace: bool = False):
    """Oracle encoder forward. x NCTHW float32. Returns (out [items*rows, dim], trace or None)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, Cc, T, H, W = x.shape
    items = B if T > 1 or rows_per_item != (H // 16) * (W // 16) + 1 else B * T
    return _encode(path, x, rows_per_item, dim, n_layers, trace, items)


def _encode(path, x, rows, dim, n_layers, trace, items):
    B, Cc, T, H, W = x.shape
    out = np.zeros(items * rows * dim, dtype=np.float32)
    tr = None
    if trace:
        tr = np.zeros(items * (n_layers + 1) * rows * dim, dtype=np.float32)
    r = lib().or_encode_file(path.encode(), _p(x), B, Cc, T, H, W, _p(out), out.size,
                             None if tr is None else _p(tr), 0 if tr is None else tr.size, n_layers, threads())
    if r < 0:
        raise RuntimeError("oracle encode failed")
    out = out.reshape(-1, dim)
    if tr is not None:
        tr = tr.reshape(items, n_layers + 1, rows, dim)
    return out, tr


def head(path: str, x: np.ndarray, n_classes: int):
    """Oracle attentive-pool head on encoder rows x [N, D]. Returns (pooled [D], logits [n_classes])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    pooled = np.zeros(x.shape[1], dtype=np.float32)
    logits = np.zeros(max(n_classes, 1), dtype=np.float32)
    r = lib().or_head_file(path.encode(), _p(x), x.shape[0], _p(pooled), _p(logits), logits.size, threads())
    if r < 0:
        raise RuntimeError("oracle head failed")
    return pooled, logits[:r]


def predict(path: str, enc: np.ndarray, ctx_ids, tgt_ids, out_dim: int, mask_index: int = 1, modality: int = 1):
    """Oracle masked predictor: enc [n_tok, enc_dim], int id lists -> [len(tgt_ids), out_dim]."""
    enc = np.ascontiguousarray(enc, dtype=np.float32)
    ci = np.ascontiguousarray(ctx_ids, dtype=np.int32)
    ti = np.ascontiguousarray(tgt_ids, dtype=np.int32)
    out = np.zeros((len(ti), out_dim), dtype=np.float32)
    r = lib().or_predict_file(path.encode(), _p(enc), enc.shape[0], _p(ci) if len(ci) else None, len(ci), _p(ti), len(ti),
                              mask_index, modality, _p(out), out.size, threads())
    if r < 0:
        raise RuntimeError("oracle predict failed")
    return out


def encode(path: str, x: np.ndarray, n_items: int, rows: int, dim: int, n_layers: int = 0, trace: bool = False):
    """Oracle forward with an explicit item count (video: n_batch; image: n_batch * n_frames)."""
    return _encode(path, np.ascontiguousarray(x, dtype=np.float32), rows, dim, n_layers, trace, n_items)


def fp32_to_fp16(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of x rounded to f16 by the oracle's software conversion"""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(x.size, dtype=np.uint16)
    lib().or_fp32_to_fp16_row(_p(x), _p(out), x.size)
    return out


def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.zeros(h.size, dtype=np.float32)
    lib().or_fp16_to_fp32_row(_p(h), _p(out), h.size)
    return out


def vec_dot(wtype: int, n: int, wrow: np.ndarray, arow: np.ndarray) -> float:
    """one weight row (wtype blocks) . one activation row (its vec-dot type blocks)"""
    w = np.ascontiguousarray(wrow, dtype=np.uint8)
    a = np.ascontiguousarray(arow, dtype=np.uint8)
    return float(lib().or_vec_dot(wtype, n, _p(w), _p(a)))


def gelu_erf(x: float) -> float:
    return float(lib().or_gelu_erf(x))


def gelu_erf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_gelu_erf_n(_p(x), _p(y), x.size)
    return y


def set_ggml_lanes(on: bool) -> None:
    """Sum the quantized dots in ggml's x86 lane order (AVX2 vec_dot / llamafile tiles: eight float lanes
    of four consecutive products, q4_K mins in four lanes, horizontal sums at the end) instead of one
    chain per output."""
    lib().or_set_ggml_lanes(1 if on else 0)


def get_ggml_lanes() -> bool:
    return bool(lib().or_get_ggml_lanes())


def set_reverse_block_order(on: bool) -> None:
    lib().or_set_reverse_block_order(1 if on else 0)


def set_k_split(s: int) -> None:
    """q8_0 / q4_0 dots: sum the blocks in s consecutive K ranges, one chain each, then add the chains"""
    lib().or_set_k_split(int(s))


def set_attn_f16(on: bool) -> None:
    """Round q and the softmax weights to f16 in attentions with f16 K/V (an f16 matrix-core kernel)."""
    lib().or_set_attn_f16(1 if on else 0)


# rounding switches (oracle.c): the GPU kernels' roundings, one bit each
ROUND_Q16, ROUND_P16, ROUND_EXP2, ROUND_GELU = 1, 2, 4, 8
ROUND_GPU = ROUND_Q16 | ROUND_P16 | ROUND_EXP2 | ROUND_GELU


def set_rounding(bits: int) -> None:
    """Take the GPU's rounding for the sources in `bits` (0: the reference's CPU arithmetic)."""
    lib().or_set_rounding(int(bits))


def get_rounding() -> int:
    return int(lib().or_get_rounding())


def encode_teacher(path: str, x: np.ndarray, n_items: int, rows: int, dim: int, teacher: np.ndarray, first_block: int = 0):
    """Oracle forward in which block l starts from teacher[:, l] (teacher [n_items][L + 1][rows][dim],
    e.g. the GPU's residual-stream trace): returns the oracle's trace, whose entry l + 1 is the
    oracle's block l applied to the teacher's entry l (entry 0 is the oracle's own patch embedding).
    Blocks before first_block are not run (their entries are the teacher's own)."""
    t = np.ascontiguousarray(teacher, dtype=np.float32)
    n_layers = t.shape[1] - 1
    lib().or_set_teacher(_p(t), t.size)
    lib().or_set_first_block(int(first_block))
    try:
        return _encode(path, np.ascontiguousarray(x, dtype=np.float32), rows, dim, n_layers, True, n_items)
    finally:
        lib().or_set_teacher(None, 0)
        lib().or_set_first_block(0)
