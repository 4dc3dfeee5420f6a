"""GGUF v3 writer/reader and ggml block quantizers (numpy) for jepa GGUF files.

This is the host-side tooling that produces the files the library loads: the role
tools/jepa-quantize.cpp plays in the reference (type table tools/jepa-quantize.cpp:47-58, the
"only 2-D attention/FFN matrices are re-typed" rule :91-129, docs/gguf-schema.md "Quantization
rules"). Block layouts are ggml's (ggml-common.h):

  q8_0  {f16 d; int8 qs[32]}                      34 B / 32 values   x = d*q
  q4_0  {f16 d; u8 qs[16]}                        18 B / 32 values   x = d*(q-8), low nibbles = 0..15
  q4_K  {f16 d, dmin; u8 scales[12]; u8 qs[128]}  144 B / 256 values x = d*sc_j*q - dmin*m_j

q8_0, q4_0 and q4_K use ggml's reference quantizers (quantize_row_q8_0_ref / q4_0_ref / q4_K_ref with
its make_qkx2_quants search), restated in numpy.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

# ggml_type ids stored in tensor infos
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q8_K = 0, 1, 2, 8, 12, 15
TYPE_NAMES = {GGML_F32: "f32", GGML_F16: "f16", GGML_Q4_0: "q4_0", GGML_Q8_0: "q8_0", GGML_Q4_K: "q4_K"}
GGML_BF16 = 30
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144),
         GGML_Q8_K: (256, 292), GGML_BF16: (1, 2)}
# general.file_type values (GGML_FTYPE_*), reference src/jepa-gguf.cpp:62-93
FTYPE = {"f32": 0, "f16": 1, "q4_0": 2, "q8_0": 7, "q4_k": 12}

# GGUF metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR_FMT = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f",
               _BOOL: "<?", _U64: "<Q", _I64: "<q", _F64: "<d"}
ALIGN = 32

F32 = np.float32


def row_bytes(gtype: int, n: int) -> int:
    blk, size = BLOCK[gtype]
    if n % blk:
        raise ValueError(f"row of {n} is not a whole number of {TYPE_NAMES.get(gtype, gtype)} blocks")
    return n // blk * size


def _round_half_away(v: np.ndarray) -> np.ndarray:
    """C roundf on float32 values, exactly (no double rounding)."""
    t = np.trunc(v)
    frac = v - t                       # exact for |v| < 2^23
    return t + np.where(np.abs(frac) >= F32(0.5), np.sign(v), F32(0)).astype(F32)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """quantize_row_q8_0_ref over the last axis. Returns uint8 bytes [..., n/32*34]."""
    x = np.ascontiguousarray(x, dtype=F32)
    lead = x.shape[:-1]
    b = x.reshape(-1, 32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / F32(127)).astype(F32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, F32(1) / np.where(d != 0, d, F32(1)), F32(0)).astype(F32)
    q = _round_half_away((b * idv[:, None]).astype(F32)).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(*lead, -1)


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """quantize_row_q4_0_ref over the last axis."""
    x = np.ascontiguousarray(x, dtype=F32)
    lead = x.shape[:-1]
    b = x.reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)                       # first index of the largest |x|
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / F32(-8)).astype(F32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, F32(1) / np.where(d != 0, d, F32(1)), F32(0)).astype(F32)
    v = (b * idv[:, None]).astype(F32) + F32(8.5)
    q = np.minimum(np.trunc(v).astype(np.int32), 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(*lead, -1)


def _make_qkx2(x, w, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20):
    """ggml's make_qkx2_quants on rows of 32 (x, w: float32 [rows, 32]), vectorized over rows with the
    sums taken sequentially in element order (float32 throughout). Returns (scale, the_min, L)."""
    n = x.shape[1]
    mn, mx = x[:, 0].copy(), x[:, 0].copy()
    sum_w = w[:, 0].copy()
    sum_x = (sum_w * x[:, 0]).astype(F32)
    for i in range(1, n):
        mn = np.where(x[:, i] < mn, x[:, i], mn)
        mx = np.where(x[:, i] > mx, x[:, i], mx)
        sum_w = (sum_w + w[:, i]).astype(F32)
        sum_x = (sum_x + (w[:, i] * x[:, i]).astype(F32)).astype(F32)
    mn = np.where(mn > 0, F32(0), mn).astype(F32)
    flat = mx == mn
    # (ggml updates `min` inside the search, and later candidates are formed against the updated value)
    rng = np.where(flat, F32(1), (mx - mn).astype(F32)).astype(F32)
    xm = (x - mn[:, None]).astype(F32)

    def err(sc, m, L):
        e = np.zeros(x.shape[0], F32)
        for i in range(n):
            diff = (((sc * L[:, i]).astype(F32) + m).astype(F32) - x[:, i]).astype(F32)
            e = (e + (w[:, i] * (diff * diff).astype(F32)).astype(F32)).astype(F32)
        return e

    iscale = (F32(nmax) / rng).astype(F32)
    scale = (F32(1) / iscale).astype(F32)
    L = np.clip(np.rint((iscale[:, None] * xm).astype(F32)), 0, nmax).astype(F32)
    best = err(scale, mn, L)
    for step in range(nstep + 1):
        rng = np.where(flat, F32(1), (mx - mn).astype(F32)).astype(F32)
        xm = (x - mn[:, None]).astype(F32)
        isc = (((F32(rmin) + (F32(rdelta) * F32(step)).astype(F32)).astype(F32) + F32(nmax)).astype(F32) / rng).astype(F32)
        La = np.clip(np.rint((isc[:, None] * xm).astype(F32)), 0, nmax).astype(F32)
        sum_l = np.zeros(x.shape[0], F32); sum_l2 = np.zeros(x.shape[0], F32); sum_xl = np.zeros(x.shape[0], F32)
        for i in range(n):
            wl = (w[:, i] * La[:, i]).astype(F32)
            sum_l = (sum_l + wl).astype(F32)
            sum_l2 = (sum_l2 + (wl * La[:, i]).astype(F32)).astype(F32)
            sum_xl = (sum_xl + (wl * x[:, i]).astype(F32)).astype(F32)
        D = ((sum_w * sum_l2).astype(F32) - (sum_l * sum_l).astype(F32)).astype(F32)
        ok = D > 0
        Ds = np.where(ok, D, F32(1)).astype(F32)
        ts = ((((sum_w * sum_xl).astype(F32) - (sum_x * sum_l).astype(F32)).astype(F32)) / Ds).astype(F32)
        tm = ((((sum_l2 * sum_x).astype(F32) - (sum_l * sum_xl).astype(F32)).astype(F32)) / Ds).astype(F32)
        pos = tm > 0
        with np.errstate(divide="ignore", invalid="ignore"):
            ts = np.where(pos, (sum_xl / np.where(pos, sum_l2, F32(1))).astype(F32), ts).astype(F32)
        tm = np.where(pos, F32(0), tm).astype(F32)
        cur = err(ts, tm, La)
        upd = ok & (cur < best)
        L = np.where(upd[:, None], La, L)
        best = np.where(upd, cur, best)
        scale = np.where(upd, ts, scale).astype(F32)
        mn = np.where(upd, tm, mn).astype(F32)
    scale = np.where(flat, F32(0), scale).astype(F32)
    L = np.where(flat[:, None], F32(0), L)
    return scale, (-mn).astype(F32), L.astype(np.uint8)


def quantize_q4_K(x: np.ndarray) -> np.ndarray:
    """ggml's quantize_row_q4_K_ref over the last axis (no importance matrix): per 32-value sub-block a
    weighted make_qkx2_quants fit (weights sqrt(mean x^2) + |x|), 6-bit scales and mins against their
    maxima, the values re-fitted to the quantized scale / min."""
    x = np.ascontiguousarray(x, dtype=F32)
    lead = x.shape[:-1]
    sb = x.reshape(-1, 8, 32)
    nb = sb.shape[0]
    flat = sb.reshape(-1, 32)
    sum_x2 = np.zeros(flat.shape[0], F32)
    for i in range(32):
        sum_x2 = (sum_x2 + (flat[:, i] * flat[:, i]).astype(F32)).astype(F32)
    av_x = np.sqrt((sum_x2 / F32(32)).astype(F32)).astype(F32)
    w = (av_x[:, None] + np.abs(flat)).astype(F32)
    sc, mi, L = _make_qkx2(flat, w)
    scales, mins, L = sc.reshape(nb, 8), mi.reshape(nb, 8), L.reshape(nb, 8, 32)
    max_scale = np.maximum(scales.max(axis=1), F32(0)).astype(F32)
    max_min = np.maximum(mins.max(axis=1), F32(0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv_s = np.where(max_scale > 0, F32(63) / np.where(max_scale > 0, max_scale, F32(1)), F32(0)).astype(F32)
        inv_m = np.where(max_min > 0, F32(63) / np.where(max_min > 0, max_min, F32(1)), F32(0)).astype(F32)
    # uint8_t ls = nearest_int(...); ls = MIN(63, ls): the int is truncated to a byte before the clamp
    ls = np.minimum(np.rint((inv_s[:, None] * scales).astype(F32)).astype(np.int64) & 0xFF, 63).astype(np.uint8)
    lm = np.minimum(np.rint((inv_m[:, None] * mins).astype(F32)).astype(np.int64) & 0xFF, 63).astype(np.uint8)
    d16 = (max_scale / F32(63)).astype(F32).astype(np.float16)
    dm16 = (max_min / F32(63)).astype(F32).astype(np.float16)
    dd = (d16.astype(F32)[:, None] * ls.astype(F32)).astype(F32)
    dm = (dm16.astype(F32)[:, None] * lm.astype(F32)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        qv = np.rint(((sb + dm[:, :, None]).astype(F32) / np.where(dd != 0, dd, F32(1))[:, :, None]).astype(F32))
    q = np.where(dd[:, :, None] != 0, np.clip(qv, 0, 15), L).astype(np.uint8).reshape(-1, 256)
    scales12 = np.zeros((nb, 12), dtype=np.uint8)
    for j in range(8):
        if j < 4:
            scales12[:, j] = ls[:, j]
            scales12[:, j + 4] = lm[:, j]
        else:
            scales12[:, j + 4] = (ls[:, j] & 0xF) | ((lm[:, j] & 0xF) << 4)
            scales12[:, j - 4] |= (ls[:, j] >> 4) << 6
            scales12[:, j] |= (lm[:, j] >> 4) << 6
    qs = np.empty((nb, 128), dtype=np.uint8)
    for c in range(4):   # 64-value chunks: low nibbles = first 32, high nibbles = next 32
        qs[:, 32 * c:32 * c + 32] = q[:, 64 * c:64 * c + 32] | (q[:, 64 * c + 32:64 * c + 64] << 4)
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dm16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = scales12
    out[:, 16:] = qs
    return out.reshape(*lead, -1)


def dequantize(gtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    """Dequantize rows of `n` values (raw: uint8 [..., row_bytes])."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    lead = raw.shape[:-1]
    if gtype == GGML_F32:
        return raw.view(F32).reshape(*lead, n)
    if gtype == GGML_F16:
        return raw.view(np.float16).astype(F32).reshape(*lead, n)
    if gtype == GGML_Q8_0:
        b = raw.reshape(-1, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(F32)
        q = b[:, 2:].view(np.int8).astype(F32)
        return (q * d).astype(F32).reshape(*lead, n)
    if gtype == GGML_Q4_0:
        b = raw.reshape(-1, 18)
        d = b[:, 0:2].copy().view(np.float16).astype(F32)
        lo = (b[:, 2:] & 0xF).astype(F32) - 8
        hi = (b[:, 2:] >> 4).astype(F32) - 8
        return (np.concatenate([lo, hi], axis=1) * d).astype(F32).reshape(*lead, n)
    if gtype == GGML_Q4_K:
        b = raw.reshape(-1, 144)
        d = b[:, 0:2].copy().view(np.float16).astype(F32)[:, 0]
        dmin = b[:, 2:4].copy().view(np.float16).astype(F32)[:, 0]
        sc, m = q4k_scales_mins(b[:, 4:16])
        qs = b[:, 16:]
        out = np.empty((b.shape[0], 256), dtype=F32)
        for c in range(4):
            lo = (qs[:, 32 * c:32 * c + 32] & 0xF).astype(F32)
            hi = (qs[:, 32 * c:32 * c + 32] >> 4).astype(F32)
            d1 = (d * sc[:, 2 * c]).astype(F32); m1 = (dmin * m[:, 2 * c]).astype(F32)
            d2 = (d * sc[:, 2 * c + 1]).astype(F32); m2 = (dmin * m[:, 2 * c + 1]).astype(F32)
            out[:, 64 * c:64 * c + 32] = (d1[:, None] * lo).astype(F32) - m1[:, None]
            out[:, 64 * c + 32:64 * c + 64] = (d2[:, None] * hi).astype(F32) - m2[:, None]
        return out.reshape(*lead, n)
    raise ValueError(f"cannot dequantize type {gtype}")


def q4k_scales_mins(s12: np.ndarray):
    """The 8 six-bit scales and mins of q4_K blocks (ggml get_scale_min_k4)."""
    s12 = s12.astype(np.uint8)
    sc = np.empty((s12.shape[0], 8), dtype=np.uint8)
    m = np.empty((s12.shape[0], 8), dtype=np.uint8)
    for j in range(8):
        if j < 4:
            sc[:, j] = s12[:, j] & 63
            m[:, j] = s12[:, j + 4] & 63
        else:
            sc[:, j] = (s12[:, j + 4] & 0xF) | ((s12[:, j - 4] >> 6) << 4)
            m[:, j] = (s12[:, j + 4] >> 4) | ((s12[:, j] >> 6) << 4)
    return sc, m


def quantize(gtype: int, x: np.ndarray) -> np.ndarray:
    if gtype == GGML_F32:
        return np.ascontiguousarray(x, dtype=F32).view(np.uint8)
    if gtype == GGML_F16:
        return np.ascontiguousarray(x, dtype=F32).astype(np.float16).view(np.uint8)
    if gtype == GGML_Q8_0:
        return quantize_q8_0(x)
    if gtype == GGML_Q4_0:
        return quantize_q4_0(x)
    if gtype == GGML_Q4_K:
        return quantize_q4_K(x)
    raise ValueError(f"cannot quantize to type {gtype}")


# ------------------------------------------------------------------------------------------------
# GGUF v3
# ------------------------------------------------------------------------------------------------
@dataclass
class TensorInfo:
    name: str
    gtype: int
    ne: tuple          # ggml order: ne[0] = contiguous dimension
    data: bytes | np.ndarray | None = None
    offset: int = 0


@dataclass
class GGUFWriter:
    kv: list = field(default_factory=list)        # (key, vtype, value, elem_type)
    tensors: list = field(default_factory=list)

    def add(self, key: str, value, vtype: int | None = None, elem_type: int | None = None):
        if vtype is None:
            if isinstance(value, bool):
                vtype = _BOOL
            elif isinstance(value, int):
                vtype = _U32 if value >= 0 else _I32
            elif isinstance(value, float):
                vtype = _F32
            elif isinstance(value, str):
                vtype = _STR
            elif isinstance(value, (list, tuple)):
                vtype = _ARR
                if elem_type is None:
                    if all(isinstance(v, str) for v in value):
                        elem_type = _STR
                    elif all(isinstance(v, int) and not isinstance(v, bool) for v in value):
                        elem_type = _I32
                    else:
                        elem_type = _F32
            else:
                raise TypeError(f"{key}: cannot infer GGUF type of {type(value)}")
        self.kv.append((key, vtype, value, elem_type))

    def add_tensor(self, name: str, gtype: int, ne: tuple, data):
        nbytes = row_bytes(gtype, ne[0]) * int(np.prod(ne[1:], dtype=np.int64))
        buf = memoryview(np.ascontiguousarray(data).view(np.uint8).reshape(-1))
        if buf.nbytes != nbytes:
            raise ValueError(f"{name}: {buf.nbytes} bytes for {ne} {TYPE_NAMES.get(gtype)}, expected {nbytes}")
        self.tensors.append(TensorInfo(name, gtype, tuple(int(v) for v in ne), buf))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _value(self, vtype, value, elem_type) -> bytes:
        if vtype == _STR:
            return self._str(value)
        if vtype == _ARR:
            out = struct.pack("<IQ", elem_type, len(value))
            for v in value:
                out += self._value(elem_type, v, None)
            return out
        return struct.pack(_SCALAR_FMT[vtype], value)

    def write(self, path: str):
        head = bytearray()
        head += b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))
        for key, vtype, value, et in self.kv:
            head += self._str(key) + struct.pack("<I", vtype) + self._value(vtype, value, et)
        off = 0
        for t in self.tensors:
            t.offset = off
            head += self._str(t.name) + struct.pack("<I", len(t.ne))
            head += b"".join(struct.pack("<Q", v) for v in t.ne)
            head += struct.pack("<IQ", t.gtype, t.offset)
            off += (t.data.nbytes + ALIGN - 1) // ALIGN * ALIGN
        pad = (-len(head)) % ALIGN
        with open(path, "wb") as f:
            f.write(head)
            f.write(b"\0" * pad)
            for t in self.tensors:
                f.write(t.data)
                f.write(b"\0" * ((-t.data.nbytes) % ALIGN))


@dataclass
class GGUFFile:
    kv: dict
    tensors: dict      # name -> TensorInfo with .data a uint8 memmap slice
    path: str = ""

    def tensor_bytes(self, name: str) -> np.ndarray:
        return self.tensors[name].data

    def tensor_f32(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        rows = int(np.prod(t.ne[1:], dtype=np.int64))
        return dequantize(t.gtype, np.asarray(t.data).reshape(rows, -1), t.ne[0]).reshape(tuple(reversed(t.ne)))


def read_gguf(path: str) -> GGUFFile:
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    buf = memoryview(mm)
    p = 0

    def take(fmt):
        nonlocal p
        v = struct.unpack_from(fmt, buf, p)
        p += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def rstr():
        nonlocal p
        n = take("<Q")
        s = bytes(buf[p:p + n]).decode("utf-8", errors="replace")
        p += n
        return s

    def rval(vt):
        if vt == _STR:
            return rstr()
        if vt == _ARR:
            et = take("<I")
            n = take("<Q")
            return [rval(et) for _ in range(n)]
        return take(_SCALAR_FMT[vt])

    if bytes(buf[0:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    p = 4
    _ver = take("<I")
    nt = take("<Q")
    nkv = take("<Q")
    kv = {}
    for _ in range(nkv):
        k = rstr()
        vt = take("<I")
        kv[k] = rval(vt)
    infos = []
    for _ in range(nt):
        name = rstr()
        nd = take("<I")
        ne = tuple(take("<Q") for _ in range(nd))
        gt = take("<I")
        off = take("<Q")
        infos.append(TensorInfo(name, gt, ne, None, off))
    align = int(kv.get("general.alignment", ALIGN))
    data0 = (p + align - 1) // align * align
    tensors = {}
    for t in infos:
        nbytes = row_bytes(t.gtype, t.ne[0]) * int(np.prod(t.ne[1:], dtype=np.int64))
        t.data = mm[data0 + t.offset: data0 + t.offset + nbytes]
        tensors[t.name] = t
    return GGUFFile(kv, tensors, path)
