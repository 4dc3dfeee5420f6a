"""Seeded synthetic encoder inputs, the same numbers tools/jepa-bench.cpp feeds.

jepa-bench (tools/jepa-bench.cpp:124-149) draws uint8 "pixels" from xorshift64* (seed 1234 by
default, :306), u8 = next() >> 33, and normalises them with the model's jepa.pre.* values:
x = (u8 * (1/255) - mean[c]) * (1/std[c]), in NCTHW order (batch, channel, frame, pixel).
"""
from __future__ import annotations

import numpy as np

_MASK = (1 << 64) - 1


def xorshift_u8(seed: int, n: int) -> np.ndarray:
    """n bytes of the xorshift64* stream, exactly as jepa-bench's rng::u8()."""
    s = seed if seed else 0x9E3779B97F4A7C15
    out = np.empty(n, dtype=np.uint8)
    # vectorised in chunks: the recurrence is sequential, so run it in pure Python per value but
    # keep it cheap by working on Python ints (about 1.5 M values/s)
    for i in range(n):
        s ^= s >> 12
        s ^= (s << 25) & _MASK
        s ^= s >> 27
        out[i] = ((s * 0x2545F4914F6CDD1D) & _MASK) >> 33 & 0xFF
    return out


def make_input(n_batch: int, n_frames: int, h: int, w: int, seed: int = 1234,
               mean=(0.485, 0.456, 0.406), std=(0.229, 0.224, 0.225), fast: bool = False) -> np.ndarray:
    """NCTHW float32 input. fast=True replaces the xorshift stream by numpy's PCG64 (same
    distribution, different numbers) for shapes too large for the sequential generator."""
    n = n_batch * 3 * n_frames * h * w
    if fast:
        u8 = np.random.default_rng(seed).integers(0, 256, size=n, dtype=np.uint8)
    else:
        u8 = xorshift_u8(seed, n)
    x = u8.astype(np.float32).reshape(n_batch, 3, n_frames * h * w)
    out = np.empty_like(x)
    for c in range(3):
        m = np.float32(mean[c])
        istd = np.float32(1.0) / np.float32(std[c] if std[c] != 0 else 1.0)
        out[:, c, :] = ((x[:, c, :] * np.float32(1.0 / 255.0)).astype(np.float32) - m) * istd
    return out.reshape(n_batch, 3, n_frames, h, w)
