"""The oracle's 3-D RoPE (tables and application) against the reference's own golden vectors.

tests/golden/rope3d holds the fixtures the reference checks src/rope3d.cpp with (reference
tests/vectors/rope3d, produced by its scripts/gen_rope_ref.py from the transformers / Meta V-JEPA 2
and 2.1 code). Each case gives the per-axis cos/sin rows [2, gt+gh+gw, d], an input x [N, D] and the
rotated output [N, D]; the checks mirror reference tests/test-ops.cpp:151-245 with its tolerance 1e-5.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "rope3d")
TOL = 1e-5


def _cases():
    out = []
    for line in open(os.path.join(GOLD, "manifest.txt")):
        if line.startswith("#") or not line.strip():
            continue
        name, tag, variant, hd, gt, gh, gw, n, interp, tt, th, tw, theta = line.split()
        out.append(dict(name=name, tag=tag, variant=int(variant), hd=int(hd), grid=(int(gt), int(gh), int(gw)),
                        n=int(n), interp=int(interp), train=(int(th), int(tw)), theta=float(theta)))
    return out


def _load(name):
    return np.load(os.path.join(GOLD, name + ".npy"), allow_pickle=False)


def _reference_tables(axes, grid, D, ids):
    """[n, D] tables from the factorised axis rows: dims [a*d, (a+1)*d) rotate with axis a, the rest
    are identity (cos 1, sin 0); token i -> (t, h, w) T-major (reference src/rope3d.h:10-14)."""
    gt, gh, gw = grid
    d = axes.shape[2]
    cos = np.ones((len(ids), D), np.float32)
    sin = np.zeros((len(ids), D), np.float32)
    for r, i in enumerate(ids):
        t, h, w = i // (gh * gw), (i % (gh * gw)) // gw, i % gw
        for a, row in enumerate((t, gt + h, gt + gh + w)):
            cos[r, a * d:(a + 1) * d] = axes[0, row]
            sin[r, a * d:(a + 1) * d] = axes[1, row]
    return cos, sin


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c['name']}-{c['tag']}")
def test_rope_golden(case):
    D, grid = case["hd"], case["grid"]
    n_full = grid[0] * grid[1] * grid[2]
    axes = _load(f"{case['name']}_{case['tag']}_axes")
    x = _load(f"{case['name']}_x")
    want = _load(f"{case['name']}_{case['tag']}_out")
    sub = case["n"] < n_full
    ids = _load(f"{case['name']}_ids") if sub else np.arange(n_full, dtype=np.int32)
    kw = dict(variant=case["variant"], interpolate=case["interp"], train=case["train"], theta=case["theta"])

    # full-grid raw tables
    c_full, s_full = O.rope_tables(grid, D, signed=False, **kw)
    rc, rs = _reference_tables(axes, grid, D, np.arange(n_full))
    assert max(np.abs(c_full - rc).max(), np.abs(s_full - rs).max()) < TOL
    # the rows of the case (subsampled when the case has ids)
    c_raw, s_raw = O.rope_tables(grid, D, ids=ids if sub else None, signed=False, **kw)
    rc, rs = _reference_tables(axes, grid, D, ids)
    assert max(np.abs(c_raw - rc).max(), np.abs(s_raw - rs).max()) < TOL
    # the signed table is exactly the raw one with the even lanes negated
    c_sgn, s_sgn = O.rope_tables(grid, D, ids=ids if sub else None, signed=True, **kw)
    lanes = np.arange(D) % 2 == 0
    np.testing.assert_array_equal(s_sgn.view(np.uint32), np.where(lanes, -s_raw, s_raw).view(np.uint32))
    np.testing.assert_array_equal(c_sgn.view(np.uint32), c_raw.view(np.uint32))
    # application on two identical heads
    xh = np.repeat(x[:, None, :], 2, axis=1)
    got = O.rope_apply(xh, c_sgn, s_sgn)
    assert np.abs(got - want[:, None, :]).max() < TOL


def test_rope_identity_at_origin():
    """Position (0, 0, 0) rotates nothing: cos 1, sin 0 on every lane (both variants)."""
    for variant in (0, 1):
        c, s = O.rope_tables((2, 2, 2), 64, variant=variant, signed=False)
        np.testing.assert_array_equal(c[0], np.ones(64, np.float32))
        np.testing.assert_array_equal(s[0], np.zeros(64, np.float32))


def test_rope_apply_is_a_rotation_for_interleaved_pairs():
    """V-JEPA 2.1 tables rotate each interleaved pair by one angle: pair norms are preserved."""
    rng = np.random.default_rng(3)
    c, s = O.rope_tables((2, 3, 5), 64, variant=1)
    x = rng.standard_normal((30, 1, 64)).astype(np.float32)
    y = O.rope_apply(x, c, s)
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(ny, nx, rtol=1e-5, atol=1e-6)


def _product_tables(case, ids, signed):
    """The tables libjepa.so uploads (jepa_amd_rope_tables, host only)."""
    import ctypes as C

    from jepa_amd import _lib
    L = _lib.lib()
    L.jepa_amd_rope_tables.restype = C.c_int
    L.jepa_amd_rope_tables.argtypes = [C.c_int] * 8 + [C.c_float, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
    D, (gt, gh, gw) = case["hd"], case["grid"]
    n = len(ids)
    c = np.zeros((n, D), np.float32)
    s = np.zeros((n, D), np.float32)
    ids32 = np.ascontiguousarray(ids, dtype=np.int32)
    rc = L.jepa_amd_rope_tables(D, gt, gh, gw, case["variant"], case["interp"], case["train"][0], case["train"][1], case["theta"],
                                ids32.ctypes.data, n, 1 if signed else 0, c.ctypes.data, s.ctypes.data)
    assert rc == 0
    return c, s


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c['name']}-{c['tag']}")
def test_product_rope_tables_golden(case):
    """The product's own tables (csrc/rope3d.cpp), not only the oracle's: within 1e-5 of the reference
    golden rows, bit-identical to the oracle's tables, and the rotation they drive reproduces the
    golden output (reference tests/test-ops.cpp:151-245)."""
    D, grid = case["hd"], case["grid"]
    n_full = grid[0] * grid[1] * grid[2]
    sub = case["n"] < n_full
    ids = _load(f"{case['name']}_ids") if sub else np.arange(n_full, dtype=np.int32)
    axes = _load(f"{case['name']}_{case['tag']}_axes")
    rc, rs = _reference_tables(axes, grid, D, ids)
    c_raw, s_raw = _product_tables(case, ids, signed=False)
    assert max(np.abs(c_raw - rc).max(), np.abs(s_raw - rs).max()) < TOL
    kw = dict(variant=case["variant"], interpolate=case["interp"], train=case["train"], theta=case["theta"])
    oc, os_ = O.rope_tables(grid, D, ids=ids if sub else None, signed=True, **kw)
    c_sgn, s_sgn = _product_tables(case, ids, signed=True)
    np.testing.assert_array_equal(c_sgn.view(np.uint32), oc.view(np.uint32))
    np.testing.assert_array_equal(s_sgn.view(np.uint32), os_.view(np.uint32))
    x = _load(f"{case['name']}_x")
    want = _load(f"{case['name']}_{case['tag']}_out")
    got = O.rope_apply(np.repeat(x[:, None, :], 2, axis=1), c_sgn, s_sgn)
    assert np.abs(got - want[:, None, :]).max() < TOL


def test_product_rope_tables_refuse_bad_ids():
    import ctypes as C

    from jepa_amd import _lib
    L = _lib.lib()
    L.jepa_amd_rope_tables.restype = C.c_int
    L.jepa_amd_rope_tables.argtypes = [C.c_int] * 8 + [C.c_float, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
    c = np.zeros((1, 64), np.float32)
    s = np.zeros((1, 64), np.float32)
    bad = np.array([8], np.int32)      # a 2x2x2 grid has ids 0..7
    assert L.jepa_amd_rope_tables(64, 2, 2, 2, 0, 0, 0, 0, 10000.0, bad.ctypes.data, 1, 1, c.ctypes.data, s.ctypes.data) == -1
    assert L.jepa_amd_rope_tables(64, 2, 2, 2, 0, 0, 0, 0, 10000.0, None, 9, 1, c.ctypes.data, s.ctypes.data) == -1
