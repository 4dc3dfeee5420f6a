"""Pinning of the CPU oracle's scalar numerics and ggml block formats (no GPU).

Each check is chosen so that a plausible slip in the restatement (a rounding mode, a sign, a block
layout, a dropped term, a summation order) fails it: exhaustive f16 conversion against numpy's IEEE
routines, quantizers against an independent numpy implementation plus closed-form round-trip bounds,
rounding-mode and tie-break known answers, dots against exact integer block sums, and LayerNorm /
GELU / attention against float64 references.
"""
import math

import numpy as np
import pytest

from jepa_amd import gguf
from oracle import oracle as O


# ------------------------------------------------------------------------------------------------- f16
def test_fp16_to_fp32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(8),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),          # subnormal halves
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6e-8, 2.98e-8, 5.96e-8,
                  np.inf, -np.inf, 1.00048828125, 1.0009765625, 1.00146484375], np.float32),   # overflow -> inf
        # exact ties between two halves: 1 + (2k + 1) * 2^-11 must go to the even neighbour
        (1.0 + (2 * np.arange(64) + 1) * 2.0 ** -11).astype(np.float32),
    ])
    got = O.fp32_to_fp16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------------------------- weight quantizers
@pytest.mark.parametrize("gtype", [gguf.GGML_Q8_0, gguf.GGML_Q4_0, gguf.GGML_Q4_K])
def test_weight_quantizers_match_independent_numpy(gtype):
    """The oracle's C quantizers and jepa_amd.gguf's numpy ones are separate implementations of the
    same ggml *_ref rules; they must agree byte for byte."""
    rng = np.random.default_rng(gtype)
    x = (rng.standard_normal((64, 512)) * 0.05).astype(np.float32)
    x[3] = 0.0                                   # all-zero row
    x[5, :32] = 1e-3                             # constant block
    np.testing.assert_array_equal(O.quantize_weight(gtype, x), gguf.quantize(gtype, x))


def test_q8_0_weight_roundtrip_bound_and_layout():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    raw = O.quantize_weight(O.OR_Q8_0, x)
    assert raw.shape == (16, 8 * 34)
    y = O.dequantize(O.OR_Q8_0, raw, 256)
    blocks = raw.reshape(-1, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(16, 8)
    q = blocks[:, 2:].view(np.int8)
    # d = amax/127 as f16, the largest element maps to +-127, every element within d/2 (+ f16 slack)
    amax = np.abs(x.reshape(16, 8, 32)).max(-1)
    np.testing.assert_array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.abs(q).max() == 127
    err = np.abs(y - x).reshape(16, 8, 32).max(-1)
    assert np.all(err <= d * 0.5 + amax * 2e-3)


def test_q4_0_codes_and_roundtrip():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    raw = O.quantize_weight(O.OR_Q4_0, x)
    b = raw.reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    # d = max / -8 where max is the signed value of largest magnitude: that element gets code 0
    xb = x.reshape(-1, 32)
    idx = np.argmax(np.abs(xb), axis=1)
    mx = xb[np.arange(len(idx)), idx]
    np.testing.assert_array_equal(d, (mx / np.float32(-8)).astype(np.float16).astype(np.float32))
    lo, hi = b[:, 2:] & 0xF, b[:, 2:] >> 4
    codes = np.concatenate([lo, hi], axis=1)
    assert np.all(codes[np.arange(len(idx)), idx] == 0)
    y = O.dequantize(O.OR_Q4_0, raw, 128).reshape(-1, 32)
    # codes span [-8, 7] d with the extreme at -8 d: same-sign elements round to within d/2, elements of
    # the opposite sign beyond 7.5 d clamp to 7 d (error up to d)
    same = np.sign(xb) == np.sign(mx)[:, None]
    err = np.abs(y - xb)
    slack = np.abs(mx)[:, None] * 2e-3
    half = np.broadcast_to(np.abs(d)[:, None] * 0.5 + slack, err.shape)
    assert np.all(err[same] <= half[same])
    assert np.all(err <= np.abs(d)[:, None] + slack)


def test_q4_K_dequantize_matches_numpy_and_bounds():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((4, 512)) * 0.1).astype(np.float32)
    raw = O.quantize_weight(O.OR_Q4_K, x)
    y = O.dequantize(O.OR_Q4_K, raw, 512)
    np.testing.assert_array_equal(y.view(np.uint32), gguf.dequantize(gguf.GGML_Q4_K, raw, 512).view(np.uint32))
    # 4-bit codes over a per-sub-block [min, max] range: error within ~ one code step of the range
    xs = x.reshape(-1, 32)
    step = (xs.max(1) - np.minimum(xs.min(1), 0)) / 15
    assert np.all(np.abs(y.reshape(-1, 32) - xs).max(1) <= step * 0.75 + 2e-3)


def _q4k_subblocks(rng, count):
    """Sub-blocks of 32 values of the shapes the fit treats differently: centred, all positive (the
    min clamps to 0), uniform, heavy-tailed, and one outlier over a tiny spread."""
    out = []
    for i in range(count):
        k = i % 5
        if k == 0:
            x = rng.standard_normal(32)
        elif k == 1:
            x = rng.standard_normal(32) + 3.0
        elif k == 2:
            x = rng.uniform(-1, 1, 32)
        elif k == 3:
            x = rng.standard_t(2, 32)
        else:
            x = rng.standard_normal(32) * 0.01
            x[rng.integers(32)] = 0.5
        out.append(x.astype(np.float32))
    return out


def _q4k_weights(x):
    # the weights quantize_row_q4_K_ref gives a sub-block: sqrt(mean x^2) + |x|
    return (np.float32(np.sqrt(np.float32((x * x).sum()) / np.float32(32))) + np.abs(x)).astype(np.float32)


def _wls(L, x, w):
    """Weighted least-squares scale and min of x ~ s * L + m by numpy's lstsq, the min clamped to <= 0
    (then the scale alone is refitted)."""
    sw = np.sqrt(w)
    (s, m), *_ = np.linalg.lstsq(np.stack([L, np.ones_like(L)], 1) * sw[:, None], x * sw, rcond=None)
    if m > 0:
        m, s = 0.0, float((w * L * x).sum() / (w * L * L).sum())
    return float(s), float(m)


def test_q4_K_subblock_fit_replays_the_candidate_search():
    """make_qkx2_quants (ggml-quants.c of ggml 36da5713, which the reference pins and does not ship) is
    pinned without retyping its sums: a float64 replay of its search, each candidate's scale and min
    solved by numpy's weighted lstsq, must pick the same levels. Candidate i has levels
    clamp(rint(iscale (x - min)), 0, 15) with iscale = (-1 + 0.1 i + 15) / (max - min) over the current
    min, which an accepted candidate replaces (a search over a fixed min picks other levels on many
    sub-blocks). Every result is also a weighted least-squares fit of its own levels, or the min/max
    start, and never worse than that start."""
    rng = np.random.default_rng(7)
    n = same = 0
    for x in _q4k_subblocks(rng, 1500):
        w = _q4k_weights(x)
        s, m, L = O.make_qkx2_quants(x, w)
        x64, w64, L64 = x.astype(np.float64), w.astype(np.float64), L.astype(np.float64)
        err = lambda s_, m_, L_: float((w64 * (s_ * L_ + m_ - x64) ** 2).sum())
        mn, mx = np.float32(min(float(x.min()), 0.0)), np.float32(x.max())
        isc = np.float32(15) / (mx - mn)
        L0 = np.clip(np.rint(isc * (x - mn)), 0, 15).astype(np.float64)
        s0, m0 = float(np.float32(1) / isc), float(mn)
        rs, rm, rL, best = s0, m0, L0, err(s0, m0, L0)
        for i in range(21):
            isc = (np.float32(-1) + np.float32(0.1) * np.float32(i) + np.float32(15)) / (mx - np.float32(rm))
            Li = np.clip(np.rint(isc * (x - np.float32(rm))), 0, 15).astype(np.float64)
            if Li.min() == Li.max():
                continue
            cs, cm = _wls(Li, x64, w64)
            e = err(cs, cm, Li)
            if e < best:
                rs, rm, rL, best = cs, cm, Li, e
        n += 1
        e = err(s, m, L64)
        assert e <= err(s0, m0, L0) * (1 + 1e-6)
        if np.array_equal(L64, L0) and abs(s - s0) <= 1e-6 * s0:
            pass                                           # kept the min/max start
        else:
            fs, fm = _wls(L64, x64, w64)
            assert abs(s - fs) <= 2e-4 * abs(fs) and abs(m - fm) <= 2e-4 * abs(fs), (s, m, fs, fm)
        if np.array_equal(L64, rL):
            same += 1
            assert abs(s - rs) <= 2e-4 * abs(rs) and abs(m - rm) <= 2e-4 * abs(rs)
        else:
            # a near-tie decided the other way in float32 sums: then no worse than the replay's pick
            assert e <= best * (1 + 1e-4), (e, best)
    assert same >= 0.99 * n, (same, n)


def test_q4_K_block_scales_and_final_levels():
    """quantize_row_q4_K_ref after the fits: d = f16(max scale / 63), dmin = f16(max min / 63), six-bit
    sub-block scales and mins rint(63 * s_j / max), and every value re-fitted to the nearest level of
    its quantized sub-block scale and min, clamped to [0, 15]."""
    rng = np.random.default_rng(11)
    subs = _q4k_subblocks(rng, 8 * 40)
    x = np.concatenate(subs).reshape(40, 256)
    raw = O.quantize_weight(O.OR_Q4_K, x).reshape(-1, 144)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = raw[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mq = gguf.q4k_scales_mins(raw[:, 4:16])
    y = O.dequantize(O.OR_Q4_K, raw, 256).reshape(40, 8, 32)
    for b in range(40):
        fits = [O.make_qkx2_quants(v, _q4k_weights(v)) for v in x[b].reshape(8, 32)]
        scales = np.array([f[0] for f in fits], np.float32)
        mins = np.array([-f[1] for f in fits], np.float32)
        ms, mm = scales.max(), mins.max()
        assert d[b] == np.float16(ms / np.float32(63)).astype(np.float32)
        assert dmin[b] == np.float16(mm / np.float32(63)).astype(np.float32)
        np.testing.assert_array_equal(sc[b], np.minimum(np.rint(np.float32(63) / ms * scales), 63))
        np.testing.assert_array_equal(mq[b], np.minimum(np.rint(np.float32(63) / mm * mins), 63))
        for j in range(8):
            dj, mj = np.float32(d[b] * sc[b, j]), np.float32(dmin[b] * mq[b, j])
            if dj == 0:
                continue
            xs = x[b, 32 * j:32 * j + 32].astype(np.float64)
            levels = dj * np.arange(16, dtype=np.float64) - mj
            nearest = levels[np.abs(xs[:, None] - levels[None, :]).argmin(1)]
            np.testing.assert_allclose(y[b, j], nearest, rtol=0, atol=1e-5 * float(dj))


def test_q4_K_recovers_values_on_its_own_grid():
    """Values that lie exactly on a q4_K grid (f16 d and dmin, six-bit scales and mins with 63 among
    them, every sub-block using levels 0 and 15) come back exactly: the fit, the requantization of the
    scales and the final levels all reproduce the grid."""
    rng = np.random.default_rng(12)
    for _ in range(20):
        d = np.float32(np.float16(rng.uniform(1e-3, 2e-2)))
        dmin = np.float32(np.float16(rng.uniform(1e-3, 2e-2)))
        sc = rng.integers(1, 64, 8)
        sc[rng.integers(8)] = 63
        m = rng.integers(0, 64, 8)
        m[rng.integers(8)] = 63
        q = rng.integers(0, 16, (8, 32))
        q[:, 0], q[:, 1] = 0, 15
        a = (d * sc.astype(np.float32)).astype(np.float32)
        b = (dmin * m.astype(np.float32)).astype(np.float32)
        x = ((a[:, None] * q.astype(np.float32)).astype(np.float32) - b[:, None]).reshape(1, 256)
        raw = O.quantize_weight(O.OR_Q4_K, x)
        y = O.dequantize(O.OR_Q4_K, raw, 256)
        np.testing.assert_allclose(y, x, rtol=0, atol=1e-6 * float(np.abs(x).max()))
        got_sc, got_m = gguf.q4k_scales_mins(raw.reshape(-1, 144)[:, 4:16])
        np.testing.assert_array_equal(got_sc[0], sc)
        np.testing.assert_array_equal(got_m[0], m)


# ------------------------------------------------------------------------------ activation quantizers
def test_q8_0_activation_rounds_half_to_even():
    """The x86 CPU path rounds x*127/amax half-to-even (quantize_row_q8_0, AVX2); roundf (half away
    from zero) would give 1, 3, -1, -3 below."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0                                 # amax = 127, so id = 1 exactly
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -3.5]
    raw = O.quantize_act(O.OR_Q8_0, x)
    d = raw[:2].copy().view(np.float16)[0]
    q = raw[2:].view(np.int8)
    assert d == np.float16(1.0)
    assert q[0] == 127
    np.testing.assert_array_equal(q[1:9], [0, 2, 2, 0, -2, -2, 126, -4])


def test_q8_0_activation_reciprocal_form():
    """ggml's x86 quantize_row_q8_0 (AVX2 path, ggml 36da5713) multiplies by id = 127 / amax, computed
    once per block in float32; the _ref form takes id = 1 / d with d = amax / 127, and a third reading
    divides x / d. At amax = 47.538044 the two reciprocals differ in the last bit (2.6715446 against
    2.6715443), and the x below sit where that decides the code: x * (127 / amax) rounds to exactly
    1.5 and 3.5 in float32 (ties, half-even: 2 and 4), while x * (1 / d) and x / d land one unit below
    (codes 1 and 3). The oracle must give the 127 / amax codes."""
    from fractions import Fraction as Fr
    f = np.float32
    amax = f(47.53804397583008)
    xs = [f(0.5614729523658752), f(1.3101035356521606)]
    id_a = f(127) / amax
    d = amax / f(127)
    id_b = f(1) / d
    assert id_a != id_b
    # the products, exactly: float32 rounding of the exact rational products
    for x, tie in zip(xs, (Fr(3, 2), Fr(7, 2))):
        assert Fr(float(f(x * id_a))) == tie
        assert Fr(float(f(x * id_b))) < tie and Fr(float(f(x / d))) < tie
    x = np.zeros(32, np.float32)
    x[0] = amax
    x[1], x[2], x[3], x[4] = xs[0], xs[1], -xs[0], -xs[1]
    raw = O.quantize_act(O.OR_Q8_0, x)
    q = raw[2:].view(np.int8)
    assert raw[:2].copy().view(np.float16)[0] == np.float16(d)
    np.testing.assert_array_equal(q[:5], [127, 2, 4, -2, -4])


def test_q8_0_activation_scale_and_zero_block():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(64).astype(np.float32)
    x[32:] = 0.0
    raw = O.quantize_act(O.OR_Q8_0, x).reshape(2, 34)
    d0 = raw[0, :2].copy().view(np.float16)[0]
    assert d0 == np.float16(np.abs(x[:32]).max() / np.float32(127))
    assert np.abs(raw[0, 2:].view(np.int8)).max() == 127
    assert raw[1, :2].copy().view(np.uint16)[0] == 0 and not raw[1, 2:].any()


def test_q8_K_first_largest_and_sign_convention():
    """quantize_row_q8_K_ref: max = the FIRST element of largest |x| (kept signed), iscale = -127/max,
    q = min(127, nearest_int(iscale * x)), d = 1/iscale, bsums over 16."""
    x = np.zeros(256, np.float32)
    x[3] = -5.0
    x[10] = 5.0                                  # same magnitude, later: must not be chosen
    x[20:36] = np.linspace(-4, 4, 16, dtype=np.float32)
    raw = O.quantize_act(O.OR_Q8_K, x)
    assert raw.size == 4 + 256 + 32
    d = raw[:4].copy().view(np.float32)[0]
    q = raw[4:260].view(np.int8)
    bs = raw[260:].copy().view(np.int16)
    iscale = np.float32(-127.0) / np.float32(-5.0)
    assert d == np.float32(1.0) / iscale
    assert q[3] == -127 and q[10] == 127
    np.testing.assert_array_equal(bs, q.reshape(16, 16).astype(np.int32).sum(1))


# ------------------------------------------------------------------------------------------- vec dot
def _f32_fma(a, b, c):
    # a*b is exact in float64 here (|a| < 2^24 integer, b a product of two f16 values); one rounding
    # of the float64 sum to float32 differs from a true fma only on exact halfway cases
    return np.float32(float(a) * float(b) + float(c))


def test_vec_dot_q8_0_is_blockwise_fma_of_exact_integer_sums():
    rng = np.random.default_rng(6)
    n = 1024
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    wr = O.quantize_weight(O.OR_Q8_0, w)
    ar = O.quantize_act(O.OR_Q8_0, x)
    got = O.vec_dot(O.OR_Q8_0, n, wr, ar)
    wb, ab = wr.reshape(-1, 34), ar.reshape(-1, 34)
    acc = np.float32(0)
    for b in range(n // 32):
        S = int((wb[b, 2:].view(np.int8).astype(np.int64) * ab[b, 2:].view(np.int8).astype(np.int64)).sum())
        dw = np.float32(wb[b, :2].copy().view(np.float16)[0])
        da = np.float32(ab[b, :2].copy().view(np.float16)[0])
        acc = _f32_fma(np.float32(S), dw * da, acc)
    assert np.float32(got) == acc


def test_vec_dot_q4_K_matches_superblock_formula():
    """Per super-block: s += (d*da) * sum_j sc_j S_j and sm += (dmin*da) * sum_j m_j (bsum_2j + bsum_2j+1),
    two accumulators joined at the end as s - sm (the structure of ggml's x86 q4_K x q8_K dot)."""
    rng = np.random.default_rng(7)
    n = 512
    w = (rng.standard_normal(n) * 0.05).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    wr = O.quantize_weight(O.OR_Q4_K, w)
    ar = O.quantize_act(O.OR_Q8_K, x)
    got = O.vec_dot(O.OR_Q4_K, n, wr, ar)
    acc = accm = np.float32(0)
    for sb in range(n // 256):
        blk = wr[sb * 144:(sb + 1) * 144]
        a = ar[sb * 292:(sb + 1) * 292]
        d = np.float32(blk[0:2].copy().view(np.float16)[0]); dmin = np.float32(blk[2:4].copy().view(np.float16)[0])
        sc, m = gguf.q4k_scales_mins(blk[None, 4:16])
        qs = blk[16:]
        q8 = a[4:260].view(np.int8).astype(np.int64)
        da = a[:4].copy().view(np.float32)[0]
        bs = a[260:].copy().view(np.int16).astype(np.int64)
        sumi = summ = 0
        for j in range(8):
            c = j // 2
            q4 = (qs[32 * c:32 * c + 32] & 0xF) if j % 2 == 0 else (qs[32 * c:32 * c + 32] >> 4)
            sumi += int(sc[0, j]) * int((q4.astype(np.int64) * q8[32 * j:32 * j + 32]).sum())
            summ += int(m[0, j]) * int(bs[2 * j] + bs[2 * j + 1])
        acc = _f32_fma(np.float32(sumi), np.float32(d * da), acc)
        accm = _f32_fma(np.float32(summ), np.float32(dmin * da), accm)
    assert np.float32(got) == np.float32(acc - accm)


@pytest.mark.parametrize("gtype", [O.OR_Q8_0, O.OR_Q4_0, O.OR_Q4_K, O.OR_F16])
def test_mul_mat_equals_vec_dot(gtype):
    """or_mul_mat's pre-expanded fast path gives exactly or_vec_dot's value for every output."""
    rng = np.random.default_rng(8 + gtype)
    n_out, n_in, M = 8, 512, 5
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.1).astype(np.float32)
    raw = w.astype(np.float16).view(np.uint8) if gtype == O.OR_F16 else O.quantize_weight(gtype, w)
    y = O.mul_mat(gtype, raw, n_out, n_in, x, bias)
    if gtype == O.OR_F16:
        act = [O.fp32_to_fp16(x[m]).view(np.uint8) for m in range(M)]
    else:
        act = [O.quantize_act(O.OR_Q8_K if gtype == O.OR_Q4_K else O.OR_Q8_0, x[m]) for m in range(M)]
    for m in range(M):
        for o in range(n_out):
            want = np.float32(np.float32(O.vec_dot(gtype, n_in, raw[o], act[m])) + bias[o])
            assert y[m, o].view(np.uint32) == want.view(np.uint32), (m, o)


# ------------------------------------------------------------------------------ ggml's x86 lane order
@pytest.fixture
def lanes():
    O.set_ggml_lanes(True)
    yield
    O.set_ggml_lanes(False)


def _lane_dot(gtype, w, x, no_mins=False):
    wr = O.quantize_weight(gtype, w)
    if no_mins:                       # q4_K: dmin = 0 in every super-block, so the mins term is zero
        wr.reshape(-1, 144)[:, 2:4] = 0
    ar = O.quantize_act(O.OR_Q8_K if gtype == O.OR_Q4_K else O.OR_Q8_0, x)
    return np.float32(O.vec_dot(gtype, w.size, wr, ar))


@pytest.mark.parametrize("gtype", [O.OR_Q8_0, O.OR_Q4_0, O.OR_Q4_K])
def test_ggml_lanes_one_lane_is_the_block_chain(gtype):
    """With the activations zero outside the four elements 4l..4l+3 of every 32-element group, only
    lane l of ggml's eight is ever non-zero: its per-block fma chain is the whole dot and the
    horizontal sum adds zeros, so the lane order equals the one-chain order bit for bit, for every l
    (q4_K with dmin set to zero in every super-block, so the mins lanes vanish too). This pins which
    elements share a lane (four consecutive ones) and that a lane takes one fma per block."""
    rng = np.random.default_rng(30 + gtype)
    n = 1024
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    nm = gtype == O.OR_Q4_K
    for l in range(8):
        x = rng.standard_normal(n).astype(np.float32)
        keep = np.zeros(32, bool)
        keep[4 * l:4 * l + 4] = True
        x[~np.tile(keep, n // 32)] = 0.0
        O.set_ggml_lanes(False)
        chain = _lane_dot(gtype, w, x, nm)
        O.set_ggml_lanes(True)
        try:
            lane = _lane_dot(gtype, w, x, nm)
        finally:
            O.set_ggml_lanes(False)
        assert lane.view(np.uint32) == chain.view(np.uint32), (l, lane, chain)


def _move_groups(v, perm):
    """element group g (elements 4g..4g+3 of every 32-element block) moved to group perm[g]"""
    b = v.reshape(-1, 8, 4)
    out = np.empty_like(b)
    out[:, list(perm), :] = b
    return out.reshape(v.shape)


@pytest.mark.parametrize("gtype", [O.OR_Q8_0, O.OR_Q4_0])
def test_ggml_lanes_horizontal_sum_symmetries(lanes, gtype):
    """hsum_float_8 = ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)) is unchanged when lanes are
    exchanged by the symmetries of that tree (0<->4; the pair (0,4)<->(2,6); the halves
    (0,4,2,6)<->(1,5,3,7)). Moving the element groups of both operands that way moves whole lanes, so
    the dot must come out bit-identical; the one-chain order sees only exact integer block sums and is
    unchanged by any move. Exchanging lanes 0 and 1 alone is not a symmetry of the tree and changes
    the value on these data, which shows the lanes are really summed apart."""
    rng = np.random.default_rng(40 + gtype)
    n = 4096
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    x = (rng.standard_normal(n) * np.repeat(rng.uniform(0.1, 10.0, n // 32), 32)).astype(np.float32)
    base = _lane_dot(gtype, w, x)
    # (the block quantizers are permutation-equivariant within a block: the scale comes from the
    # block's largest magnitude, each code from its own value)
    sym = [(4, 1, 2, 3, 0, 5, 6, 7), (2, 1, 0, 3, 6, 5, 4, 7), (1, 0, 3, 2, 5, 4, 7, 6)]
    for perm in sym:
        got = _lane_dot(gtype, _move_groups(w, perm), _move_groups(x, perm))
        assert got.view(np.uint32) == base.view(np.uint32), (perm, got, base)
    swap01 = (1, 0, 2, 3, 4, 5, 6, 7)
    other = _lane_dot(gtype, _move_groups(w, swap01), _move_groups(x, swap01))
    assert other != base


def test_ggml_lanes_q4_K_against_simd_restatement(lanes):
    """q4_K x q8_K in ggml's AVX2 form, restated with numpy arrays shaped as the registers: per
    super-block an [8] int32 register of sc_j * (four consecutive products) summed over sub-blocks,
    acc[8] += (y.d * x.d) * sumi; a [4] register of m_2k q8s_2k + m_2k+1 q8s_2k+1 with q8s the
    pairwise-added bsums, acc_m[4] += (-y.d * x.dmin) * prod; then hsum_float_8(acc) + the two-step
    sum of acc_m. Weights of both signs (non-zero mins) and activations of varying block scale."""
    rng = np.random.default_rng(50)
    n = 2048
    f = np.float32
    for trial in range(4):
        w = (rng.standard_normal(n) * 0.05 + 0.01 * trial).astype(np.float32)
        x = (rng.standard_normal(n) * np.repeat(rng.uniform(0.2, 5.0, n // 256), 256)).astype(np.float32)
        wr = O.quantize_weight(O.OR_Q4_K, w)
        ar = O.quantize_act(O.OR_Q8_K, x)
        got = np.float32(O.vec_dot(O.OR_Q4_K, n, wr, ar))
        acc = np.zeros(8, np.float32)
        accm = np.zeros(4, np.float32)
        for sb in range(n // 256):
            blk = wr[sb * 144:(sb + 1) * 144]
            a = ar[sb * 292:(sb + 1) * 292]
            d = f(blk[0:2].copy().view(np.float16)[0]); dmin = f(blk[2:4].copy().view(np.float16)[0])
            sc, m = gguf.q4k_scales_mins(blk[None, 4:16])
            qs = blk[16:]
            q8 = a[4:260].view(np.int8).astype(np.int64).reshape(8, 32)
            yd = a[:4].copy().view(np.float32)[0]
            bs = a[260:].copy().view(np.int16).astype(np.int64)
            q4 = np.stack([(qs[32 * (j // 2):32 * (j // 2) + 32] & 0xF) if j % 2 == 0 else (qs[32 * (j // 2):32 * (j // 2) + 32] >> 4)
                           for j in range(8)]).astype(np.int64)
            sumi = ((q4 * q8).reshape(8, 8, 4).sum(2) * sc[0].astype(np.int64)[:, None]).sum(0)     # [8] lanes
            q8s = bs.reshape(8, 2).sum(1)
            prod = (m[0].astype(np.int64) * q8s).reshape(4, 2).sum(1)                            # [4] lanes
            dd, dm = f(yd * d), f(-yd * dmin)
            acc = np.array([_f32_fma(f(v), dd, c) for v, c in zip(sumi, acc)], np.float32)
            accm = np.array([_f32_fma(f(v), dm, c) for v, c in zip(prod, accm)], np.float32)
        h8 = f(f(f(acc[0] + acc[4]) + f(acc[2] + acc[6])) + f(f(acc[1] + acc[5]) + f(acc[3] + acc[7])))
        h4 = f(f(accm[0] + accm[2]) + f(accm[1] + accm[3]))
        want = f(h8 + h4)
        assert got.view(np.uint32) == want.view(np.uint32), (trial, got, want)


@pytest.mark.parametrize("gtype", [O.OR_Q8_0, O.OR_Q4_K])
def test_ggml_lanes_mul_mat_equals_vec_dot(lanes, gtype):
    """The pre-expanded mul_mat path and vec_dot agree in the lane order too."""
    rng = np.random.default_rng(60 + gtype)
    n_out, n_in, M = 6, 512, 4
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    raw = O.quantize_weight(gtype, w)
    y = O.mul_mat(gtype, raw, n_out, n_in, x, None)
    for m in range(M):
        act = O.quantize_act(O.OR_Q8_K if gtype == O.OR_Q4_K else O.OR_Q8_0, x[m])
        for o in range(n_out):
            want = np.float32(O.vec_dot(gtype, n_in, raw[o], act))
            assert y[m, o].view(np.uint32) == want.view(np.uint32), (m, o)


# ------------------------------------------------------------------------------ LayerNorm, GELU, attn
def test_layer_norm_against_float64():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((33, 1024)) * 3 + 0.5).astype(np.float32)
    w = rng.standard_normal(1024).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    y = O.layer_norm(x, w, b, 1e-6)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-6) * w + b
    assert np.abs(y - ref).max() <= 2e-6 * np.abs(ref).max()


def test_gelu_erf_against_math_erf():
    xs = np.concatenate([np.linspace(-8, 8, 4001), [0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0]]).astype(np.float32)
    for v in xs:
        ref = 0.5 * float(v) * (1.0 + math.erf(float(v) / math.sqrt(2.0)))
        got = O.gelu_erf(float(v))
        assert abs(got - ref) <= 4e-7 * max(1.0, abs(ref)), (v, got, ref)


def test_gpu_gelu_form_against_float64():
    """The oracle's restatement of the GPU epilogue's GELU (x Phi(x), the normal tail h = Phi(-|x|) as
    2^Q(min(|x|, 5.5)) with one degree-8 polynomial) against the exact x Phi(x): Phi within 3 units of
    2^-24 over every f16 value in [-12, 12] and a dense sample, GELU(x) = x exactly from 5.5 on, and
    GELU(0) = 0. A coefficient slip, a dropped Horner step or a swapped branch moves Phi far past this."""
    from scipy.special import erfc
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[h <= 12.0]
    x = np.concatenate([h, -h[1:], np.linspace(-8, 8, 400001, dtype=np.float32)]).astype(np.float32)
    prev = O.get_rounding()
    try:
        O.set_rounding(O.ROUND_GELU)
        got = O.gelu_erf_array(x).astype(np.float64)
    finally:
        O.set_rounding(prev)
    xd = x.astype(np.float64)
    phi = 0.5 * erfc(-xd / np.sqrt(2.0))
    exact = xd * phi
    err = np.abs(got - exact)
    # |x| * (3 units of 2^-24 in Phi) plus the final product's rounding
    assert np.all(err <= np.abs(xd) * 3 * 2.0 ** -24 + np.abs(exact) * 2.0 ** -24), float((err / np.maximum(np.abs(xd), 1e-30)).max())
    assert np.all(got[x >= 5.5] == x[x >= 5.5]) and np.all(got[x == 0] == 0)


def test_attention_against_float64():
    rng = np.random.default_rng(10)
    n, H, hd = 77, 3, 64
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    k = rng.standard_normal((n, H * hd)).astype(np.float32)
    v = rng.standard_normal((n, H * hd)).astype(np.float32)
    out = O.attention(q, k, v, H, kv_f16=True)
    ref = np.zeros((n, H * hd))
    for h in range(H):
        sl = slice(h * hd, (h + 1) * hd)
        kh = k[:, sl].astype(np.float16).astype(np.float64)
        vh = v[:, sl].astype(np.float16).astype(np.float64)
        s = q[:, sl].astype(np.float64) @ kh.T / 8.0
        p = np.exp(s - s.max(1, keepdims=True))
        ref[:, sl] = (p / p.sum(1, keepdims=True)) @ vh
    assert np.abs(out - ref).max() <= 2e-5 * np.abs(ref).max()


# ------------------------------------------------------------------------------------ block-causal mask
@pytest.mark.parametrize("gt,gh,gw,npre", [(4, 4, 4, 1), (3, 5, 7, 0), (2, 2, 3, 2)])
def test_block_causal_mask_rule(oracle, gt, gh, gw, npre):
    """Every entry against the rule of the reference's mask test (tests/test-ops.cpp:271-290): prefix
    rows see everything; a patch query sees a patch key of its own or an earlier temporal slot and
    never a prefix key; closed entries are -inf."""
    m = oracle.block_causal_mask(gt, gh, gw, npre)
    tpf = gh * gw
    n = npre + gt * tpf
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    want = (i < npre) | ((j >= npre) & ((j - npre) // tpf <= (i - npre) // tpf))
    assert m.shape == (n, n)
    assert np.array_equal(m == 0.0, want)
    assert np.all(np.isneginf(m[~want]))


def test_block_causal_mask_levjepa_density(oracle):
    """16 x 14 x 14 + CLS = 3137 rows: 53.1 % of the entries are open (docs/gguf-schema.md, levjepa note)."""
    m = oracle.block_causal_mask(16, 14, 14, 1)
    assert m.shape == (3137, 3137)
    assert round(100.0 * float((m == 0.0).mean()), 1) == 53.1


def test_masked_attention_matches_visible_key_softmax(oracle):
    """or_attention with the additive mask equals softmax over the visible keys only (double reference),
    and a row with no visible key gives zeros."""
    rng = np.random.default_rng(3)
    n, H, hd = 65, 2, 64
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    k = rng.standard_normal((n, H * hd)).astype(np.float32)
    v = rng.standard_normal((n, H * hd)).astype(np.float32)
    m = oracle.block_causal_mask(4, 4, 4, 1)
    m[5] = -np.inf                                   # a row with nothing visible
    got = oracle.attention(q, k, v, H, kv_f16=False, mask=m)
    for h in range(H):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T / 8.0 + m
        with np.errstate(invalid="ignore"):
            p = np.exp(s - s.max(1, keepdims=True))
        p[5] = 0.0
        den = p.sum(1, keepdims=True)
        ref = np.where(den > 0, p @ v[:, sl].astype(np.float64) / np.where(den > 0, den, 1), 0.0)
        assert np.abs(got[:, sl] - ref).max() < 1e-5
    assert np.all(got[5] == 0.0)
