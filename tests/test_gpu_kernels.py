"""Single-kernel parity on the GPU: each HIP kernel against the CPU oracle on the same inputs.

Bars: integer / block work (dequantization, activation quantization, q8_0 and q4_0 GEMMs) is
bit-exact; floating-point kernels are held to float round-off against the oracle (LayerNorm) or to
the reference's own attention gates (rel <= 1e-2, per-row cosine >= 0.9999; tests/test-attn.cpp:350-354).
"""
import ctypes as C

import numpy as np
import pytest

from jepa_amd import gguf

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a: np.ndarray):
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    torch.cuda.synchronize()
    return t


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_mfma_accumulator_layout(jlib):
    """The (lane, register) -> (row, col) map of v_mfma_f32_32x32x16_f16 that every epilogue uses."""
    L = jlib.lib()
    rng = np.random.default_rng(0)
    a = rng.integers(-8, 8, size=(32, 16)).astype(np.float32)
    b = rng.integers(-8, 8, size=(16, 32)).astype(np.float32)
    d = np.zeros((32, 32), np.float32)
    assert L.jepa_amd_mfma_probe(0, a.ctypes.data, b.ctypes.data, d.ctypes.data) == 0, jlib.error_text()
    np.testing.assert_array_equal(d, a @ b)


@pytest.mark.parametrize("gtype", [gguf.GGML_Q8_0, gguf.GGML_Q4_0, gguf.GGML_Q4_K, gguf.GGML_F16])
def test_dequantize_bitexact(jlib, oracle, gtype):
    rng = np.random.default_rng(gtype)
    n_rows, n_cols = 96, 1024
    w = (rng.standard_normal((n_rows, n_cols)) * 0.02).astype(np.float32)
    w[3, :] = 0.0                                   # all-zero blocks: d = 0
    w[5, :32] = np.linspace(-1, 1, 32)              # extremes of a block
    raw = gguf.quantize(gtype, w)
    want = oracle.dequantize(gtype, raw, n_cols) if gtype != gguf.GGML_F16 else w.astype(np.float16).astype(np.float32)
    draw = dev(raw.reshape(-1))
    y = torch.zeros((n_rows, n_cols), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    assert jlib.lib().jepa_amd_dequantize(0, gtype, draw.data_ptr(), n_rows, n_cols, y.data_ptr()) == 0, jlib.error_text()
    got = host(y)
    np.testing.assert_array_equal(got.view(np.uint32), want.reshape(n_rows, n_cols).view(np.uint32))


def _act_rows(rng, n_rows, n_cols):
    x = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
    x[1] = 0.0                                            # zero blocks
    x[2, :] = 1e-30                                       # tiny (subnormal scale)
    x[3, 0:256:2] = 3.0; x[3, 1:256:2] = -3.0             # equal |x| of both signs: first wins (q8_K)
    x[4, 7] = 1000.0                                      # one outlier
    x[5] = np.round(x[5] * 4) / 4                         # exact halves after scaling are likely
    # a q8_0 block where x * (127 / amax) lands on the ties 1.5 and 3.5 but x * (1 / d) and x / d one
    # unit below them (the reciprocal form of ggml's x86 quantize_row_q8_0 decides the codes)
    x[6, 0:32] = 0.25
    x[6, 0], x[6, 1], x[6, 2], x[6, 3], x[6, 4] = 47.53804397583008, 0.5614729523658752, 1.3101035356521606, -0.5614729523658752, -1.3101035356521606
    return x


@pytest.mark.parametrize("atype", [gguf.GGML_Q8_0, gguf.GGML_Q8_K])
def test_activation_quantization_bitexact(jlib, oracle, atype):
    rng = np.random.default_rng(atype)
    n_rows, n_cols = 512, 1024
    x = _act_rows(rng, n_rows, n_cols)
    want = oracle.quantize_act(atype, x)
    dx = dev(x)
    out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    rc = jlib.lib().jepa_amd_rownorm(0, dx.data_ptr(), n_rows, n_cols, None, None, 0.0, 0, atype, out.data_ptr())
    assert rc == 0, jlib.error_text()
    got = host(out).reshape(want.shape)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first rows {np.unique(bad[:, 0])[:8]}"


@pytest.mark.parametrize("out_type", [gguf.GGML_F32, gguf.GGML_Q8_0, gguf.GGML_Q8_K])
def test_layer_norm(jlib, oracle, out_type):
    rng = np.random.default_rng(7)
    n_rows, D = 1024, 1024
    x = (rng.standard_normal((n_rows, D)) * 3 + rng.standard_normal((n_rows, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    ref = oracle.layer_norm(x, w, b, 1e-6)
    dx, dw, db = dev(x), dev(w), dev(b)
    L = jlib.lib()
    if out_type == gguf.GGML_F32:
        y = torch.zeros((n_rows, D), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        assert L.jepa_amd_rownorm(0, dx.data_ptr(), n_rows, D, dw.data_ptr(), db.data_ptr(), 1e-6, 1, out_type, y.data_ptr()) == 0
        got = host(y)
        # both are ggml_norm in f32 with double accumulation: agreement to a few f32 ulps
        assert np.abs(got - ref).max() <= 4e-6 * np.abs(ref).max()
        # and to the double-precision definition (the reference's gate is < 1e-4, test-attn.cpp:628-653)
        xd = x.astype(np.float64)
        dref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * w + b
        assert np.abs(got - dref).max() < 1e-4
    else:
        want = oracle.quantize_act(out_type, ref)
        out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        assert L.jepa_amd_rownorm(0, dx.data_ptr(), n_rows, D, dw.data_ptr(), db.data_ptr(), 1e-6, 1, out_type, out.data_ptr()) == 0
        got = host(out).reshape(want.shape)
        # LN values agree to round-off, so a code can differ only where x*scale sits on a rounding tie
        blk = 34 if out_type == gguf.GGML_Q8_0 else 292
        frac = (got != want).mean()
        assert frac < 1e-3, f"{frac:.2e} of the bytes differ"


def _mul_mat_as_gpu(jlib, oracle, gtype, raw, n_out, n_in, x, bias, split=None):
    """the oracle's mul_mat with the K split the GPU uses for this shape (q8_0 / q4_0 with N <= 1024 run
    as two K halves whose sums are added; one chain otherwise)"""
    oracle.set_k_split(split if split is not None else jlib.lib().jepa_amd_gemm_split_of(gtype, n_out, n_in))
    try:
        return oracle.mul_mat(gtype, raw, n_out, n_in, x, bias)
    finally:
        oracle.set_k_split(1)


C2_SHAPES = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)]


@pytest.mark.parametrize("gtype,M", [(gguf.GGML_Q8_0, 256), (gguf.GGML_Q4_0, 256), (gguf.GGML_Q4_K, 256), (gguf.GGML_F16, 256),
                                     (gguf.GGML_Q8_0, 2048), (gguf.GGML_Q4_0, 2048), (gguf.GGML_Q4_K, 2048)])
@pytest.mark.parametrize("shape", C2_SHAPES)
def test_matmul_vs_oracle(jlib, oracle, gtype, M, shape):
    """GEMM microbench shapes (ViT-L qkv / proj / fc1 / fc2), at 256 tokens and, for the block-quantized
    types, at the configured 2048 tokens (the tiles and workgroup counts the encoder runs). q8_0, q4_0
    and q4_K: bit-exact with the oracle's ggml vec_dot restatement (same exact block sums, same fma per
    block in K order, q4_K's mins in their own accumulator); f16 within f32 summation-order rounding."""
    n_out, n_in = shape
    rng = np.random.default_rng(n_out * 7 + n_in + gtype + M)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.02).astype(np.float32)
    raw = gguf.quantize(gtype, w)
    want = _mul_mat_as_gpu(jlib, oracle, gtype, raw, n_out, n_in, x, bias)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    y = torch.zeros((M, n_out), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ms = C.c_double(0)
    rc = jlib.lib().jepa_amd_matmul(0, gtype, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, y.data_ptr(), 1, C.byref(ms))
    assert rc == 0, jlib.error_text()
    got = host(y)
    if gtype != gguf.GGML_F16:
        diff = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
        assert diff.size == 0, f"{len(diff)} outputs differ, max abs {np.abs(got - want).max():.3e}"
    else:
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 2e-5 * scale


def test_matmul_full_m2048_q8_0(jlib, oracle):
    """The C2 qkv shape at M = 2048 tokens, bit-exact."""
    n_out, n_in, M = 3072, 1024, 2048
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    raw = gguf.quantize(gguf.GGML_Q8_0, w)
    want = _mul_mat_as_gpu(jlib, oracle, gguf.GGML_Q8_0, raw, n_out, n_in, x, None)
    dw, dx = dev(raw.reshape(-1)), dev(x)
    y = torch.zeros((M, n_out), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    assert jlib.lib().jepa_amd_matmul(0, gguf.GGML_Q8_0, dw.data_ptr(), n_out, n_in, None, dx.data_ptr(), M, y.data_ptr(), 1, None) == 0
    np.testing.assert_array_equal(host(y).view(np.uint32), want.view(np.uint32))


def _q8k_blocks(raw, n_rows, n_cols):
    """ggml block_q8_K bytes -> (d f32 [rows][nb], codes int8 [rows][n_cols], bsums int16 [rows][nb*16])"""
    b = raw.reshape(n_rows, n_cols // 256, 292)
    d = b[:, :, 0:4].copy().view(np.float32)[..., 0]
    q = b[:, :, 4:260].copy().view(np.int8).reshape(n_rows, n_cols)
    bs = b[:, :, 260:292].copy().view(np.int16).reshape(n_rows, -1)
    return d, q, bs


@pytest.mark.parametrize("gtype,out_type,tile", [(gguf.GGML_Q4_K, gguf.GGML_Q8_K, -1), (gguf.GGML_Q4_K, gguf.GGML_Q8_K, 6),
                                                 (gguf.GGML_Q8_0, gguf.GGML_Q8_K, -1), (gguf.GGML_Q8_0, gguf.GGML_Q8_K, 7),
                                                 (gguf.GGML_F16, gguf.GGML_Q8_K, -1), (gguf.GGML_Q8_0, gguf.GGML_Q8_0, -1),
                                                 (gguf.GGML_Q4_0, gguf.GGML_F32, -1)])
def test_matmul_gelu_epilogue(jlib, oracle, gtype, out_type, tile):
    """fc1 with its fused epilogue: gelu_erf(X W^T + b) quantized for fc2 in the GEMM (q8_K: one
    256-block per workgroup row of waves, cross-wave max in LDS; both 256-wide tiles, 4 waves of 64
    features (tile 6) and 8 waves of 32 (tile 7, q4_K's default)). Against the oracle's exact GEMM, libm
    GELU and ggml quantizer: the GPU's erff and libm's may round differently, so a code can differ where
    a value sits at a rounding tie; rows 256..511 of W and b are zero (all-zero blocks, d = 0). M = 389 is
    ragged. The q8_K output must also hold its own invariants: bsums = sums of the codes, and the block
    maximum coded as -127 at its first position."""
    n_out, n_in, M = 768, 512 if gtype != gguf.GGML_Q4_K else 768, 389
    rng = np.random.default_rng(gtype * 31 + out_type)
    w = (rng.standard_normal((n_out, n_in)) * 0.05).astype(np.float32)
    w[256:512] = 0.0
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.1).astype(np.float32)
    bias[256:512] = 0.0
    raw = w.astype(np.float16).view(np.uint8) if gtype == gguf.GGML_F16 else gguf.quantize(gtype, w)
    pre = _mul_mat_as_gpu(jlib, oracle, gtype, raw, n_out, n_in, x, bias)
    ref = oracle.gelu_erf_array(pre)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    if out_type == gguf.GGML_F32:
        out = torch.zeros((M, n_out), dtype=torch.float32, device="cuda")
    else:
        out = torch.zeros(oracle.quantize_act(out_type, ref[:1]).size * M, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    L = jlib.lib()
    assert L.jepa_amd_gemm_tile(tile) == 0
    try:
        rc = L.jepa_amd_matmul_gelu(0, gtype, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, out_type, out.data_ptr(), 1,
                                    None)
    finally:
        L.jepa_amd_gemm_tile(-1)
    assert rc == 0, jlib.error_text()
    got = host(out)
    if out_type == gguf.GGML_F32:
        assert np.abs(got - ref).max() <= 4e-7 * np.abs(ref).max()
        return
    want = oracle.quantize_act(out_type, ref).reshape(-1)
    frac = (got != want).mean()
    assert frac < (5e-3 if gtype == gguf.GGML_F16 else 1e-3), f"{frac:.2e} of the bytes differ"
    if out_type == gguf.GGML_Q8_K:
        d, q, bs = _q8k_blocks(got, M, n_out)
        np.testing.assert_array_equal(bs, q.reshape(M, -1, 16).astype(np.int32).sum(-1))
        assert (d[:, 1] == 0).all() and (q[:, 256:512] == 0).all()
        live = np.delete(np.arange(n_out // 256), 1)
        qb = q.reshape(M, -1, 256)[:, live]
        assert (qb.min(-1) == -127).all()
        vals = ref.reshape(M, -1, 256)[:, live]
        first = np.abs(vals).argmax(-1)
        assert (np.take_along_axis(qb, first[..., None], -1) == -127).all()


def test_gelu_epilogue_every_f16_input(jlib, oracle):
    """The fused GELU (x Phi(x), the normal tail Phi(-|x|) as 2^Q(min(|x|, 5.5)) with one polynomial and
    one hardware exp2) on every finite f16 value in [-12, 12], through an f16 identity GEMM (exact: one
    product of 1.0 per output), against the oracle's libm form 0.5 x (1 + erff(x / sqrt 2)). Both are
    within a few units of 2^-24 of Phi, so outputs agree to 0.5 |x| 3.6e-7 plus an output rounding;
    subnormal and zero inputs, the clamp at 5.5 and the saturation of Phi to 1 are all in the set."""
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[h <= 12.0]
    x = np.concatenate([h, -h[1:]])
    n = 256
    rows = -(-x.size // n)
    xs = np.zeros(rows * n, dtype=np.float32)
    xs[:x.size] = x
    xs = xs.reshape(rows, n)
    w = np.eye(n, dtype=np.float16)
    dw, dx = dev(w.view(np.uint8).reshape(-1)), dev(xs)
    out = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    rc = jlib.lib().jepa_amd_matmul_gelu(0, gguf.GGML_F16, dw.data_ptr(), n, n, None, dx.data_ptr(), rows, gguf.GGML_F32,
                                         out.data_ptr(), 1, None)
    assert rc == 0, jlib.error_text()
    got = host(out).reshape(-1)[:x.size]
    want = oracle.gelu_erf_array(x)
    bound = 0.5 * np.abs(x) * 3.6e-7 + np.abs(want) * 2.0 ** -23
    bad = np.abs(got.astype(np.float64) - want) > bound
    assert not bad.any(), f"{bad.sum()} values out of bound, worst x = {x[np.argmax(np.abs(got - want) - bound)]}"
    assert np.array_equal(got[x == 0], want[x == 0]) and np.all(got[x >= 6] == x[x >= 6])


@pytest.mark.parametrize("gtype", [gguf.GGML_Q8_0, gguf.GGML_Q4_0, gguf.GGML_Q4_K])
@pytest.mark.parametrize("shape,M", [((1024, 4096), 2048), ((1024, 1024), 389), ((256, 512), 64)])
def test_matmul_split_k(jlib, oracle, gtype, shape, M):
    """Split-K (two workgroups per tile, one per K half; the second to finish adds the first's partial
    sums and runs the epilogue; the default for q4_K from K = 2048, forced for the other types): forced
    on and off, each bit-exact with the oracle summing the same K
    ranges (q4_K: whole super-blocks per half), over three launches in a row (the arrival counters
    must come back to zero); on a ragged M."""
    n_out, n_in = shape
    rng = np.random.default_rng(n_out + n_in + M + gtype)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.02).astype(np.float32)
    raw = gguf.quantize(gtype, w)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    L = jlib.lib()
    got = {}
    for split in (1, 2):
        y = torch.full((M, n_out), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        assert L.jepa_amd_gemm_split(split) == 0
        try:
            rc = L.jepa_amd_matmul(0, gtype, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, y.data_ptr(), 3, None)
        finally:
            L.jepa_amd_gemm_split(-1)
        assert rc == 0, jlib.error_text()
        got[split] = host(y)
        want = _mul_mat_as_gpu(jlib, oracle, gtype, raw, n_out, n_in, x, bias, split=split)
        diff = np.argwhere(got[split].view(np.uint32) != want.view(np.uint32))
        assert diff.size == 0, f"split {split}: {len(diff)} outputs differ, first {diff[:4].tolist()}"
    # by default only q4_K splits (from K = 2048); q8_0 / q4_0 run unsplit
    assert L.jepa_amd_gemm_split_of(gtype, n_out, n_in) == (2 if gtype == gguf.GGML_Q4_K and n_in >= 2048 else 1)
    # the two orders agree to rounding
    assert np.abs(got[1] - got[2]).max() <= 1e-5 * np.abs(got[1]).max()


@pytest.mark.parametrize("shape", [(384, 1536), (384, 384), (1024, 4096)])
def test_matmul_f16_split_parts(jlib, oracle, shape):
    """f16 split-K over few rows (S workgroups per tile, one per K part of whole 64-column stages; the last
    to finish adds the parts in part order and runs the epilogue): every S the shape allows, forced, within
    f32 summation-order rounding of the oracle; three launches in a row, then a new call, give the same bits
    (the arrival counters come back to zero and the sum does not depend on the arrival order); 197 rows
    (one ViT-S/16 image: ragged against the 64-row tiles)."""
    n_out, n_in = shape
    M = 197
    rng = np.random.default_rng(n_out + 3 * n_in)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.02).astype(np.float32)
    raw = gguf.quantize(gguf.GGML_F16, w)
    want = oracle.mul_mat(gguf.GGML_F16, raw, n_out, n_in, x, bias)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    L = jlib.lib()
    scale = np.abs(want).max()
    ran = []
    for S in (1, 2, 3, 4):
        if (n_in // 64) % S or n_in // 64 // S < 2:
            continue
        outs = []
        for reps in (3, 1):
            y = torch.full((M, n_out), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            assert L.jepa_amd_gemm_split(S) == 0
            try:
                rc = L.jepa_amd_matmul(0, gguf.GGML_F16, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, y.data_ptr(),
                                       reps, None)
            finally:
                L.jepa_amd_gemm_split(-1)
            assert rc == 0, jlib.error_text()
            outs.append(host(y))
        np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        err = np.abs(outs[0] - want).max()
        assert err <= 2e-5 * scale, (S, err / scale)
        ran.append(S)
    print(f"{shape}: parts {ran} within 2e-5 of the oracle, repeatable")
    assert len(ran) >= 3


# workgroup tiles of the MFMA GEMM (weight rows x tokens), by index
TILES = {0: (256, 128), 1: (192, 128), 2: (128, 128), 3: (128, 128), 4: (64, 128), 5: (128, 64), 6: (256, 64), 7: (256, 64),
         8: (384, 64)}


@pytest.mark.parametrize("tile", sorted(TILES))
@pytest.mark.parametrize("gtype", [gguf.GGML_Q8_0, gguf.GGML_Q4_0, gguf.GGML_Q4_K, gguf.GGML_F16])
def test_matmul_every_tile(jlib, oracle, gtype, tile):
    """Every workgroup tile shape of the MFMA GEMM, forced, on a ragged token count (M = 389: partial
    last tile, rows past M clamped) and K = 768 (6 or 12 stages, so the pipeline's prologue, steady
    state and tail all run; three q4_K super-blocks). The 4-bit layouts need tiles whose weight rows
    pair up in whole copies: q4_0 runs every tile but 1 and 4 (and alone tile 8, whose three LDS
    stages fit only with 4-bit weights), q4_K tiles 2, 3, 5 and 6 (four accumulator sets must fit);
    forcing another tile leaves a launch on the automatic choice.
    Block-quantized types bit-exact, f16 within f32 rounding."""
    bn = TILES[tile][0]
    n_out, n_in, M = bn * (3 if bn == 128 else 2) if bn != 64 else 256, 768, 389
    rng = np.random.default_rng(tile * 100 + gtype)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    bias = (rng.standard_normal(n_out) * 0.02).astype(np.float32)
    if gtype == gguf.GGML_F16:
        raw = w.astype(np.float16).view(np.uint8)
    else:
        raw = gguf.quantize(gtype, w)
    want = _mul_mat_as_gpu(jlib, oracle, gtype, raw, n_out, n_in, x, bias)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    y = torch.zeros((M, n_out), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    L = jlib.lib()
    assert L.jepa_amd_gemm_tile(tile) == 0
    try:
        rc = L.jepa_amd_matmul(0, gtype, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, y.data_ptr(), 1, None)
    finally:
        L.jepa_amd_gemm_tile(-1)
    assert rc == 0, jlib.error_text()
    got = host(y)
    if gtype != gguf.GGML_F16:
        diff = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
        assert diff.size == 0, f"{len(diff)} outputs differ, first {diff[:4].tolist()}, max abs {np.abs(got - want).max():.3e}"
    else:
        assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()


@pytest.mark.parametrize("n_in,tile", [(704, -1), (704, 1), (768, 0), (768, 5), (768, 8), (1152, -1)])
def test_matmul_q4_0_layouts(jlib, oracle, n_in, tile):
    """q4_0 rows that are a multiple of 128 stay 4-bit on the device (codes 16 (q - 8) unpacked in
    registers, the 1.5 * 2^19 float offset on the integer sums); other multiples of 64 are expanded to
    int8 codes at load. Both bit-exact with the oracle, on a ragged M, with weights that use the whole
    4-bit range (codes 0 and 15 in every block) and a block of all-equal values."""
    n_out, M = 768, 389
    rng = np.random.default_rng(n_in + tile)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    w[:, 0::32] = 0.08; w[:, 1::32] = -0.08             # both extremes of every block
    w[7, 64:96] = 0.01                                  # one constant block
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    x[3] = 0.0
    bias = (rng.standard_normal(n_out) * 0.02).astype(np.float32)
    raw = gguf.quantize(gguf.GGML_Q4_0, w)
    codes = raw.reshape(n_out, n_in // 32, 18)[:, :, 2:]
    q = np.concatenate([(codes & 0xF).ravel(), (codes >> 4).ravel()])
    assert q.min() == 0 and q.max() == 15
    want = _mul_mat_as_gpu(jlib, oracle, gguf.GGML_Q4_0, raw, n_out, n_in, x, bias)
    dw, dx, db = dev(raw.reshape(-1)), dev(x), dev(bias)
    y = torch.zeros((M, n_out), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    L = jlib.lib()
    assert L.jepa_amd_gemm_tile(tile) == 0
    try:
        rc = L.jepa_amd_matmul(0, gguf.GGML_Q4_0, dw.data_ptr(), n_out, n_in, db.data_ptr(), dx.data_ptr(), M, y.data_ptr(), 2, None)
    finally:
        L.jepa_amd_gemm_tile(-1)
    assert rc == 0, jlib.error_text()
    got = host(y)
    diff = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert diff.size == 0, f"{len(diff)} outputs differ, first {diff[:4].tolist()}, max abs {np.abs(got - want).max():.3e}"


def test_gemm_tile_hook_rejects_unknown(jlib):
    assert jlib.lib().jepa_amd_gemm_tile(len(TILES)) == -1
    assert jlib.lib().jepa_amd_gemm_tile(-1) == 0


def _attention_ref(qkv, n_items, n_tok, H, rope=None, mask=None, hd=64):
    """double-precision softmax(q k^T / sqrt(hd) + mask) v per head, K/V rounded to f16 like ggml_cast"""
    D = H * hd
    out = np.zeros((n_items * n_tok, D))
    for it in range(n_items):
        blk = qkv[it * n_tok:(it + 1) * n_tok].astype(np.float64)
        for h in range(H):
            q = blk[:, h * hd:(h + 1) * hd]
            k = blk[:, D + h * hd:D + (h + 1) * hd]
            v = blk[:, 2 * D + h * hd:2 * D + (h + 1) * hd]
            if rope is not None:
                c, s = rope
                q = q * c + q[:, np.arange(hd) ^ 1] * s
                k = k * c + k[:, np.arange(hd) ^ 1] * s
            k = k.astype(np.float16).astype(np.float64)
            v = v.astype(np.float16).astype(np.float64)
            sc = q @ k.T / np.sqrt(hd)
            if mask is not None:
                sc = sc + mask
            sc -= sc.max(1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(1, keepdims=True)
            out[it * n_tok:(it + 1) * n_tok, h * hd:(h + 1) * hd] = p @ v
    return out


# token counts cover the three key-split counts (one split up to 1024 keys, four up to 4096, two above),
# 64-key tile counts that the splits of a workgroup share equally or not, one tile (three of four splits
# empty), a last tile with a single valid key, padding
ATTN_CASES = [(1, 2048, 4, True), (2, 197, 6, False), (1, 576, 2, True), (3, 17, 2, False), (1, 129, 1, False),
              (1, 64, 1, False), (2, 65, 2, True), (1, 1088, 2, False), (1, 4160, 1, True)]


@pytest.mark.parametrize("n_items,n_tok,H,rope", ATTN_CASES)
def test_attention(jlib, oracle, n_items, n_tok, H, rope):
    rng = np.random.default_rng(n_tok + H)
    D = H * 64
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    rc = rs = None
    if rope:
        g = int(round(n_tok ** 0.5))
        grid = (n_tok // (g * g), g, g) if n_tok % (g * g) == 0 else (1, 1, n_tok)
        c, s = oracle.rope_tables(grid, 64, variant=0)
        rc, rs = dev(c), dev(s)
    out = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    dq = dev(qkv)
    r = jlib.lib().jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 64, rc.data_ptr() if rope else None,
                                      rs.data_ptr() if rope else None, 0, 0, 0, out.data_ptr())
    assert r == 0, jlib.error_text()
    got = host(out).astype(np.float64)
    ref = _attention_ref(qkv, n_items, n_tok, H, (c.astype(np.float64), s.astype(np.float64)) if rope else None)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    cos = (got * ref).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    assert rel <= 1e-2, rel
    assert cos.min() >= 0.9999, cos.min()


@pytest.mark.parametrize("hd,n_tok,order", [(64, 2048, "rising"), (64, 1000, "falling"), (80, 300, "rising"), (64, 333, "spikes")])
def test_attention_running_maximum_moves(jlib, oracle, hd, n_tok, order):
    """Scores spread over a wide range in key order, so the running maximum (kept in the exp2 domain and
    moved only when a block exceeds it by 2^8) moves many times per sweep: key norms rising along the
    sequence (a move in most blocks), falling (set by the first block, never moved), or a few isolated
    keys far above the rest (moves in single blocks, some key splits never see one). Both kernels (head
    width 64 and the generic width 80) against the float64 softmax."""
    rng = np.random.default_rng(n_tok + hd)
    H = 2
    D = H * hd
    qkv = rng.standard_normal((n_tok, 3 * D)).astype(np.float32)
    j = np.arange(n_tok, dtype=np.float32)[:, None]
    if order == "rising":
        gain = 0.05 + 6.0 * j / n_tok
    elif order == "falling":
        gain = 6.05 - 6.0 * j / n_tok
    else:
        gain = np.full_like(j, 0.3)
        gain[rng.choice(n_tok, 5, replace=False)] = 8.0
    qkv[:, D:2 * D] *= gain                                   # the keys
    qkv[:, :D] *= 2.0                                        # the queries
    out = torch.zeros((n_tok, D), dtype=torch.float32, device="cuda")
    dq = dev(qkv)
    r = jlib.lib().jepa_amd_attention(0, dq.data_ptr(), 1, n_tok, H, hd, None, None, 0, 0, 0, out.data_ptr())
    assert r == 0, jlib.error_text()
    got = host(out).astype(np.float64)
    ref = _attention_ref(qkv, 1, n_tok, H, hd=hd)
    assert np.isfinite(got).all()
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    cos = (got * ref).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    assert rel <= 1e-2, rel
    assert cos.min() >= 0.9999, cos.min()


# head width 32 (the masked predictor's 12 x 32 heads): stored 64 wide with a zero upper half
@pytest.mark.parametrize("n_items,n_tok,H,rope", [(1, 300, 12, True), (2, 65, 3, False), (1, 2048, 2, True)])
def test_attention_hd32(jlib, oracle, n_items, n_tok, H, rope):
    rng = np.random.default_rng(n_tok + 5 * H)
    D = H * 32
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    rc = rs = None
    if rope:
        ids = rng.integers(0, 8 * 16 * 16, n_tok).astype(np.int32)
        c, s = oracle.rope_tables((8, 16, 16), 32, variant=0, ids=ids)
        rc, rs = dev(c), dev(s)
    out = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    oq = torch.zeros((n_items * n_tok, D // 32 * 34), dtype=torch.uint8, device="cuda")
    dq = dev(qkv)
    L = jlib.lib()
    for ot, buf in ((0, out), (gguf.GGML_Q8_0, oq)):
        r = L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 32, rc.data_ptr() if rope else None,
                                 rs.data_ptr() if rope else None, 0, 0, ot, buf.data_ptr())
        assert r == 0, jlib.error_text()
    got = host(out).astype(np.float64)
    ref = _attention_ref(qkv, n_items, n_tok, H, (c.astype(np.float64), s.astype(np.float64)) if rope else None, hd=32)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    cos = (got * ref).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    assert rel <= 1e-2, rel
    assert cos.min() >= 0.9999, cos.min()
    want = oracle.quantize_act(oracle.OR_Q8_0, host(out))
    np.testing.assert_array_equal(host(oq), want.reshape(host(oq).shape))


# other head widths (multiples of 16 up to 128, stored rounded up to 32 with zero padding): 80 is I-JEPA
# ViT-H/14's (16 heads of 80, 256 tokens, RoPE from the reference's hd-80 table layout); 48 and 128 bound
# the range. Against the double softmax; the q8_0 output is refused (its 32-dim blocks would span heads).
@pytest.mark.parametrize("n_items,n_tok,H,hd,rope", [(1, 256, 16, 80, False), (2, 197, 3, 80, True), (1, 130, 2, 48, False),
                                                     (1, 300, 2, 128, True), (1, 33, 1, 80, False)])
def test_attention_other_widths(jlib, oracle, n_items, n_tok, H, hd, rope):
    rng = np.random.default_rng(n_tok + 7 * H + hd)
    D = H * hd
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    rc = rs = None
    if rope:
        c, s = oracle.rope_tables((1, 1, n_tok), hd, variant=0)
        rc, rs = dev(c), dev(s)
    out = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    dq = dev(qkv)
    L = jlib.lib()
    r = L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, hd, rc.data_ptr() if rope else None,
                             rs.data_ptr() if rope else None, 0, 0, 0, out.data_ptr())
    assert r == 0, jlib.error_text()
    got = host(out).astype(np.float64)
    ref = _attention_ref(qkv, n_items, n_tok, H, (c.astype(np.float64), s.astype(np.float64)) if rope else None, hd=hd)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    cos = (got * ref).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    assert rel <= 1e-2, rel
    assert cos.min() >= 0.9999, cos.min()
    oq = torch.zeros((n_items * n_tok, D // 32 * 34 + 34), dtype=torch.uint8, device="cuda")
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, hd, None, None, 0, 0, gguf.GGML_Q8_0, oq.data_ptr()) == -1
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 72, None, None, 0, 0, 0, out.data_ptr()) == -1


# block-causal (LeVJEPA) shapes (n_items, gt, gh, gw, n_prefix, H): the reference's mask KAT shape (65
# rows), 513 rows (five query blocks; slots of 64 rows against tiles of 64 keys shifted by the CLS),
# slots of 35 rows with no prefix, the 16 x 224^2 clip (3137 rows, slots of 196), and 4097 rows (two key
# splits)
MASK_CASES = [(1, 4, 4, 4, 1, 2), (2, 8, 8, 8, 1, 2), (1, 3, 5, 7, 0, 2), (1, 16, 14, 14, 1, 1), (1, 16, 16, 16, 1, 1)]


@pytest.mark.parametrize("n_items,gt,gh,gw,n_prefix,H", MASK_CASES)
def test_attention_block_causal(jlib, oracle, n_items, gt, gh, gw, n_prefix, H):
    """The kernel's block-causal mask (per-query key ranges, skipped tiles and blocks) against a double
    softmax over the oracle's [N][N] mask, and the q8_0 epilogue against the separate quantizer."""
    n_tok = n_prefix + gt * gh * gw
    rng = np.random.default_rng(n_tok * 7 + H)
    D = H * 64
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    mask = oracle.block_causal_mask(gt, gh, gw, n_prefix).astype(np.float64)
    dq = dev(qkv)
    out = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    oq = torch.zeros((n_items * n_tok, D // 32 * 34), dtype=torch.uint8, device="cuda")
    L = jlib.lib()
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 64, None, None, n_prefix, gh * gw, 0, out.data_ptr()) == 0, \
        jlib.error_text()
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 64, None, None, n_prefix, gh * gw, gguf.GGML_Q8_0,
                                oq.data_ptr()) == 0
    got = host(out).astype(np.float64)
    ref = _attention_ref(qkv, n_items, n_tok, H, None, mask)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    cos = (got * ref).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    assert rel <= 1e-2, rel
    assert cos.min() >= 0.9999, cos.min()
    want = oracle.quantize_act(oracle.OR_Q8_0, host(out))
    np.testing.assert_array_equal(host(oq), want.reshape(host(oq).shape))


@pytest.mark.parametrize("n_items,n_tok,H", [(1, 2048, 4), (2, 197, 6), (1, 65, 2)])
def test_attention_fused_q8_0_equals_separate_quantizer(jlib, oracle, n_items, n_tok, H):
    """The attention epilogue's q8_0 output is byte-identical to quantizing the f32 attention output
    with the activation quantizer (what the out-projection would otherwise get)."""
    rng = np.random.default_rng(n_tok * 3 + H)
    D = H * 64
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    dq = dev(qkv)
    o32 = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    oq = torch.zeros((n_items * n_tok, D // 32 * 34), dtype=torch.uint8, device="cuda")
    L = jlib.lib()
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 64, None, None, 0, 0, 0, o32.data_ptr()) == 0
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, 64, None, None, 0, 0, gguf.GGML_Q8_0, oq.data_ptr()) == 0
    want = oracle.quantize_act(oracle.OR_Q8_0, host(o32))
    np.testing.assert_array_equal(host(oq), want.reshape(host(oq).shape))


@pytest.mark.parametrize("n_items,n_tok,H,hd", [(1, 197, 6, 64), (2, 256, 4, 64), (1, 65, 2, 32)])
def test_attention_f16_output_equals_rounded_f32(jlib, n_items, n_tok, H, hd):
    """The attention epilogue's f16 output (the input of an f16 out-projection) is the f32 output
    rounded to nearest, what the separate conversion would give."""
    rng = np.random.default_rng(n_tok * 5 + H)
    D = H * hd
    qkv = (rng.standard_normal((n_items * n_tok, 3 * D)) * 1.5).astype(np.float32)
    dq = dev(qkv)
    o32 = torch.zeros((n_items * n_tok, D), dtype=torch.float32, device="cuda")
    o16 = torch.zeros((n_items * n_tok, D), dtype=torch.float16, device="cuda")
    L = jlib.lib()
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, hd, None, None, 0, 0, 0, o32.data_ptr()) == 0
    assert L.jepa_amd_attention(0, dq.data_ptr(), n_items, n_tok, H, hd, None, None, 0, 0, gguf.GGML_F16, o16.data_ptr()) == 0
    want = host(o32).astype(np.float16)
    np.testing.assert_array_equal(host(o16).view(np.uint16), want.view(np.uint16))


def test_gemm_step_probe(jlib):
    """The register-only step probe (the q8_0 GEMM's ceiling measurement) runs for every mode and
    occupancy; each half alone is faster than the whole step, and bad arguments are refused."""
    L = jlib.lib()
    res = {}
    for wps in (2, 4):
        for mode in range(4):
            ns = C.c_double(0)
            assert L.jepa_amd_gemm_step_probe(0, mode, wps, 2000, C.byref(ns)) == 0, jlib.error_text()
            assert 1.0 < ns.value < 10000.0, (mode, wps, ns.value)
            res[mode, wps] = ns.value
        assert res[1, wps] < res[0, wps] and res[2, wps] < res[0, wps], res
    ns = C.c_double(0)
    assert L.jepa_amd_gemm_step_probe(0, 4, 2, 10, C.byref(ns)) == -1
    assert L.jepa_amd_gemm_step_probe(0, 0, 5, 10, C.byref(ns)) == -1


# ------------------------------------------------------------------------------------------------ ingest
def _pre_params(jlib, resize_short=224, crop=224, resample=0, mode=0, fused=True):
    p = jlib.PreprocessParams()
    for c, (m, sd) in enumerate(zip((0.485, 0.456, 0.406), (0.229, 0.224, 0.225))):
        p.mean[c], p.std[c] = m, sd
    p.resize_short, p.crop, p.resample, p.resize_mode, p.rescale, p.fused_norm = resize_short, crop, resample, mode, 1.0 / 255.0, fused
    return p


@pytest.mark.parametrize("hw,kw", [((300, 400), {}), ((400, 300), dict(resample=1)), ((256, 256), dict(resize_short=256, crop=256)),
                                   ((180, 320), dict(mode=1, resize_short=224)), ((200, 260), dict(crop=320, fused=False)),
                                   ((1080, 1920), dict(resample=1))])
def test_preprocess_device_equals_host(jlib, hw, kw):
    """jepa_amd_preprocess_frames_device (uint8 frames on the device -> NCTHW floats) equals the host
    jepa_preprocess_frames_rgb_ex bit for bit: down / up / identity resizes, bicubic, squash, a crop
    larger than the image (zero padding), the unfused normalisation, a 1080p frame."""
    rng = np.random.default_rng(hw[0] + hw[1])
    T = 3
    frames = rng.integers(0, 256, (T, hw[0], hw[1], 3), dtype=np.uint8)
    p = _pre_params(jlib, **kw)
    want = jlib.preprocess_frames(p, list(frames))
    d = torch.from_numpy(frames).cuda()
    out = torch.zeros(want.size, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    oh, ow = C.c_int(0), C.c_int(0)
    rc = jlib.lib().jepa_amd_preprocess_frames_device(0, C.byref(p), d.data_ptr(), T, hw[0], hw[1], out.data_ptr(), out.numel(),
                                                     C.byref(oh), C.byref(ow))
    assert rc == 0, jlib.error_text()
    assert (oh.value, ow.value) == want.shape[2:]
    got = host(out).reshape(want.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{int((got != want).sum())} values differ"
