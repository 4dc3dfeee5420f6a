"""Full-size encoders on the GPU (through the C ABI) against the CPU oracle, on the benchmark
configurations: V-JEPA 2 ViT-L/16 16f q8_0 and q4_K, V-JEPA 2.1 ViT-B/16 384^2 at batch 8, LeVJEPA
ViT-L/16 16f 224^2 (block-causal, 3137 rows), I-JEPA ViT-H/14 224^2 q8_0 (32 layers, heads of 80); plus the
pooled outputs of C1 (CLS) and C3 (mean).

Three views of the same forward:

1. End to end, against the oracle with the reference's CPU arithmetic: token cosine >= 0.9999 (the
   fixed bar). Quantized activations amplify last-bit differences over 12-32 layers (an int8 / q8_K
   code flips when its input crosses a rounding boundary), so two equally valid summation orders of
   the oracle itself already differ by about 1e-4 in cosine on these models; where that puts the bar
   out of reach the case is marked as a known failure with the measured numbers, not relaxed.
2. Per layer, teacher-forced: the oracle's block l is fed the GPU's own input of block l (its
   residual-stream trace), so each block's error is measured without what earlier blocks passed on.
   Max relative error <= 1e-2 on every block (the per-layer bar), and on the patch embedding.
3. Per layer, teacher-forced against the oracle with the GPU kernels' roundings switched on (f16 q
   and softmax weights, the exp2 softmax form, the erf polynomial; oracle.ROUND_GPU): what remains is
   summation order inside the MFMAs and the hardware exp2, so the gate is tight (cosine >= 0.99999).
"""
import numpy as np
import pytest

from jepa_amd import forge, inputs

pytestmark = pytest.mark.gpu

# (config, n_batch, n_frames, size, rows per item)
FULL = {
    "vitl16_q8_0": (1, 16, 256, 2048),
    "vitl16_q4_k": (1, 16, 256, 2048),
    "vitb16_2_1_q8_0": (8, 1, 384, 576),
    "levjepa_vitl16_q8_0": (1, 16, 224, 3137),
    "vith14_ijepa_q8_0": (1, 1, 224, 256),
}

# End-to-end cosine below the fixed bar: (floor, why). The floor sits just under the measured cosine, so a
# regression still fails; the reason quotes the oracle against itself in ggml's own x86 summation order
# (AVX2 vec_dot / llamafile tiles, oracle.set_ggml_lanes) and in reversed block order, measured on the CPU
# (tests/parity_attribution.py): two valid orders of the reference arithmetic already differ by that much.
KNOWN_E2E = {
    "vitl16_q4_k": (0.9997, "q8_K activations over 24 layers: the oracle in ggml's x86 lane order against the oracle's "
                            "one-chain order reaches only cosine 0.99983 (reversed block order 0.99983), below 0.9999"),
    "levjepa_vitl16_q8_0": (0.99985, "3137 rows x 24 layers of q8_0 activations: the oracle in ggml's x86 lane order "
                                     "against its one-chain order reaches cosine 0.99990 (reversed block order 0.99990), "
                                     "at the bar"),
    "vith14_ijepa_q8_0": (0.99980, "32 layers of q8_0 activations: the oracle in ggml's x86 lane order against its "
                                   "one-chain order reaches cosine 0.99988 (reversed block order 0.99988), below 0.9999"),
}

_cache = {}


def cos_rows(a, b):
    a = a.astype(np.float64); b = b.astype(np.float64)
    return (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1) + 1e-300)


def rel_max(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def _run(jlib, oracle, models_dir, name):
    if name in _cache:
        return _cache[name]
    n_batch, n_frames, size, rows = FULL[name]
    cfg = forge.CONFIGS[name]
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    x = inputs.make_input(n_batch, n_frames, size, size, seed=1234)
    video = cfg.family in ("vjepa2", "vjepa2_1", "levjepa")
    n_items = n_batch if (video and n_frames > 1) else n_batch * n_frames
    assert m.token_grid(n_frames if video else 1, size, size) == rows
    got, gtr = ctx.encode_trace(x, n_items, rows)
    print(f"{name}: GPU done", flush=True)
    prev = oracle.get_rounding()
    want_lanes = None
    try:
        oracle.set_rounding(0)
        want, wtr = oracle.encode(path, x, n_items, rows, m.dim, n_layers=m.n_layer, trace=True)
        _, ttr = oracle.encode_teacher(path, x, n_items, rows, m.dim, gtr)
        if name in KNOWN_E2E:
            # the same arithmetic with the quantized dots in ggml's own x86 lane order
            oracle.set_ggml_lanes(True)
            try:
                want_lanes, _ = oracle.encode(path, x, n_items, rows, m.dim)
            finally:
                oracle.set_ggml_lanes(False)
        oracle.set_rounding(oracle.ROUND_GPU)
        _, mtr = oracle.encode_teacher(path, x, n_items, rows, m.dim, gtr)
    finally:
        oracle.set_rounding(prev)
    print(f"{name}: oracle done", flush=True)
    r = dict(model=m, got=got, gtr=gtr, want=want, wtr=wtr, ttr=ttr, mtr=mtr, rows=rows, n_items=n_items, want_lanes=want_lanes)
    _cache.clear()          # one full-size model's traces at a time
    _cache[name] = r
    return r


@pytest.mark.parametrize("name", list(FULL))
def test_end_to_end(jlib, oracle, models_dir, name):
    r = _run(jlib, oracle, models_dir, name)
    c = cos_rows(r["got"], r["want"])
    rl = [rel_max(r["gtr"][:, l], r["wtr"][:, l]) for l in range(r["gtr"].shape[1])]
    print(f"{name}: end-to-end token cosine mean {c.mean():.7f} min {c.min():.6f}; residual-stream rel_max "
          f"by layer: first {rl[1]:.2e}, last {rl[-1]:.2e}, max {max(rl):.2e}")
    if r["want_lanes"] is not None:
        cl = cos_rows(r["got"], r["want_lanes"])
        co = cos_rows(r["want"], r["want_lanes"])
        print(f"{name}: against the oracle in ggml's x86 lane order: GPU cosine mean {cl.mean():.7f} min {cl.min():.6f}; "
              f"oracle one-chain order against it {co.mean():.7f}")
        if cl.mean() >= 0.9999:
            return          # within the bar of ggml's own summation order
    if name in KNOWN_E2E:
        floor, why = KNOWN_E2E[name]
        assert c.mean() >= floor, (c.mean(), floor)
        if c.mean() < 0.9999:
            pytest.xfail(f"cosine {c.mean():.6f}: {why}")
    assert c.mean() >= 0.9999, (c.mean(), c.min())


@pytest.mark.parametrize("name", list(FULL))
def test_per_layer_teacher_forced(jlib, oracle, models_dir, name):
    r = _run(jlib, oracle, models_dir, name)
    gtr, ttr, wtr = r["gtr"], r["ttr"], r["wtr"]
    patch = rel_max(gtr[:, 0], wtr[:, 0])
    rl = [rel_max(gtr[:, l], ttr[:, l]) for l in range(1, gtr.shape[1])]
    cl = [cos_rows(gtr[:, l], ttr[:, l]).mean() for l in range(1, gtr.shape[1])]
    print(f"{name}: patch embedding rel {patch:.2e}; per block (teacher-forced) rel_max max {max(rl):.2e} "
          f"(block {int(np.argmax(rl))}), mean {np.mean(rl):.2e}; cosine min {min(cl):.8f}")
    assert patch <= 1e-2
    assert max(rl) <= 1e-2, (max(rl), int(np.argmax(rl)))


@pytest.mark.parametrize("name", list(FULL))
def test_per_layer_rounding_matched(jlib, oracle, models_dir, name):
    r = _run(jlib, oracle, models_dir, name)
    gtr, mtr = r["gtr"], r["mtr"]
    rl = [rel_max(gtr[:, l], mtr[:, l]) for l in range(1, gtr.shape[1])]
    cl = [cos_rows(gtr[:, l], mtr[:, l]).mean() for l in range(1, gtr.shape[1])]
    print(f"{name}: per block vs rounding-matched oracle: rel_max max {max(rl):.2e}, mean {np.mean(rl):.2e}; "
          f"cosine min {min(cl):.9f}")
    assert min(cl) >= 0.99999, (min(cl), int(np.argmin(cl)))


def test_pool_mean_vitb16_batch8(jlib, oracle, models_dir):
    """C3 as configured: 8 images in one call, each mean-pooled (jepa_pool_mean on its 576 rows)."""
    r = _run(jlib, oracle, models_dir, "vitb16_2_1_q8_0")
    m, rows = r["model"], r["rows"]
    got = np.stack([m.pool_mean(r["got"][i * rows:(i + 1) * rows]) for i in range(8)])
    want = r["want"].reshape(8, rows, -1).astype(np.float64).mean(1)
    c = cos_rows(got, want)
    print(f"vitb16 batch 8 mean-pooled: cosine per image min {c.min():.7f}, rel_max {rel_max(got, want):.2e}")
    assert c.min() >= 0.9999
    # the pooling itself: exactly the double-accumulated mean of the GPU's own rows
    own = r["got"].reshape(8, rows, -1).astype(np.float64).mean(1).astype(np.float32)
    assert np.abs(got - own).max() <= 1e-6 * np.abs(own).max()


def test_pool_cls_vits16(jlib, oracle, models_dir):
    """C1 as configured: LeJEPA ViT-S/16 224^2 f16, batch 1, CLS-pooled (jepa_pool_cls)."""
    cfg = forge.CONFIGS["vits16_f16"]
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    x = inputs.make_input(1, 1, 224, 224, seed=1234)
    got = ctx.encode(x)
    want, _ = oracle.encode(path, x, 1, 197, m.dim)
    cls = m.pool_cls(got)
    np.testing.assert_array_equal(cls, got[0])
    c = cos_rows(cls, want[0])
    print(f"vits16 CLS: cosine {c:.8f}, rel {rel_max(cls, want[0]):.2e}")
    assert c >= 0.9999 and rel_max(cls, want[0]) <= 1e-2
    with pytest.raises(RuntimeError):          # the mean of zero patch rows is refused
        m.pool_mean(got[:1])
