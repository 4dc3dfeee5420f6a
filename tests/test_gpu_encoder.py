"""Encoder forward on the GPU (through the C ABI: jepa_model_load_ex / jepa_encode) against the CPU
oracle's ggml-semantics restatement on the same synthetic GGUF and the same seeded inputs.

Gates (north star): per-token cosine >= 0.9999 (mean; the minimum is reported and held to a looser
bar, since a low-variance token amplifies one activation-rounding flip - docs/quantization.md "Reading
the numbers"), and max relative error <= 1e-2 per layer on the residual stream.
"""
import numpy as np
import pytest

from jepa_amd import forge, inputs

pytestmark = pytest.mark.gpu


def cos_rows(a, b):
    a = a.astype(np.float64); b = b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-300)


def rel_max(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def _case(jlib, oracle, models_dir, cfg, n_batch, n_frames, size, trace=True):
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    x = inputs.make_input(n_batch, n_frames, size, size, seed=1234)
    video = cfg.family in ("vjepa2", "vjepa2_1")
    rows = m.token_grid(n_frames if video else 1, size, size)
    n_items = n_batch if video else n_batch * n_frames
    if trace:
        got, gtr = ctx.encode_trace(x, n_items, rows)
    else:
        got, gtr = ctx.encode(x), None
    want, wtr = oracle.encode(path, x, n_items, rows, m.dim, n_layers=m.n_layer, trace=trace)
    return got, want, gtr, wtr, m, ctx, x


TINY = [("hfvit", "f16", 2, 1, 64), ("hfvit", "q8_0", 1, 2, 64), ("vjepa2", "q8_0", 1, 4, 64), ("vjepa2", "q4_k", 1, 4, 64),
        ("vjepa2", "q4_0", 2, 4, 64), ("vjepa2", "f16", 1, 4, 64), ("vjepa2_1", "q8_0", 2, 1, 64), ("vjepa2_1", "q8_0", 1, 4, 64)]


@pytest.mark.parametrize("family,ftype,n_batch,n_frames,size", TINY)
def test_tiny_encoder_parity(jlib, oracle, models_dir, family, ftype, n_batch, n_frames, size):
    cfg = forge.tiny(family, ftype, ln_random=True, layer_scale=(ftype == "q4_0"),
                     ffn_dim=1024 if ftype == "q4_k" else 512, embed_dim=256 if ftype == "q4_k" else 128,
                     n_head=4 if ftype == "q4_k" else 2)
    got, want, gtr, wtr, m, ctx, x = _case(jlib, oracle, models_dir, cfg, n_batch, n_frames, size)
    c = cos_rows(got, want)
    assert c.mean() >= 0.9999, (c.mean(), c.min())
    assert c.min() >= 0.999, c.min()
    for l in range(gtr.shape[1]):
        r = rel_max(gtr[:, l], wtr[:, l])
        assert r <= 1e-2, f"layer {l}: rel_max {r:.3e}"


def test_batch_equals_single(jlib, models_dir):
    """Items of one call equal separate calls bit for bit (reference tests/test-batch.cpp:12-21)."""
    for family, nb, nf in (("hfvit", 3, 1), ("vjepa2", 2, 4)):
        cfg = forge.tiny(family, "q8_0")
        m = jlib.Model(forge.cached_model(cfg, models_dir))
        ctx = jlib.Context(m)
        x = inputs.make_input(nb, nf, 64, 64, seed=5)
        both = ctx.encode(x)
        parts = np.concatenate([ctx.encode(x[i:i + 1]) for i in range(nb)])
        np.testing.assert_array_equal(both.view(np.uint32), parts.view(np.uint32))


def test_graph_replay_equals_direct(jlib, models_dir):
    cfg = forge.tiny("vjepa2", "q8_0")
    m = jlib.Model(forge.cached_model(cfg, models_dir))
    ctx = jlib.Context(m)
    x = inputs.make_input(1, 4, 64, 64, seed=9)
    first = ctx.encode(x)
    again = [ctx.encode(x) for _ in range(3)]        # graph replays
    ctx.set_graph(False)
    direct = ctx.encode(x)
    for a in again + [direct]:
        np.testing.assert_array_equal(a.view(np.uint32), first.view(np.uint32))


def test_vits16_f16_full(jlib, oracle, models_dir):
    """LeJEPA ViT-S/16 224x224 f16 (hfvit, CLS + learned positions), batch 1, CLS-pooled."""
    got, want, gtr, wtr, m, ctx, x = _case(jlib, oracle, models_dir, forge.CONFIGS["vits16_f16"], 1, 1, 224)
    c = cos_rows(got, want)
    assert got.shape == (197, 384)
    assert c.mean() >= 0.9999 and c.min() >= 0.999, (c.mean(), c.min())
    for l in range(gtr.shape[1]):
        assert rel_max(gtr[:, l], wtr[:, l]) <= 1e-2


def test_vitb16_2_1_image_q8_0(jlib, oracle, models_dir):
    """V-JEPA 2.1 ViT-B/16 384x384 image path (576 tokens), two images in one call."""
    got, want, gtr, wtr, m, ctx, x = _case(jlib, oracle, models_dir, forge.CONFIGS["vitb16_2_1_q8_0"], 2, 1, 384)
    assert got.shape == (2 * 576, 768)
    c = cos_rows(got, want)
    assert c.mean() >= 0.9999 and c.min() >= 0.999, (c.mean(), c.min())
    for l in range(gtr.shape[1]):
        assert rel_max(gtr[:, l], wtr[:, l]) <= 1e-2


@pytest.mark.parametrize("name", ["vitl16_q8_0", "vitl16_q4_k"])
def test_vitl16_16f_full(jlib, oracle, models_dir, name):
    """V-JEPA 2 ViT-L/16, 16 frames 256x256 = 2048 tokens, 24 layers: the benchmark configuration."""
    got, want, gtr, wtr, m, ctx, x = _case(jlib, oracle, models_dir, forge.CONFIGS[name], 1, 16, 256)
    assert got.shape == (2048, 1024)
    c = cos_rows(got, want)
    print(f"{name}: token cosine mean {c.mean():.7f} min {c.min():.6f}")
    assert c.mean() >= 0.9999, (c.mean(), c.min())
    for l in range(gtr.shape[1]):
        r = rel_max(gtr[:, l], wtr[:, l])
        assert r <= 1e-2, f"layer {l}: rel_max {r:.3e}"


def test_encode_errors(jlib, models_dir):
    cfg = forge.tiny("vjepa2", "q8_0")
    m = jlib.Model(forge.cached_model(cfg, models_dir))
    ctx = jlib.Context(m)
    for shape in [(1, 3, 3, 64, 64), (1, 3, 4, 60, 64), (1, 2, 4, 64, 64)]:   # odd frames / not /16 / channels
        with pytest.raises(RuntimeError):
            ctx.encode(np.zeros(shape, np.float32))
