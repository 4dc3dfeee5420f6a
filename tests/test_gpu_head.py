"""Attentive-pool head on the GPU (through the C ABI: jepa_head_ex / jepa_amd_head_device) against the
oracle's head (reference src/jepa.cpp:1026-1112) on the same synthetic GGUF and the same encoder rows.

Gates: pooled token and logits within max relative error 1e-2 of the oracle's (relative to the largest
magnitude) and pooled cosine >= 0.9999. The classifier's 10 / 174 outputs are not a multiple of the
GEMM's 128-row tiles: the loader pads the matrix with zero rows, and only the file's rows come back.
"""
import numpy as np
import pytest

from jepa_amd import forge, inputs

pytestmark = pytest.mark.gpu


def rel_max(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def cos(a, b):
    a = a.astype(np.float64); b = b.astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def check(got_p, got_l, want_p, want_l, label):
    rp, rl, c = rel_max(got_p, want_p), rel_max(got_l, want_l), cos(got_p, want_p)
    print(f"{label}: pooled rel {rp:.3e} cos {c:.8f}, logits rel {rl:.3e}, argmax {int(np.argmax(got_l))} / {int(np.argmax(want_l))}")
    assert got_l.shape == want_l.shape
    assert rp <= 1e-2 and rl <= 1e-2 and c >= 0.9999, (rp, rl, c)


def _tiny(ftype, **kw):
    big = ftype == "q4_k"     # q4_K needs rows that are a multiple of 256
    return forge.tiny("vjepa2", ftype, ln_random=True, n_classes=10, n_pool_layers=2, embed_dim=256 if big else 128,
                      ffn_dim=1024 if big else 512, n_head=4 if big else 2, **kw)


@pytest.mark.parametrize("ftype,n_tok", [("q8_0", 40), ("q8_0", 300), ("q4_0", 513), ("f16", 257), ("q4_k", 300), ("f32", 64),
                                         ("q8_0", 2500)])
def test_tiny_head_parity(jlib, oracle, models_dir, ftype, n_tok):
    """Head alone on the same rows, every weight format: the pool attention's 64-key chunks from 1 to 40
    (the merge pass takes eight chunks per wave at a time, then the rest one by one: 2500 rows give 40
    chunks, the last one of 4 keys, so a wave runs both loops)."""
    cfg = _tiny(ftype)
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    rows = np.random.default_rng(n_tok).standard_normal((n_tok, cfg.embed_dim)).astype(np.float32)
    got_p, got_l = ctx.head(rows)
    want_p, want_l = oracle.head(path, rows, cfg.n_classes)
    check(got_p, got_l, want_p, want_l, f"tiny {ftype} N={n_tok}")


def test_tiny_classifier_pipeline(jlib, oracle, models_dir):
    """jepa_encode -> jepa_head (what jepa-classify does) against oracle encode -> oracle head."""
    cfg = _tiny("q8_0")
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    x = inputs.make_input(1, 4, 64, 64, seed=77)
    enc = ctx.encode(x)
    want_enc, _ = oracle.encode(path, x, 1, enc.shape[0], cfg.embed_dim, n_layers=cfg.n_layer)
    got_p, got_l = ctx.head(enc)
    want_p, want_l = oracle.head(path, want_enc, cfg.n_classes)
    check(got_p, got_l, want_p, want_l, "tiny pipeline")


def test_head_outputs_optional_and_repeatable(jlib, models_dir):
    """pooled / logits may each be NULL; repeated calls and the device entry point give the same bits."""
    import torch
    cfg = _tiny("q8_0")
    m = jlib.Model(forge.cached_model(cfg, models_dir))
    ctx = jlib.Context(m)
    rows = np.random.default_rng(3).standard_normal((100, cfg.embed_dim)).astype(np.float32)
    p, l = ctx.head(rows)
    p2, none = ctx.head(rows, logits=False)
    none2, l2 = ctx.head(rows, pooled=False)
    assert none is None and none2 is None
    np.testing.assert_array_equal(p.view(np.uint32), p2.view(np.uint32))
    np.testing.assert_array_equal(l.view(np.uint32), l2.view(np.uint32))
    x = torch.from_numpy(rows).cuda()
    pd = torch.zeros(cfg.embed_dim, device="cuda")
    ld = torch.zeros(cfg.n_classes, device="cuda")
    torch.cuda.synchronize()
    assert ctx.head_device(x.data_ptr(), rows.shape[0], pd.data_ptr(), ld.data_ptr()) == cfg.n_classes
    np.testing.assert_array_equal(pd.cpu().numpy().view(np.uint32), p.view(np.uint32))
    np.testing.assert_array_equal(ld.cpu().numpy().view(np.uint32), l.view(np.uint32))
    # a different token count rebuilds the buffers; the first count still gives the same bits after it
    ctx.head(rows[:37])
    p3, l3 = ctx.head(rows)
    np.testing.assert_array_equal(l3.view(np.uint32), l.view(np.uint32))


def test_head_errors(jlib, models_dir):
    cfg = _tiny("q8_0")
    m = jlib.Model(forge.cached_model(cfg, models_dir))
    ctx = jlib.Context(m)
    assert m.has_head and m.n_classes == 10 and m.label(3) == "class 3"
    with pytest.raises(RuntimeError, match="rows are 64 wide, expected 128"):
        ctx.head(np.zeros((10, 64), np.float32))
    plain = jlib.Model(forge.cached_model(forge.tiny("vjepa2", "q8_0"), models_dir))
    with pytest.raises(RuntimeError, match="has no attentive-pool head"):
        jlib.Context(plain).head(np.zeros((10, 128), np.float32))


def test_vitl16_ssv2_head_q8_0(jlib, oracle, models_dir):
    """V-JEPA 2 ViT-L SSv2 classifier head at its real shape: 3 pooler blocks over 2048 tokens of width
    1024, 16 heads, 174 classes (padded to 256 rows on the device)."""
    cfg = forge.CONFIGS["vitl16_ssv2_q8_0"]
    path = forge.cached_model(cfg, models_dir)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    rows = np.random.default_rng(11).standard_normal((2048, 1024)).astype(np.float32)
    got_p, got_l = ctx.head(rows)
    print(f"vitl16 ssv2 head: {ctx.last_compute_ms:.3f} ms")
    want_p, want_l = oracle.head(path, rows, cfg.n_classes)
    check(got_p, got_l, want_p, want_l, "vitl16 ssv2 head")
