"""The reference's own command-line tools, compiled as they lie against include/jepa.h and linked to
libjepa.so (`make -C oracle ref-tools`, which build() runs where the reference tree is present; the
binaries travel in oracle/_ref/), run on the GPU: a caller of the reference switches to this library
with no change to its code. What they print or save is compared with this library's Python binding
of the same entry points (bit for bit: the same library code on the same inputs) and, for the
encoder rows, with the oracle.

- tools/jepa-bench.cpp: --mode encoder (batched), head and predictor, with its --json record.
- tools/jepa-embed.cpp: an image (tests/golden/media) through jepa_load_image_rgb,
  jepa_preprocess_image_rgb, jepa_encode and --pool none / cls; a THWC uint8 clip (--frames-npy)
  through the same route with --pool mean and the attentive-pool head (--logits).
- tools/jepa-classify.cpp: a THWC uint8 clip through its own preprocessing loop, the encoder, the
  head and its top-k listing.
- tests/test-batch.cpp: the reference's own batched-against-single test, with its exit status.
- tests/test-predictor.cpp: the reference's own predictor test in its numpy-case mode, on cases the
  oracle's predictor writes.
"""
import json
import os
import re
import subprocess

import numpy as np
import pytest

from jepa_amd import forge

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_BIN = os.path.join(ROOT, "oracle", "_ref")
IMAGE = os.path.join(ROOT, "tests", "golden", "media", "coco_000000000724.jpg")

pytestmark = pytest.mark.gpu


def _tool(name):
    p = os.path.join(REF_BIN, name)
    if not os.access(p, os.X_OK):
        pytest.skip(f"oracle/_ref/{name} is not built (make -C oracle ref-tools needs the reference tree)")
    return p


def _run(cmd, timeout=300):
    print("run:", " ".join(os.path.basename(c) if os.path.isabs(c) else c for c in cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-3000:])
    return r


def _bench_json(exe, path, tmp_path, *args):
    out = tmp_path / "bench.json"
    _run([exe, "-m", path, *args, "--json", str(out)])
    d = json.loads(out.read_text())
    assert d["tool"] == "jepa-bench" and len(d["runs"]) == 1, d
    return d["runs"][0]


def _cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


def test_jepa_bench_encoder_batched(jlib, models_dir, tmp_path):
    """jepa-bench --mode encoder, two clips per jepa_encode call (its own synthetic input, the
    generator this repository's inputs.make_input is pinned to): the run is on the GPU, and its token
    count and device name are this library's."""
    exe = _tool("jepa-bench")
    path = forge.cached_model(forge.tiny("vjepa2", "q8_0"), models_dir)
    r = _bench_json(exe, path, tmp_path, "--frames", "4", "--size", "64x64", "--batch", "2", "--repeat", "3", "--warmup", "1")
    m = jlib.Model(path)
    assert r["gpu"] is True and r["mode"] == "encoder"
    assert r["device"] == jlib.lib().jepa_device_name(0).decode()
    assert r["tokens"] == 2 * m.token_grid(4, 64, 64) and r["units"] == 2
    assert 0 < r["ms_min"] <= r["ms_mean"] and r["wall_ms_min"] >= r["ms_min"]


@pytest.mark.parametrize("mode", ["head", "predictor"])
def test_jepa_bench_head_and_predictor(models_dir, tmp_path, mode):
    """jepa-bench --mode head / predictor: the attentive-pool head and the masked predictor on one
    item's encoder rows, through jepa_head and jepa_predict."""
    exe = _tool("jepa-bench")
    cfg = forge.tiny("vjepa2", "q8_0", n_classes=10, n_pool_layers=1, pred_dim=128, pred_layers=2, pred_ffn=512)
    path = forge.cached_model(cfg, models_dir)
    r = _bench_json(exe, path, tmp_path, "--mode", mode, "--frames", "4", "--size", "64x64", "--repeat", "3", "--warmup", "1")
    assert r["gpu"] is True and r["mode"] == mode and r["units"] == 1
    assert r["ms_mean"] > 0 and r["encoder_ms"] > 0


def test_jepa_bench_vitl16_16f(jlib, models_dir, tmp_path):
    """The reference's headline row (V-JEPA 2 ViT-L/16, 16 frames of 256x256, q8_0, one clip per call)
    timed by its own tool on this library: jepa_context_last_compute_ms per call (device time of the
    forward, as the tool reports it) and the wall time of jepa_encode (host input and output copies
    included)."""
    exe = _tool("jepa-bench")
    path = forge.cached_model(forge.CONFIGS["vitl16_q8_0"], models_dir)
    r = _bench_json(exe, path, tmp_path, "--repeat", "10", "--warmup", "2")
    print(f"jepa-bench {r['model']} {r['shape']} {r['ftype']} on {r['device']}: {r['ms_mean']:.3f} ms mean "
          f"(min {r['ms_min']:.3f}), wall {r['wall_ms_mean']:.3f} ms, {r['tokens_per_s']:.0f} tokens/s")
    assert r["gpu"] is True and r["tokens"] == 2048 and r["frames"] == 16 and r["height"] == 256
    assert 0 < r["ms_min"] <= r["ms_mean"] and r["wall_ms_min"] >= r["ms_min"]


def test_jepa_embed_image(jlib, oracle, models_dir, tmp_path):
    """jepa-embed on a JPEG with an image model (CLS token): the preprocessed input it dumps equals
    jepa_preprocess_frames_rgb_ex with the model's default parameters on jepa_load_image_rgb's pixels,
    its --pool none rows equal jepa_encode's on that input bit for bit (and the oracle's within the
    encoder gate), and --pool cls gives jepa_pool_cls of those rows."""
    exe = _tool("jepa-embed")
    path = forge.cached_model(forge.tiny("hfvit", "f16", ln_random=True), models_dir)
    rows_f, pooled_f, x_f = tmp_path / "rows.npy", tmp_path / "cls.npy", tmp_path / "x.npy"
    _run([exe, "-m", path, "-i", IMAGE, "--pool", "none", "-o", str(rows_f), "--dump-input", str(x_f), "--print-n", "0"])
    _run([exe, "-m", path, "-i", IMAGE, "-o", str(pooled_f), "--print-n", "0"])
    x, rows, pooled = np.load(x_f), np.load(rows_f), np.load(pooled_f)
    m = jlib.Model(path)
    want_x = jlib.preprocess_frames(jlib.lib().jepa_preprocess_default_params(m.ptr), [jlib.load_image(IMAGE)])
    np.testing.assert_array_equal(x.view(np.uint32), want_x[None].view(np.uint32))
    ctx = jlib.Context(m)
    got = ctx.encode(x)
    np.testing.assert_array_equal(rows.view(np.uint32), got.view(np.uint32))
    np.testing.assert_array_equal(pooled.reshape(-1).view(np.uint32), m.pool_cls(got).view(np.uint32))
    want, _ = oracle.encode(path, x, 1, got.shape[0], m.dim)
    c = _cos_rows(got, want)
    print(f"jepa-embed image: {rows.shape[0]} rows x {rows.shape[1]}, cosine vs oracle mean {c.mean():.7f} min {c.min():.7f}")
    assert c.mean() >= 0.9999 and c.min() >= 0.999


def test_jepa_embed_clip_with_head(jlib, models_dir, tmp_path):
    """jepa-embed --frames-npy on a THWC uint8 clip with a video model that carries an attentive-pool
    head: --pool mean equals jepa_pool_mean of jepa_encode's rows on the input it dumps, and --logits
    equals jepa_head_ex on those rows, bit for bit."""
    exe = _tool("jepa-embed")
    cfg = forge.tiny("vjepa2", "q8_0", ln_random=True, n_classes=10, n_pool_layers=1)
    path = forge.cached_model(cfg, models_dir)
    rng = np.random.default_rng(7)
    frames = rng.integers(0, 256, size=(4, 72, 90, 3), dtype=np.uint8)
    clip_f, feat_f, logit_f, x_f = (tmp_path / n for n in ("clip.npy", "feat.npy", "logits.npy", "x.npy"))
    np.save(clip_f, frames)
    _run([exe, "-m", path, "--frames-npy", str(clip_f), "--pool", "mean", "-o", str(feat_f), "--logits", str(logit_f),
          "--dump-input", str(x_f), "--print-n", "0"])
    x, feat, logits = np.load(x_f), np.load(feat_f), np.load(logit_f)
    m = jlib.Model(path)
    want_x = jlib.preprocess_frames(jlib.lib().jepa_preprocess_default_params(m.ptr), list(frames))
    np.testing.assert_array_equal(x.view(np.uint32), want_x[None].view(np.uint32))
    ctx = jlib.Context(m)
    got = ctx.encode(x)
    np.testing.assert_array_equal(feat.reshape(-1).view(np.uint32), m.pool_mean(got).view(np.uint32))
    _, want_logits = ctx.head(got, pooled=False, logits=True)
    assert logits.shape == (1, m.n_classes)
    np.testing.assert_array_equal(logits.reshape(-1).view(np.uint32), want_logits.view(np.uint32))


def test_jepa_classify_clip(jlib, models_dir, tmp_path):
    """jepa-classify --frames-npy on a THWC uint8 clip with a video model that carries an attentive-pool
    head: the logits it saves equal jepa_head_ex on jepa_encode's rows of the input it dumps, bit for
    bit, and its printed top-k (jepa_softmax, jepa_top_k, jepa_model_label) ranks those logits with
    their softmax percentages."""
    exe = _tool("jepa-classify")
    cfg = forge.tiny("vjepa2", "q8_0", ln_random=True, n_classes=10, n_pool_layers=1)
    path = forge.cached_model(cfg, models_dir)
    frames = np.random.default_rng(11).integers(0, 256, size=(4, 80, 64, 3), dtype=np.uint8)
    clip_f, logit_f, x_f = (tmp_path / n for n in ("clip.npy", "logits.npy", "x.npy"))
    np.save(clip_f, frames)
    r = _run([exe, "-m", path, "--frames-npy", str(clip_f), "-k", "3", "--logits", str(logit_f), "--dump-input", str(x_f)])
    x, logits = np.load(x_f), np.load(logit_f)
    m = jlib.Model(path)
    ctx = jlib.Context(m)
    got = ctx.encode(x)
    _, want = ctx.head(got, pooled=False, logits=True)
    assert logits.shape == (m.n_classes,)
    np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32))
    # "  %2d. %6.2f%%  [%3d] label" per class
    top = [m_.groups() for m_ in (re.match(r"^\s*(\d+)\.\s+([\d.]+)%\s+\[\s*(\d+)\]", line) for line in r.stdout.splitlines()) if m_]
    assert len(top) == 3, r.stdout
    p = np.exp(want.astype(np.float64) - want.max())
    p /= p.sum()
    order = np.argsort(-want, kind="stable")[:3]
    for rank, ((k, pct, idx), i) in enumerate(zip(top, order)):
        assert int(k) == rank + 1 and int(idx) == i, (top, order)
        assert abs(float(pct) - 100 * p[i]) <= 0.006, (pct, p[i])


def test_reference_test_batch(models_dir, tmp_path):
    """The reference's own tests/test-batch.cpp, compiled as it lies against this library: the eight
    COCO fixture images (tests/golden/media, the reference's tests/fixtures/media) through image models
    in one call, in chunks of 3 and one at a time (f32 bit for bit, other file types at its cosine gate),
    and two clips of 18 frames (2304 rows each) of an f16 video model in one call against two calls,
    bit for bit for every file type."""
    exe = _tool("test-batch")
    media = os.path.join(ROOT, "tests", "golden", "media")
    models = [forge.cached_model(cfg, models_dir) for cfg in (
        forge.tiny("hfvit", "f32", ln_random=True), forge.tiny("hfvit", "f16", ln_random=True),
        forge.tiny("ijepa", "q8_0"))]
    video = forge.cached_model(forge.tiny("vjepa2", "f16", ffn_dim=1024, img_size=256, ln_random=True), models_dir)
    rng = np.random.default_rng(3)
    clips = []
    for i in range(2):
        c = tmp_path / f"clip{i}.npy"
        np.save(c, rng.integers(0, 256, size=(18, 256, 256, 3), dtype=np.uint8))
        clips += ["--clip", str(c)]
    args = [exe, "--media", media]
    for p in models:
        args += ["--image", p]
    r = _run(args + ["--video", video] + clips)
    print(r.stdout)
    assert "all batched outputs match the per-item path" in r.stdout
    assert r.stdout.count(" OK") >= 3 * 5 + 1 and " FAIL" not in r.stdout


@pytest.mark.parametrize("family,ftype", [("vjepa2", "q8_0"), ("vjepa2", "f16"), ("vjepa2", "f32"), ("vjepa2_1", "q8_0"),
                                          ("vitl16", "q8_0")])
def test_reference_test_predictor_case(oracle, models_dir, tmp_path, family, ftype):
    """The reference's own tests/test-predictor.cpp in its --case mode (DIR/{enc,ctx_idx,tgt_idx,pred}.npy,
    tests/test-predictor.cpp:612-637), compiled as it lies against this library: jepa_predict_mod on the
    case's encoder rows and ids against pred.npy, written here by the oracle's predictor on the same
    file, under the reference's own GPU bars for the file type. Tiny V-JEPA 2 / 2.1 predictors, and the
    V-JEPA 2 ViT-L predictor (384 wide, 12 blocks) over 2048 tokens split 1024 / 1024."""
    exe = _tool("test-predictor")
    if family == "vitl16":
        cfg = forge.CONFIGS["vitl16_pred_q8_0"]
        n_tok, n_ctx = 2048, 1024
    else:
        kw = {"pred_mlp_embed": True} if family == "vjepa2_1" else {}
        cfg = forge.tiny(family, ftype, ln_random=True, pred_dim=128, pred_layers=2, pred_ffn=512, w_std=0.08, **kw)
        n_tok, n_ctx = 32, 20
    path = forge.cached_model(cfg, models_dir)
    rng = np.random.default_rng(17)
    enc = rng.standard_normal((n_tok, cfg.embed_dim)).astype(np.float32)
    perm = rng.permutation(n_tok)
    ctx_ids, tgt_ids = perm[:n_ctx], perm[n_ctx:]
    pred = oracle.predict(path, enc, ctx_ids, tgt_ids, cfg.embed_dim, mask_index=1, modality=1)
    for f, a in (("enc", enc), ("ctx_idx", ctx_ids.astype(np.int64)), ("tgt_idx", tgt_ids.astype(np.int64)), ("pred", pred)):
        np.save(tmp_path / f"{f}.npy", a)
    r = _run([exe, "--vjepa2", path, "--case", str(tmp_path)])
    print(r.stdout)
    assert r.stdout.rstrip().endswith("PASS") and " OK" in r.stdout, r.stdout


@pytest.mark.parametrize("name", ["vitb16_2_1_q8_0", "vits16_f16"])
def test_reference_test_batch_full_size(models_dir, name):
    """The reference's own tests/test-batch.cpp on two of the benchmark configurations at full size: V-JEPA
    2.1 ViT-B/16 384x384 q8_0 through its image path (eight images in one call: the batch of 8 images
    the image benchmark runs) and the LeJEPA-shaped ViT-S/16 224x224 f16 model, over the eight COCO
    fixtures in one call, in chunks of 3 and one at a time."""
    exe = _tool("test-batch")
    path = forge.cached_model(forge.CONFIGS[name], models_dir)
    r = _run([exe, "--media", os.path.join(ROOT, "tests", "golden", "media"), "--image", path])
    print(r.stdout)
    assert "all batched outputs match the per-item path" in r.stdout and " FAIL" not in r.stdout
