"""The oracle's whole encoder forward, pinned against an independent float64 forward written from the
reference graph (no GPU): patchify row order (reference src/jepa.cpp:476-505), patch linear, CLS and
learned positions for the image families (586-627), modality embedding, and 3-D RoPE on q and k for the
video families (846-895), pre-LN blocks with fused qkv, attention with f16-rounded K/V, erf-GELU MLP,
optional layer scale (444-471), final LayerNorm. Models are tiny f32 GGUFs, so the only differences
left are float32 rounding (no activation quantization). Also: GGUF writer/reader round trip and the
oracle's batch invariance."""
import math

import numpy as np
import pytest

from jepa_amd import forge, gguf, inputs
from oracle import oracle as O


def _ln(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _gelu(x):
    return 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))


def _rope_tables64(grid, hd, variant, interp, train, theta):
    """float64 cos / sin tables from the definitions (reference src/rope3d.h:9-48), lanes past 3d identity."""
    gt, gh, gw = grid
    d = 2 * ((hd // 3) // 2)
    omega = 1.0 / theta ** (np.arange(d // 2) / (d // 2))
    lane = np.arange(d) % (d // 2) if variant == 0 else np.arange(d) // 2
    n = gt * gh * gw
    C, S = np.ones((n, hd)), np.zeros((n, hd))
    for i in range(n):
        t, h, w = i // (gh * gw), (i % (gh * gw)) // gw, i % gw
        if interp:
            h = h * (train[0] - 1) / (gh - 1) if gh > 1 else h
            w = w * (train[1] - 1) / (gw - 1) if gw > 1 else w
        for a, pos in enumerate((t, h, w)):
            C[i, a * d:(a + 1) * d] = np.cos(pos * omega[lane])
            S[i, a * d:(a + 1) * d] = np.sin(pos * omega[lane])
    return C, S


def _rot(x, C, S):
    """out[2k] = x[2k] C[2k] - x[2k+1] S[2k]; out[2k+1] = x[2k+1] C[2k+1] + x[2k] S[2k+1]"""
    sw = x.copy()
    sw[..., 0::2], sw[..., 1::2] = -x[..., 1::2], x[..., 0::2]
    return x * C + sw * S


def _block64(T, has, p, h, D, H, rope, mask, kv_f16):
    """One pre-LN block (reference src/jepa.cpp:444-471) in float64."""
    n, hd = h.shape[0], D // H
    a = _ln(h, T(p + "ln1.weight"), T(p + "ln1.bias"), 1e-6)
    if has(p + "attn_qkv.weight"):
        qkv = a @ T(p + "attn_qkv.weight").T + T(p + "attn_qkv.bias")
    else:   # separate q, k, v linears (reference src/jepa.cpp:408-414)
        qkv = np.concatenate([a @ T(p + f"attn_{j}.weight").T + T(p + f"attn_{j}.bias") for j in "qkv"], axis=1)
    q, k, v = (qkv[:, j * D:(j + 1) * D].reshape(n, H, hd) for j in range(3))
    if rope is not None:
        q, k = _rot(q, rope[0][:, None], rope[1][:, None]), _rot(k, rope[0][:, None], rope[1][:, None])
    if kv_f16:
        k = k.astype(np.float32).astype(np.float16).astype(np.float64)
        v = v.astype(np.float32).astype(np.float16).astype(np.float64)
    att = np.zeros((n, H, hd))
    for hh in range(H):
        s = q[:, hh] @ k[:, hh].T / math.sqrt(hd) + (0 if mask is None else mask)
        pr = np.exp(s - s.max(1, keepdims=True))
        att[:, hh] = (pr / pr.sum(1, keepdims=True)) @ v[:, hh]
    o = att.reshape(n, D) @ T(p + "attn_out.weight").T + T(p + "attn_out.bias")
    if has(p + "ls1"):
        o = o * T(p + "ls1")
    h = h + o
    f = _ln(h, T(p + "ln2.weight"), T(p + "ln2.bias"), 1e-6) @ T(p + "ffn_up.weight").T + T(p + "ffn_up.bias")
    f = _gelu(f) @ T(p + "ffn_down.weight").T + T(p + "ffn_down.bias")
    if has(p + "ls2"):
        f = f * T(p + "ls2")
    return h + f


def head64(path, rows):
    """The attentive-pool head (reference src/jepa.cpp:1026-1075) in float64 on encoder rows [N, D]:
    pooler blocks without RoPE, one query cross-attending to LN_kv(x) with no output projection, the
    residual on the raw query, LN2 + MLP, then the classifier. Returns (pooled, logits)."""
    g = gguf.read_gguf(path)
    kv = g.kv
    T = lambda n: g.tensor_f32(n).astype(np.float64)
    has = lambda n: n in g.tensors
    D, H = kv["jepa.enc.embed_dim"], kv["jepa.enc.n_head"]
    hd = D // H
    x = rows.astype(np.float64)
    for i in range(kv["jepa.head.n_pool_layers"]):
        x = _block64(T, has, f"head.blk.{i}.", x, D, H, None, None, kv["general.file_type"] != 0)
    q0 = T("head.query").reshape(D)
    kvn = _ln(x, T("head.xattn.ln_kv.weight"), T("head.xattn.ln_kv.bias"), 1e-6)
    q = (q0 @ T("head.xattn.q.weight").T + T("head.xattn.q.bias")).reshape(H, hd)
    k = (kvn @ T("head.xattn.k.weight").T + T("head.xattn.k.bias")).reshape(-1, H, hd)
    v = (kvn @ T("head.xattn.v.weight").T + T("head.xattn.v.bias")).reshape(-1, H, hd)
    o = np.zeros((H, hd))
    for hh in range(H):
        s = k[:, hh] @ q[hh] / math.sqrt(hd)
        pr = np.exp(s - s.max())
        o[hh] = (pr / pr.sum()) @ v[:, hh]
    y = o.reshape(D) + q0
    f = _ln(y, T("head.xattn.ln2.weight"), T("head.xattn.ln2.bias"), 1e-6) @ T("head.xattn.ffn_up.weight").T
    f = _gelu(f + T("head.xattn.ffn_up.bias")) @ T("head.xattn.ffn_down.weight").T + T("head.xattn.ffn_down.bias")
    y = y + f
    return y, y @ T("head.cls.weight").T + T("head.cls.bias")


def predict64(path, enc, ctx_ids, tgt_ids, mask_index=1, modality=1):
    """The masked predictor (reference src/predictor.cpp:56-133) in float64: embed the context rows,
    mask-token rows for the targets, modality vector, blocks with RoPE from the token ids on the
    predictor grid, final norm and projection of the target rows."""
    g = gguf.read_gguf(path)
    kv = g.kv
    T = lambda n: g.tensor_f32(n).astype(np.float64)
    has = lambda n: n in g.tensors
    Dp, H = kv["jepa.pred.embed_dim"], kv["jepa.pred.n_head"]
    hd = Dp // H
    ids = np.concatenate([np.asarray(ctx_ids, np.int64), np.asarray(tgt_ids, np.int64)])
    rows = enc[np.asarray(ctx_ids, np.int64)].astype(np.float64)
    if has("pred.embed.0.weight"):
        h = _gelu(rows @ T("pred.embed.0.weight").T + T("pred.embed.0.bias"))
        ctx = h @ T("pred.embed.2.weight").T + T("pred.embed.2.bias")
    else:
        ctx = rows @ T("pred.embed.weight").T + T("pred.embed.bias")
    mt = T("pred.mask_tokens").reshape(-1, Dp)
    n_mask = kv.get("jepa.pred.n_mask_tokens") or mt.shape[0]
    x = np.vstack([ctx, np.repeat(mt[mask_index % n_mask][None], len(tgt_ids), 0)])
    if kv.get("jepa.pred.modality_embed"):
        x = x + T("pred.mod_embed_img" if modality == 2 else "pred.mod_embed_video")
    grid = kv.get("jepa.pred.grid_size") or kv["jepa.enc.img_size"] // kv["jepa.enc.patch_size"]
    gt = int(ids.max()) // (grid * grid) + 1
    lay = kv.get("jepa.pred.rope_freq_layout") or ("interleaved" if kv["jepa.family"] == "vjepa2_1" else "tiled")
    C, S = _rope_tables64((gt, grid, grid), hd, 0 if lay == "tiled" else 1, False, (0, 0), float(kv["jepa.enc.rope_theta"]))
    rope = (C[ids], S[ids])
    for i in range(kv["jepa.pred.n_layer"]):
        x = _block64(T, has, f"pred.blk.{i}.", x, Dp, H, rope, None, kv["general.file_type"] != 0)
    y = _ln(x[len(ctx_ids):], T("pred.norm.weight"), T("pred.norm.bias"), 1e-6)
    return y @ T("pred.proj.weight").T + T("pred.proj.bias")


def forward64(path, x):
    g = gguf.read_gguf(path)
    kv = g.kv
    T = lambda n: g.tensor_f32(n).astype(np.float64)
    has = lambda n: n in g.tensors
    fam = kv["jepa.family"]
    D, L, H, P = kv["jepa.enc.embed_dim"], kv["jepa.enc.n_layer"], kv["jepa.enc.n_head"], kv["jepa.enc.patch_size"]
    hd, eps = D // H, float(kv["jepa.enc.ln_eps"])
    video = fam in ("vjepa2", "vjepa2_1", "levjepa")
    kv_f16 = kv["general.file_type"] != 0      # the CPU's K/V type rule (reference src/jepa.cpp:531-535)
    B, Cc, Tt, Hh, Ww = x.shape
    tub = kv["jepa.enc.tubelet_size"] if video else 1
    items = []
    for b in range(B):
        clips = [x[b]] if video else [x[b][:, t:t + 1] for t in range(Tt)]
        for clip in clips:
            gt, gh, gw = clip.shape[1] // tub, Hh // P, Ww // P
            rows = []
            for t in range(gt):
                for h in range(gh):
                    for w in range(gw):
                        rows.append(clip[:, t * tub:(t + 1) * tub, h * P:(h + 1) * P, w * P:(w + 1) * P].reshape(-1))
            items.append((np.array(rows, np.float64), (gt, gh, gw)))
    outs, streams = [], []
    for rows, grid in items:
        h = rows @ T("enc.patch_embed.weight").T + T("enc.patch_embed.bias")
        if has("enc.mod_embed_video"):
            h = h + T("enc.mod_embed_video")
        if kv.get("jepa.enc.n_registers", 0):        # registers, then the CLS row, go in front
            h = np.concatenate([T("enc.reg_tokens").reshape(-1, D), h])
        if kv.get("jepa.enc.cls_token"):
            h = np.concatenate([T("enc.cls_token")[None], h])
        if has("enc.pos_embed"):
            h = h + T("enc.pos_embed")
        rope = None
        if video:
            ref = kv.get("jepa.enc.rope_ref_grid", 0)
            rope = _rope_tables64(grid, hd, 0 if kv["jepa.enc.rope_freq_layout"] == "tiled" else 1,
                                  bool(kv.get("jepa.enc.rope_interpolate")), (ref, ref), float(kv["jepa.enc.rope_theta"]))
        n = h.shape[0]
        npre = n - rows.shape[0]                  # CLS and register rows in front of the patch rows
        if rope is not None and npre:             # the prefix is not rotated (identity rows)
            rope = (np.vstack([np.ones((npre, hd)), rope[0]]), np.vstack([np.zeros((npre, hd)), rope[1]]))
        mask = np.zeros((n, n))
        if kv.get("jepa.enc.attn_mode") == "block_causal":
            # LeVJEPA (docs/gguf-schema.md, levjepa note): key j visible to query i iff frame(i) >= frame(j);
            # the CLS row is open, the CLS column closed to the patch queries
            tpf = grid[1] * grid[2]
            frame = np.concatenate([np.full(npre, -1), np.arange(n - npre) // tpf])
            vis = (frame[:, None] >= frame[None, :]) & (frame[None, :] >= 0)
            vis[:npre] = True
            mask[~vis] = -np.inf
        for i in range(L):
            h = _block64(T, has, f"enc.blk.{i}.", h, D, H, rope, mask, kv_f16)
        streams.append(h)
        outs.append(_ln(h, T("enc.norm.weight"), T("enc.norm.bias"), eps))
    return np.concatenate(outs), np.stack(streams), outs[0].shape[0], len(outs)


@pytest.mark.parametrize("family,kw", [("hfvit", {}), ("hfvit", {"layer_scale": True}), ("vjepa2", {}),
                                       ("vjepa2_1", {}), ("levjepa", {}), ("hfvit", {"n_registers": 4}),
                                       ("vjepa2", {"n_registers": 2}), ("levjepa", {"n_registers": 3}),
                                       ("hfvit", {"qkv_fused": False}), ("vjepa2", {"qkv_fused": False})])
def test_oracle_encoder_matches_float64_forward(family, kw, tmp_path):
    cfg = forge.tiny(family, "f32", ln_random=True, **kw)
    path = forge.cached_model(cfg, str(tmp_path))
    x = inputs.make_input(2, 1 if family == "hfvit" else 4, 64, 64, seed=11)
    want, stream, rows, items = forward64(path, x)
    got, tr = O.encode(path, x, items, rows, cfg.embed_dim, n_layers=cfg.n_layer, trace=True)
    # residual stream after the last block: float32 vs float64 rounding only (~1e-6 of its scale)
    err_stream = np.abs(tr[:, -1] - stream).max() / np.abs(stream).max()
    assert err_stream < 2e-5, err_stream
    # final LayerNorm output: rows with a small residual (the CLS row) have their rounding scaled up
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 5e-4, err


def test_oracle_head_matches_float64_head(tmp_path):
    """The oracle's attentive-pool head against the float64 restatement above, on a tiny f32 model with
    two pooler blocks and 10 classes; random LayerNorm affines so that ln_kv / ln2 count."""
    cfg = forge.tiny("vjepa2", "f32", ln_random=True, n_classes=10, n_pool_layers=2)
    path = forge.cached_model(cfg, str(tmp_path))
    rows = np.random.default_rng(5).standard_normal((40, cfg.embed_dim)).astype(np.float32)
    want_p, want_l = head64(path, rows)
    got_p, got_l = O.head(path, rows, cfg.n_classes)
    assert got_l.shape == (10,)
    assert np.abs(got_p - want_p).max() / np.abs(want_p).max() < 2e-5
    assert np.abs(got_l - want_l).max() / np.abs(want_l).max() < 1e-4


@pytest.mark.parametrize("family,kw", [("vjepa2", {}), ("vjepa2_1", {"pred_mlp_embed": True})])
def test_oracle_predictor_matches_float64_predictor(family, kw, tmp_path):
    """The oracle's masked predictor against the float64 restatement above on a tiny f32 model with
    heads of 32 and weights large enough for position-dependent attention: context ids and target ids
    interleaved over two temporal slices, mask index 3 of 10, the 2.1 modality vectors."""
    cfg = forge.tiny(family, "f32", ln_random=True, pred_dim=128, pred_layers=2, pred_ffn=512, w_std=0.08, **kw)
    path = forge.cached_model(cfg, str(tmp_path))
    rng = np.random.default_rng(3)
    enc = rng.standard_normal((32, cfg.embed_dim)).astype(np.float32)
    perm = rng.permutation(32)
    ctx, tgt = perm[:20], perm[20:]
    for modality in ((1, 2) if family == "vjepa2_1" else (1,)):
        want = predict64(path, enc, ctx, tgt, mask_index=3, modality=modality)
        got = O.predict(path, enc, ctx, tgt, cfg.embed_dim, mask_index=3, modality=modality)
        err = np.abs(got - want).max() / np.abs(want).max()
        assert err < 2e-5, (modality, err)
        # the targets differ from each other by more than the tolerance: the ids reach the output
        spread = np.abs(want - want.mean(0)).max() / np.abs(want).max()
        assert spread > 100 * 2e-5, spread


def test_oracle_items_are_independent(tmp_path):
    """Items of one call equal separate calls bit for bit (reference tests/test-batch.cpp:12-21)."""
    cfg = forge.tiny("vjepa2", "q8_0")
    path = forge.cached_model(cfg, str(tmp_path))
    x = inputs.make_input(2, 4, 64, 64, seed=2)
    both, _ = O.encode(path, x, 2, 16 * 2, cfg.embed_dim, n_layers=cfg.n_layer)
    for b in range(2):
        one, _ = O.encode(path, x[b:b + 1], 1, 32, cfg.embed_dim, n_layers=cfg.n_layer)
        np.testing.assert_array_equal(one.view(np.uint32), both[b * 32:(b + 1) * 32].view(np.uint32))


def test_gguf_roundtrip(tmp_path):
    rng = np.random.default_rng(1)
    w = gguf.GGUFWriter()
    w.add("a.u32", 7)
    w.add("a.i32", -3)
    w.add("a.f32", 0.25)
    w.add("a.bool", True)
    w.add("a.str", "héllo")
    w.add("a.strs", ["x", "yz"])
    w.add("a.ints", [1, -2, 3])
    w.add("a.floats", [0.5, 1.5])
    t32 = rng.standard_normal((3, 64)).astype(np.float32)
    t16 = rng.standard_normal((2, 64)).astype(np.float16)
    q8 = gguf.quantize(gguf.GGML_Q8_0, rng.standard_normal((4, 64)).astype(np.float32))
    w.add_tensor("t.f32", gguf.GGML_F32, (64, 3), t32)
    w.add_tensor("t.f16", gguf.GGML_F16, (64, 2), t16)
    w.add_tensor("t.q8", gguf.GGML_Q8_0, (64, 4), q8)
    p = str(tmp_path / "r.gguf")
    w.write(p)
    g = gguf.read_gguf(p)
    assert g.kv["a.u32"] == 7 and g.kv["a.i32"] == -3 and g.kv["a.f32"] == 0.25 and g.kv["a.bool"] is True
    assert g.kv["a.str"] == "héllo" and list(g.kv["a.strs"]) == ["x", "yz"] and list(g.kv["a.ints"]) == [1, -2, 3]
    np.testing.assert_array_equal(g.tensor_f32("t.f32"), t32)
    np.testing.assert_array_equal(g.tensor_f32("t.f16"), t16.astype(np.float32))
    np.testing.assert_array_equal(np.asarray(g.tensor_bytes("t.q8")).reshape(q8.shape), q8)
    for t in g.tensors.values():
        assert t.offset % 32 == 0
