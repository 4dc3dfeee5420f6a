"""Synthetic (random-init) jepa GGUF models for the encoder configurations.

Tensor names, shapes, dtypes and metadata keys follow the reference schema (docs/gguf-schema.md:18-96)
and its quantization rule (docs/gguf-schema.md "Quantization rules", tools/jepa-quantize.cpp:91-129):
only the 2-D block matrices (attn_qkv, attn_out, ffn_up, ffn_down) take the file type, with the
per-tensor K-quant fallback to q4_0 when the row length is not a multiple of 256; patch embeddings
are F16 in video-family files and F32 in hfvit files (the converters' choice), everything else F32.

Weights are N(0, 0.02) from a seeded numpy PCG64 generator. LayerNorm gamma/beta are 1/0 unless
`ln_random` is set (then 1 + N(0, 0.1) / N(0, 0.1), which exercises the affine terms).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, replace

import numpy as np

from .gguf import (FTYPE, GGML_F16, GGML_F32, GGML_Q4_0, GGML_Q4_K, GGML_Q8_0, GGUFWriter, quantize)


@dataclass(frozen=True)
class EncoderConfig:
    name: str
    family: str            # hfvit | ijepa | vjepa2 | vjepa2_1 | levjepa
    embed_dim: int
    n_layer: int
    n_head: int
    ffn_dim: int
    patch: int = 16
    tubelet: int = 1
    img_size: int = 224
    n_frames: int = 1
    cls_token: bool = False
    n_registers: int = 0    # register tokens after the CLS row (enc.reg_tokens)
    qkv_fused: bool = True  # False: separate attn_q / attn_k / attn_v (the rows of the fused matrix)
    qkv_parts: str = ""     # split q / k / v: per part "<dtype>" or "<dtype>+b" (with its bias), comma list; "": all
                            # parts of the file type with biases
    ftype: str = "q8_0"     # f16 | q8_0 | q4_0 | q4_k
    rope_layout: str = ""   # tiled | interleaved ('' for non-rope families)
    rope_interpolate: bool = False
    rope_ref_grid: int = 0
    modality_embed: bool = False
    image_patch_embed: bool = False
    layer_scale: bool = False
    ln_random: bool = False
    attn_mode: str = "full"  # full | block_causal (levjepa)
    n_classes: int = 0       # > 0: attentive-pool classifier head (video families)
    n_pool_layers: int = 0   # self-attention blocks of the head, run before the cross-attention
    pred_dim: int = 0        # > 0: masked predictor of this width (heads of 32, V-JEPA 2 / 2.1)
    pred_layers: int = 0
    pred_ffn: int = 0
    pred_mask_tokens: int = 10
    pred_mlp_embed: bool = False   # pred.embed.0 / .2 two-layer embedding (V-JEPA 2.1 ViT-g/G)
    pred_grid: int = 0             # jepa.pred.grid_size (0: the encoder's img_size / patch)
    w_std: float = 0.02            # standard deviation of the matmul weights
    seed: int = 1234


# The five configurations the benchmark and parity tests are quoted on.
CONFIGS = {
    # LeJEPA ViT-S/16 224x224, hfvit (CLS + learned position table), f16 weights
    "vits16_f16": EncoderConfig("lejepa-vits16-synthetic", "hfvit", 384, 12, 6, 1536, patch=16, img_size=224,
                                cls_token=True, ftype="f16"),
    # V-JEPA 2.1 ViT-B/16 384x384 image path (1x16x16 tokenizer, image modality vector, interleaved RoPE)
    "vitb16_2_1_q8_0": EncoderConfig("vjepa2_1-vitb16-384-synthetic", "vjepa2_1", 768, 12, 12, 3072, patch=16,
                                     tubelet=2, img_size=384, n_frames=64, ftype="q8_0", rope_layout="interleaved",
                                     rope_interpolate=True, rope_ref_grid=16, modality_embed=True,
                                     image_patch_embed=True),
    # V-JEPA 2 ViT-L/16 256x256, 16 frames (2048 tokens), tiled RoPE
    "vitl16_q8_0": EncoderConfig("vjepa2-vitl16-256-synthetic", "vjepa2", 1024, 24, 16, 4096, patch=16, tubelet=2,
                                 img_size=256, n_frames=16, ftype="q8_0", rope_layout="tiled"),
    "vitl16_q4_k": EncoderConfig("vjepa2-vitl16-256-synthetic", "vjepa2", 1024, 24, 16, 4096, patch=16, tubelet=2,
                                 img_size=256, n_frames=16, ftype="q4_k", rope_layout="tiled"),
    # LeVJEPA ViT-L/16 224x224, 16 frames, tubelet 1 (16 x 196 patch tokens + CLS = 3137 rows), block-causal
    # attention, tiled RoPE with an identity row for the CLS
    "levjepa_vitl16_q8_0": EncoderConfig("levjepa-vitl16-224-synthetic", "levjepa", 1024, 24, 16, 4096, patch=16,
                                         tubelet=1, img_size=224, n_frames=16, cls_token=True, ftype="q8_0",
                                         rope_layout="tiled", attn_mode="block_causal"),
    # V-JEPA 2 ViT-g/16 256x256, 64 frames (8192 tokens)
    # V-JEPA 2 ViT-L/16 256x256 16-frame classifier: the encoder plus the SSv2 attentive-pool head
    # (3 pooler blocks over the 2048 tokens, cross-attention, 174 classes)
    "vitl16_ssv2_q8_0": EncoderConfig("vjepa2-vitl16-256-ssv2-synthetic", "vjepa2", 1024, 24, 16, 4096, patch=16,
                                      tubelet=2, img_size=256, n_frames=16, ftype="q8_0", rope_layout="tiled",
                                      n_classes=174, n_pool_layers=3),
    # V-JEPA 2 ViT-L/16 with its masked predictor (384 wide, 12 blocks, 12 heads of 32, 10 mask tokens)
    "vitl16_pred_q8_0": EncoderConfig("vjepa2-vitl16-256-predictor-synthetic", "vjepa2", 1024, 24, 16, 4096, patch=16,
                                      tubelet=2, img_size=256, n_frames=16, ftype="q8_0", rope_layout="tiled",
                                      pred_dim=384, pred_layers=12, pred_ffn=1536),
    "vitg16_q8_0": EncoderConfig("vjepa2-vitg16-256-synthetic", "vjepa2", 1408, 40, 22, 6144, patch=16, tubelet=2,
                                 img_size=256, n_frames=64, ftype="q8_0", rope_layout="tiled"),
    # I-JEPA ViT-H/14 224x224 (facebook/ijepa_vith14_1k's shape: 16 x 16 = 256 patch tokens, no CLS, learned /
    # sincos position table, D 1280, 16 heads of 80, MLP 5120, 32 layers, f32 patch embedding of 588 inputs)
    "vith14_ijepa_f16": EncoderConfig("ijepa-vith14-224-synthetic", "ijepa", 1280, 32, 16, 5120, patch=14, img_size=224,
                                      ftype="f16"),
    "vith14_ijepa_q8_0": EncoderConfig("ijepa-vith14-224-synthetic", "ijepa", 1280, 32, 16, 5120, patch=14,
                                       img_size=224, ftype="q8_0"),
}


def tiny(family: str, ftype: str, **kw) -> EncoderConfig:
    """Small models for parity tests (seconds on the oracle)."""
    if family == "hfvit":
        base = EncoderConfig("tiny-hfvit", "hfvit", 128, 2, 2, 512, patch=16, img_size=64, cls_token=True, ftype=ftype)
    elif family == "vjepa2":
        base = EncoderConfig("tiny-vjepa2", "vjepa2", 128, 2, 2, 512, patch=16, tubelet=2, img_size=64, n_frames=4,
                             ftype=ftype, rope_layout="tiled")
    elif family == "vjepa2_1":
        base = EncoderConfig("tiny-vjepa2_1", "vjepa2_1", 128, 2, 2, 512, patch=16, tubelet=2, img_size=64,
                             n_frames=4, ftype=ftype, rope_layout="interleaved", rope_interpolate=True,
                             rope_ref_grid=16, modality_embed=True, image_patch_embed=True)
    elif family == "ijepa":   # heads of 80, patch 14 (588 patch inputs)
        base = EncoderConfig("tiny-ijepa", "ijepa", 640, 2, 8, 2560, patch=14, img_size=112, ftype=ftype)
    elif family == "levjepa":
        base = EncoderConfig("tiny-levjepa", "levjepa", 128, 2, 2, 512, patch=16, tubelet=1, img_size=64, n_frames=4,
                             cls_token=True, ftype=ftype, rope_layout="tiled", attn_mode="block_causal")
    else:
        raise ValueError(family)
    return replace(base, **kw)


_QTYPE = {"f16": GGML_F16, "q8_0": GGML_Q8_0, "q4_0": GGML_Q4_0, "q4_k": GGML_Q4_K, "f32": GGML_F32}


def _block_type(cfg: EncoderConfig, n_in: int) -> int:
    t = _QTYPE[cfg.ftype]
    if t == GGML_Q4_K and n_in % 256:
        return GGML_Q4_0          # K-quant fallback (tools/jepa-quantize.cpp:70-77)
    return t


def _device_q4_k():
    """The library's own q4_K block quantizer on the GPU (jepa_amd_quantize_rows, byte-equal to the numpy
    restatement), or None without a GPU. The numpy make_qkx2 search takes minutes on a ViT-L."""
    try:
        import torch
        if not torch.cuda.is_available():
            return None
        from . import _lib
        L = _lib.lib()
    except Exception:
        return None

    def q(x: np.ndarray) -> np.ndarray:
        xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32).reshape(-1)).cuda()
        out = torch.empty(xd.numel() // 256 * 144, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        if L.jepa_amd_quantize_rows(0, GGML_Q4_K, xd.data_ptr(), xd.numel(), out.data_ptr()) != 0:
            raise RuntimeError("jepa_amd_quantize_rows failed: " + _lib.error_text())
        return out.cpu().numpy()
    return q


def write_model(cfg: EncoderConfig, path: str) -> str:
    """Write the synthetic GGUF for `cfg` to `path` (returns path)."""
    rng = np.random.default_rng(cfg.seed)
    D, F = cfg.embed_dim, cfg.ffn_dim
    video = cfg.family in ("vjepa2", "vjepa2_1", "levjepa")
    w = GGUFWriter()
    w.add("general.architecture", "jepa")
    w.add("general.name", cfg.name)
    w.add("general.file_type", FTYPE[cfg.ftype])
    w.add("jepa.schema_version", 1)
    w.add("jepa.family", cfg.family)
    w.add("jepa.modality", "video" if video else "image")
    w.add("jepa.enc.embed_dim", D)
    w.add("jepa.enc.n_layer", cfg.n_layer)
    w.add("jepa.enc.n_head", cfg.n_head)
    w.add("jepa.enc.ffn_dim", F)
    w.add("jepa.enc.patch_size", cfg.patch)
    w.add("jepa.enc.tubelet_size", cfg.tubelet)
    w.add("jepa.enc.img_size", cfg.img_size)
    w.add("jepa.enc.n_frames", cfg.n_frames)
    w.add("jepa.enc.in_chans", 3)
    w.add("jepa.enc.ln_eps", 1e-6)
    w.add("jepa.enc.act", "gelu_erf")
    w.add("jepa.enc.pos_type", "rope3d" if video else "learned")
    if video:
        w.add("jepa.enc.rope_theta", 10000.0)
        w.add("jepa.enc.rope_freq_layout", cfg.rope_layout)
        w.add("jepa.enc.rope_interpolate", cfg.rope_interpolate)
        if cfg.rope_ref_grid:
            w.add("jepa.enc.rope_ref_grid", cfg.rope_ref_grid)
    w.add("jepa.enc.cls_token", cfg.cls_token)
    w.add("jepa.enc.n_registers", cfg.n_registers)
    w.add("jepa.enc.qkv_fused", cfg.qkv_fused)
    w.add("jepa.enc.modality_embed", cfg.modality_embed)
    w.add("jepa.enc.image_patch_embed", cfg.image_patch_embed)
    w.add("jepa.enc.layer_scale", cfg.layer_scale)
    if cfg.attn_mode != "full":
        w.add("jepa.enc.attn_mode", cfg.attn_mode)
    if cfg.pred_dim > 0:
        w.add("jepa.pred.kind", "masked")
        w.add("jepa.pred.embed_dim", cfg.pred_dim)
        w.add("jepa.pred.n_layer", cfg.pred_layers)
        w.add("jepa.pred.n_head", cfg.pred_dim // 32)
        w.add("jepa.pred.ffn_dim", cfg.pred_ffn)
        w.add("jepa.pred.n_mask_tokens", cfg.pred_mask_tokens)
        w.add("jepa.pred.out_dim", D)
        w.add("jepa.pred.rope_freq_layout", cfg.rope_layout)
        w.add("jepa.pred.act", "gelu_erf")
        if cfg.pred_grid:
            w.add("jepa.pred.grid_size", cfg.pred_grid)
        if cfg.modality_embed:
            w.add("jepa.pred.modality_embed", True)
    if cfg.n_classes > 0:
        w.add("jepa.head.kind", "attentive_pool")
        w.add("jepa.head.n_classes", cfg.n_classes)
        w.add("jepa.head.n_pool_layers", cfg.n_pool_layers)
        w.add("jepa.head.labels", [f"class {i}" for i in range(cfg.n_classes)])
    w.add("jepa.pre.mean", [0.485, 0.456, 0.406])
    w.add("jepa.pre.std", [0.229, 0.224, 0.225])
    w.add("jepa.pre.resize_short", cfg.img_size)
    w.add("jepa.pre.crop", cfg.img_size)
    w.add("jepa.pre.resample", "bilinear")
    w.add("jepa.pre.rescale", 1.0 / 255.0)

    def normal(*shape, std=0.02):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    dev_q4k = _device_q4_k() if cfg.ftype == "q4_k" and cfg.embed_dim >= 512 else None

    def mat(name, n_out, n_in, gtype):
        x = normal(n_out, n_in, std=cfg.w_std)
        if gtype == GGML_Q4_K and dev_q4k is not None:
            w.add_tensor(name, gtype, (n_in, n_out), dev_q4k(x))
        else:
            w.add_tensor(name, gtype, (n_in, n_out), quantize(gtype, x))

    def vec(name, n, value=None, std=0.02):
        x = np.full(n, value, dtype=np.float32) if value is not None else normal(n, std=std)
        w.add_tensor(name, GGML_F32, (n,), x)

    def ln(prefix, n=D):
        if cfg.ln_random:
            w.add_tensor(prefix + ".weight", GGML_F32, (n,), (1.0 + normal(n, std=0.1)).astype(np.float32))
            vec(prefix + ".bias", n, std=0.1)
        else:
            vec(prefix + ".weight", n, 1.0)
            vec(prefix + ".bias", n, 0.0)

    patch_type = GGML_F16 if video else GGML_F32
    if cfg.ftype == "f32":
        patch_type = GGML_F32
    kin = 3 * cfg.tubelet * cfg.patch * cfg.patch
    mat("enc.patch_embed.weight", D, kin, patch_type)
    vec("enc.patch_embed.bias", D)
    if cfg.image_patch_embed:
        mat("enc.patch_embed_img.weight", D, 3 * cfg.patch * cfg.patch, patch_type)
        vec("enc.patch_embed_img.bias", D)
    if cfg.modality_embed:
        vec("enc.mod_embed_img", D)
        vec("enc.mod_embed_video", D)
    if cfg.cls_token:
        vec("enc.cls_token", D)
    if cfg.n_registers:
        w.add_tensor("enc.reg_tokens", GGML_F32, (D, cfg.n_registers), normal(cfg.n_registers, D))
    if not video:
        n_tok = (cfg.img_size // cfg.patch) ** 2 + (1 if cfg.cls_token else 0) + cfg.n_registers
        w.add_tensor("enc.pos_embed", GGML_F32, (D, n_tok), normal(n_tok, D))
    def block(p, D=D, F=F):
        ln(p + "ln1", D)
        if cfg.qkv_fused:
            mat(p + "attn_qkv.weight", 3 * D, D, _block_type(cfg, D))
            vec(p + "attn_qkv.bias", 3 * D)
        else:   # the same random draws as the fused matrix, written as its three row blocks
            gt = _block_type(cfg, D)
            parts = cfg.qkv_parts.split(",") if cfg.qkv_parts else [""] * 3
            types = [_QTYPE[q.split("+")[0]] if q else gt for q in parts]
            x = normal(3 * D, D, std=cfg.w_std)
            for j, nm in enumerate("qkv"):
                part = np.ascontiguousarray(x[j * D:(j + 1) * D])
                pt = types[j]
                w.add_tensor(p + f"attn_{nm}.weight", pt, (D, D),
                             dev_q4k(part) if pt == GGML_Q4_K and dev_q4k is not None else quantize(pt, part))
            b = normal(3 * D, std=0.02)
            for j, nm in enumerate("qkv"):
                if not parts[j] or parts[j].endswith("+b"):
                    w.add_tensor(p + f"attn_{nm}.bias", GGML_F32, (D,), np.ascontiguousarray(b[j * D:(j + 1) * D]))
        mat(p + "attn_out.weight", D, D, _block_type(cfg, D))
        vec(p + "attn_out.bias", D)
        ln(p + "ln2", D)
        mat(p + "ffn_up.weight", F, D, _block_type(cfg, D))
        vec(p + "ffn_up.bias", F)
        mat(p + "ffn_down.weight", D, F, _block_type(cfg, F))
        vec(p + "ffn_down.bias", D)
        if cfg.layer_scale:
            vec(p + "ls1", D, std=0.1)
            vec(p + "ls2", D, std=0.1)

    for i in range(cfg.n_layer):
        block(f"enc.blk.{i}.")
    ln("enc.norm")
    if cfg.pred_dim > 0:
        # masked predictor tensors (src/jepa-gguf.cpp:990-1066); pred.embed* / pred.proj / the blocks take
        # the file type (tools/jepa-quantize.cpp:105-116), mask tokens and modality vectors stay f32
        Dp = cfg.pred_dim
        if cfg.pred_mlp_embed:
            mat("pred.embed.0.weight", 4 * Dp, D, _block_type(cfg, D))
            vec("pred.embed.0.bias", 4 * Dp)
            mat("pred.embed.2.weight", Dp, 4 * Dp, _block_type(cfg, 4 * Dp))
            vec("pred.embed.2.bias", Dp)
        else:
            mat("pred.embed.weight", Dp, D, _block_type(cfg, D))
            vec("pred.embed.bias", Dp)
        w.add_tensor("pred.mask_tokens", GGML_F32, (Dp, cfg.pred_mask_tokens), normal(cfg.pred_mask_tokens, Dp, std=1.0))
        if cfg.modality_embed:
            vec("pred.mod_embed_img", Dp, std=0.5)
            vec("pred.mod_embed_video", Dp, std=0.5)
        for i in range(cfg.pred_layers):
            block(f"pred.blk.{i}.", Dp, cfg.pred_ffn)
        ln("pred.norm", Dp)
        mat("pred.proj.weight", D, Dp, _block_type(cfg, Dp))
        vec("pred.proj.bias", D)
    if cfg.n_classes > 0:
        # head tensors (docs/gguf-schema.md:121-137); every head matrix takes the file type
        # (tools/jepa-quantize.cpp:105-116: head.blk.*, head.xattn.*, head.cls.)
        for i in range(cfg.n_pool_layers):
            block(f"head.blk.{i}.")
        w.add_tensor("head.query", GGML_F32, (D, 1), normal(1, D, std=1.0))
        ln("head.xattn.ln_kv")
        for n in ("q", "k", "v"):
            mat(f"head.xattn.{n}.weight", D, D, _block_type(cfg, D))
            vec(f"head.xattn.{n}.bias", D)
        ln("head.xattn.ln2")
        mat("head.xattn.ffn_up.weight", F, D, _block_type(cfg, D))
        vec("head.xattn.ffn_up.bias", F)
        mat("head.xattn.ffn_down.weight", D, F, _block_type(cfg, F))
        vec("head.xattn.ffn_down.bias", D)
        mat("head.cls.weight", cfg.n_classes, D, _block_type(cfg, D))
        vec("head.cls.bias", cfg.n_classes)
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    w.write(path)
    return path


def cached_model(cfg: EncoderConfig, cache_dir: str | None = None) -> str:
    """Path of the synthetic GGUF for cfg, written once per (config, cache dir)."""
    cache_dir = cache_dir or os.environ.get("JEPA_AMD_MODEL_CACHE", "/tmp/jepa_amd_models")
    key = "_".join(str(getattr(cfg, f)) for f in cfg.__dataclass_fields__)
    import hashlib
    h = hashlib.sha1(key.encode()).hexdigest()[:12]
    path = os.path.join(cache_dir, f"{cfg.name}-{cfg.ftype}-{h}.gguf")
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write_model(cfg, tmp)
        os.replace(tmp, path)
    return path
