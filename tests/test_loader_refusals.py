"""The GGUF loader's refusals by name (reference src/jepa-gguf.cpp:240-250, 942-1092; tests/test-errors.cpp):
a valid tiny model is rewritten with one key or tensor broken, and jepa_model_load_ex must return NULL with
a message naming what is wrong. Metadata refusals happen before any device work and run on the CPU; the
tensor refusals need the device the weights are uploaded to."""
import numpy as np
import pytest

from jepa_amd import _lib, forge, gguf


def rewrite(src, dst, kv=None, drop=(), tensors=None):
    """Copy GGUF `src` to `dst` with keys replaced or removed (value None) and tensors dropped or replaced
    (name -> (gtype, ne, data))."""
    g = gguf.read_gguf(src)
    w = gguf.GGUFWriter()
    kv = kv or {}
    for k, v in g.kv.items():
        if k in kv:
            if kv[k] is not None:
                w.add(k, kv[k])
        else:
            w.add(k, v)
    for k, v in kv.items():
        if k not in g.kv and v is not None:
            w.add(k, v)
    tensors = tensors or {}
    for name, t in g.tensors.items():
        if name in drop:
            continue
        if name in tensors:
            gt, ne, data = tensors[name]
            w.add_tensor(name, gt, ne, data)
        else:
            w.add_tensor(name, t.gtype, t.ne, np.asarray(t.data))
    for name, (gt, ne, data) in tensors.items():
        if name not in g.tensors:
            w.add_tensor(name, gt, ne, data)
    w.write(dst)
    return dst


def refused(path):
    L = _lib.lib()
    L.jepa_error_reset()
    p = _lib.ModelParams(False, 0)
    ptr = L.jepa_model_load_ex(path.encode(), p)
    if ptr:
        L.jepa_model_free(ptr)
        return None
    return _lib.error_text()


@pytest.fixture(scope="module")
def base(tmp_path_factory):
    d = tmp_path_factory.mktemp("refusals")
    return str(d), forge.cached_model(forge.tiny("vjepa2", "q8_0"), str(d)), forge.cached_model(forge.tiny("hfvit", "f16"), str(d))


METADATA = [
    ("unknown family", dict(kv={"jepa.family": "vjepa9"}), "unknown jepa.family"),
    ("wrong architecture", dict(kv={"general.architecture": "llama"}), "general.architecture"),
    ("missing embed_dim", dict(kv={"jepa.enc.embed_dim": None}), "missing required key jepa.enc.embed_dim"),
    ("layers out of range", dict(kv={"jepa.enc.n_layer": 100000}), "out of range"),
    ("unknown attention mode", dict(kv={"jepa.enc.attn_mode": "sliding"}), "unknown jepa.enc.attn_mode"),
    ("heads do not divide D", dict(kv={"jepa.enc.n_head": 3}), "not divisible by n_head"),
    ("interpolation without a grid", dict(kv={"jepa.enc.rope_interpolate": True, "jepa.enc.rope_ref_grid": 0}),
     "rope_ref_grid"),
    ("unknown activation", dict(kv={"jepa.enc.act": "swish9"}), "unknown activation"),
]


@pytest.mark.parametrize("label,change,message", METADATA, ids=[m[0] for m in METADATA])
def test_metadata_refusals(base, label, change, message):
    d, video, _ = base
    path = rewrite(video, f"{d}/bad_{label.replace(' ', '_')}.gguf", **change)
    err = refused(path)
    assert err is not None and message in err, (label, err)


def test_block_causal_needs_a_video_family(base):
    d, _, image = base
    err = refused(rewrite(image, f"{d}/bad_causal_image.gguf", kv={"jepa.enc.attn_mode": "block_causal"}))
    assert err is not None and "only defined for the video families" in err, err


@pytest.mark.gpu
def test_tensor_refusals(base):
    d, video, image = base
    g = gguf.read_gguf(video)
    D = g.kv["jepa.enc.embed_dim"]
    qkv = g.tensors["enc.blk.0.attn_qkv.weight"]
    cases = [
        ("missing block tensor", video, dict(drop={"enc.blk.1.ffn_up.weight"}), "enc.blk.1.* is incomplete"),
        ("qkv weight of an unsupported type", video,
         dict(tensors={"enc.blk.0.attn_qkv.weight": (gguf.GGML_BF16, qkv.ne, np.zeros(qkv.ne[0] * qkv.ne[1], np.uint16))}),
         "no GEMM kernel for"),
        ("LayerNorm weight stored f16", video,
         dict(tensors={"enc.blk.0.ln1.weight": (gguf.GGML_F16, (D,), np.ones(D, np.float16))}), "has to be f32"),
        ("registers without their tensor", video, dict(kv={"jepa.enc.n_registers": 2}), "enc.reg_tokens is missing"),
        ("registers of the wrong count", video,
         dict(kv={"jepa.enc.n_registers": 2}, tensors={"enc.reg_tokens": (gguf.GGML_F32, (D, 3), np.zeros((3, D), np.float32))}),
         "enc.reg_tokens is a different shape"),
        ("CLS flag without the CLS tensor", image, dict(drop={"enc.cls_token"}), "enc.cls_token missing"),
        ("position table of the wrong width", image,
         dict(tensors={"enc.pos_embed": (gguf.GGML_F32, (D + 1, 17), np.zeros((17, D + 1), np.float32))}), "enc.pos_embed has rows of"),
    ]
    for label, src, change, message in cases:
        err = refused(rewrite(src, f"{d}/bad_{label.replace(' ', '_')}.gguf", **change))
        assert err is not None and message in err, (label, err)
    # and the unmodified copies load
    assert refused(rewrite(video, f"{d}/copy_video.gguf")) is None
    assert refused(rewrite(image, f"{d}/copy_image.gguf")) is None
