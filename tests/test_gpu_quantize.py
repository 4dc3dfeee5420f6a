"""The GGUF quantizer (jepa_amd_quantize_file, the reference's tools/jepa-quantize.cpp) and its block
quantizer kernels, on the GPU, against the oracle's restatement of ggml's reference quantizers
(quantize_row_q8_0_ref / q4_0_ref / q4_K_ref with make_qkx2_quants): bytes must be equal.
"""
import os

import numpy as np
import pytest

from jepa_amd import forge, gguf

pytestmark = pytest.mark.gpu


def _rows():
    """random rows plus blocks that reach the quantizers' special cases"""
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((24, 512)) * 0.05).astype(np.float32)
    x[0] = 0.0                                           # zero blocks: d = 0
    x[1] = 0.25                                          # constant blocks: max == min
    x[2, :256] = np.abs(x[2, :256])                      # all positive: the fit's min clamps to 0
    x[3] = -np.abs(x[3])                                 # all negative
    x[4, 7] = 3.0                                        # one outlier per block
    x[5] = np.tile(np.arange(16, dtype=np.float32) * 0.01 - 0.05, 32)   # values on a 16-level grid
    x[6] *= 1e-6                                         # tiny values (f16 scales near subnormal)
    x[7, 100:140] = -x[7, 100:140] * 40                  # large negative runs
    return x


@pytest.mark.parametrize("gtype", [gguf.GGML_Q8_0, gguf.GGML_Q4_0, gguf.GGML_Q4_K, gguf.GGML_F16])
def test_quantize_rows_bit_exact(jlib, oracle, gtype):
    import torch
    x = _rows()
    dx = torch.from_numpy(x).cuda()
    nbytes = gguf.row_bytes(gtype, x.shape[1]) * x.shape[0]
    out = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    assert jlib.lib().jepa_amd_quantize_rows(0, gtype, dx.data_ptr(), x.size, out.data_ptr()) == 0, jlib.error_text()
    got = out.cpu().numpy()
    if gtype == gguf.GGML_F16:
        want = x.astype(np.float16).view(np.uint8).reshape(-1)
    else:
        want = oracle.quantize_weight(gtype, x).reshape(-1)
    np.testing.assert_array_equal(got, want)
    if gtype == gguf.GGML_Q4_K:   # the numpy restatement agrees too
        np.testing.assert_array_equal(got, gguf.quantize_q4_K(x).reshape(-1))


def _f32_model(models_dir):
    cfg = forge.tiny("vjepa2", "f32", n_classes=10, n_pool_layers=1, pred_dim=128, pred_layers=1, pred_ffn=512)
    return cfg, forge.cached_model(cfg, models_dir)


def _expected_type(name, n_dims, ne0, target):
    rule = (n_dims == 2 and name.endswith(".weight") and "patch_embed" not in name and "pos_embed" not in name
            and "mask_tokens" not in name and ".norm." not in name and "ln_kv" not in name and "head.query" not in name
            and any(c in name for c in (".attn_qkv.", ".attn_out.", ".ffn_up.", ".ffn_down.", "pred.proj", "pred.embed",
                                         "head.cls.", "head.xattn.")))
    if not rule:
        return None
    if target == gguf.GGML_Q4_K and ne0 % 256:
        return gguf.GGML_Q4_0
    return target


@pytest.mark.parametrize("qtype,gtype", [("q8_0", gguf.GGML_Q8_0), ("q4_0", gguf.GGML_Q4_0), ("q4_k", gguf.GGML_Q4_K),
                                         ("f16", gguf.GGML_F16)])
def test_quantize_file(jlib, oracle, models_dir, tmp_path, qtype, gtype):
    """f32 model with encoder, head and predictor -> `qtype`: metadata copied in order with general.file_type
    replaced, the rule's matrices re-typed (q4_k: 128-wide rows fall back to q4_0) with the oracle's bytes,
    every other tensor byte-identical; the file loads and encodes."""
    cfg, src = _f32_model(models_dir)
    dst = str(tmp_path / f"out-{qtype}.gguf")
    jlib.quantize_file(src, dst, qtype)
    a, b = gguf.read_gguf(src), gguf.read_gguf(dst)
    keys_a = [k for k in a.kv.keys() if k != "general.file_type"]
    assert keys_a == [k for k in b.kv.keys() if k != "general.file_type"]
    for k, v in a.kv.items():
        if k != "general.file_type":
            assert b.kv[k] == v, k
    assert list(a.tensors.keys()) == list(b.tensors.keys())
    n_q = {}
    for name, ti in a.tensors.items():
        ty, ne, bty = ti.gtype, ti.ne, b.tensors[name].gtype
        want = _expected_type(name, len(ne), ne[0], gtype)
        src_bytes = a.tensor_bytes(name)
        if want is None:
            assert bty == ty, name
            np.testing.assert_array_equal(b.tensor_bytes(name), src_bytes)
            continue
        assert bty == want, (name, bty, want)
        n_q[want] = n_q.get(want, 0) + 1
        x = a.tensor_f32(name).reshape(-1, ne[0])
        if want == gguf.GGML_F16:
            exp = x.astype(np.float16).view(np.uint8).reshape(-1)
        else:
            exp = oracle.quantize_weight(want, x).reshape(-1)
        np.testing.assert_array_equal(b.tensor_bytes(name).reshape(-1), exp)
    ft = b.kv["general.file_type"]
    major = max(n_q, key=n_q.get)
    expected_ft = {gguf.GGML_Q8_0: 7, gguf.GGML_Q4_0: 2, gguf.GGML_Q4_K: 12, gguf.GGML_F16: 1}[major if gtype == gguf.GGML_Q4_K else gtype]
    assert ft == expected_ft, (ft, n_q)
    if gtype == gguf.GGML_Q4_K and major != gtype:      # the majority rule moves the key to the end
        assert list(b.kv.keys())[-1] == "general.file_type"
    # the quantized file is a working model
    m = jlib.Model(dst)
    ctx = jlib.Context(m)
    from jepa_amd import inputs
    y = ctx.encode(inputs.make_input(1, 4, 64, 64, seed=3))
    assert y.shape == (32, cfg.embed_dim) and np.isfinite(y).all()


def test_quantize_file_widen_keep_and_errors(jlib, models_dir, tmp_path):
    cfg, src = _f32_model(models_dir)
    q8 = str(tmp_path / "q8.gguf")
    jlib.quantize_file(src, q8, "q8_0", keep=["ffn_down"])
    b = gguf.read_gguf(q8)
    assert b.tensors["enc.blk.0.ffn_down.weight"].gtype == gguf.GGML_F32
    assert b.tensors["enc.blk.0.ffn_up.weight"].gtype == gguf.GGML_Q8_0
    # f32 widens (dequantizes) every tensor
    back = str(tmp_path / "back.gguf")
    jlib.quantize_file(q8, back, "f32")
    c = gguf.read_gguf(back)
    assert all(t.gtype == gguf.GGML_F32 for t in c.tensors.values()) and c.kv["general.file_type"] == 0
    np.testing.assert_array_equal(c.tensor_f32("enc.blk.0.ffn_up.weight"), b.tensor_f32("enc.blk.0.ffn_up.weight"))
    # re-quantizing needs the flag; with it, the source is dequantized first
    with pytest.raises(RuntimeError, match="needs allow_requant"):
        jlib.quantize_file(q8, str(tmp_path / "q4.gguf"), "q4_0")
    jlib.quantize_file(q8, str(tmp_path / "q4.gguf"), "q4_0", allow_requant=True)
    with pytest.raises(RuntimeError, match="does not write type 'q5_k'"):
        jlib.quantize_file(src, str(tmp_path / "x.gguf"), "q5_k")
    with pytest.raises(RuntimeError, match="IN and OUT must differ"):
        jlib.quantize_file(src, src, "q8_0")
    assert not os.path.exists(str(tmp_path / "x.gguf"))
