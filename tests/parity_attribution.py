"""Attribution of the full-size encoders' end-to-end distance to its sources, on the CPU oracle alone.

For each benchmark model the oracle's forward with the reference's CPU arithmetic is compared with the
oracle's forward after one change at a time: each of the GPU kernels' roundings (oracle.ROUND_*: f16 q
before Q.K^T, f16 softmax weights before P.V, the exp2 form of the softmax, the GPU's erf polynomial),
all four together, the per-block float sums taken in the reverse K order (another valid summation
order, no GPU rounding at all), and the quantized dots summed in ggml's own x86 lane order (AVX2
vec_dot / llamafile tinyBLAS: eight float lanes of four consecutive products per output, the q4_K mins
in four lanes, horizontal sums at the end; oracle.set_ggml_lanes). The token cosine (mean and min) and
the final residual-stream rel_max of each against the reference arithmetic show how far each source
alone carries a 12-24 layer quantized encoder.

    python tests/parity_attribution.py [model ...]     (models: vitl16_q8_0 vitl16_q4_k vitb16_2_1_q8_0 levjepa_vitl16_q8_0 vith14_ijepa_q8_0)
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "jepa.cpp_amd", "python"))
sys.path.insert(0, ROOT)

from jepa_amd import forge, inputs  # noqa: E402
from oracle import oracle as O  # noqa: E402

# (n_batch, n_frames, size, rows per item), as the GPU parity tests run them
FULL = {
    "vitl16_q8_0": (1, 16, 256, 2048),
    "vitl16_q4_k": (1, 16, 256, 2048),
    "vitb16_2_1_q8_0": (8, 1, 384, 576),
    "levjepa_vitl16_q8_0": (1, 16, 224, 3137),
    "vith14_ijepa_q8_0": (1, 1, 224, 256),
}
# (label, rounding bits, reversed block order, ggml lane order)
CASES = [("f16 q", O.ROUND_Q16, False, False), ("f16 softmax weights", O.ROUND_P16, False, False),
         ("exp2 softmax", O.ROUND_EXP2, False, False), ("erf polynomial", O.ROUND_GELU, False, False),
         ("all four GPU roundings", O.ROUND_GPU, False, False), ("reversed block order", 0, True, False),
         ("ggml x86 lane order", 0, False, True)]


def cos_rows(a, b):
    a = a.astype(np.float64); b = b.astype(np.float64)
    return (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1) + 1e-300)


def main(names):
    O.build()
    cache = os.environ.get("JEPA_AMD_MODEL_CACHE")
    for name in names:
        n_batch, n_frames, size, rows = FULL[name]
        cfg = forge.CONFIGS[name]
        path = forge.cached_model(cfg, cache)
        video = cfg.family in ("vjepa2", "vjepa2_1", "levjepa")
        n_items = n_batch if (video and n_frames > 1) else n_batch * n_frames
        x = inputs.make_input(n_batch, n_frames, size, size, seed=1234)
        O.set_rounding(0); O.set_reverse_block_order(False)
        t0 = time.time()
        ref, _ = O.encode(path, x, n_items, rows, cfg.embed_dim)
        print(f"{name}: reference arithmetic in {time.time() - t0:.1f} s", flush=True)
        only = os.environ.get("ATTRIBUTION_CASES")
        for label, bits, rev, lanes in CASES:
            if only and label not in only.split(","):
                continue
            O.set_rounding(bits); O.set_reverse_block_order(rev); O.set_ggml_lanes(lanes)
            try:
                got, _ = O.encode(path, x, n_items, rows, cfg.embed_dim)
            finally:
                O.set_rounding(0); O.set_reverse_block_order(False); O.set_ggml_lanes(False)
            c = cos_rows(got, ref)
            rel = float(np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max())
            print(f"| {name} | {label} | {c.mean():.7f} | {c.min():.6f} | {rel:.2e} |", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(FULL))
