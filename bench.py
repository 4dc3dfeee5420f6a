#!/usr/bin/env python3
"""Throughput of the V-JEPA 2 ViT-L/16 encoder forward on one MI355X (the reference's headline
jepa-bench configuration: 16 frames of 256x256 = 2048 tokens, 24 layers, q8_0 weights, 1 clip).

One "step" is one encoder forward of one clip through the library's device-resident entry point
(jepa_amd_encode_device: input already in HBM, output left in HBM; the captured hipGraph of the
whole forward is replayed). The timed region is K steps bracketed by torch.cuda.synchronize().

Also reported on the same JSON line:
  roofline      the dominant kernel class (the q8_0 GEMMs): algorithmic int8 ops of one launch (average
                over the four ViT-L shapes) / its mean launch time, from hipEvents recorded around every
                launch on the library's stream during a second pass of K steps; HBM traffic per launch
                from the committed rocprofv3 counter summary when present.
  q4_k          the same workload with q4_K weights.
  configs       the other benchmark configurations measured by default: LeJEPA ViT-S/16 224^2 f16 (1 image,
                CLS + learned positions), V-JEPA 2.1 ViT-B/16 384^2 q8_0 (8 images per call, image path) and
                V-JEPA 2 ViT-g/16 64 frames 256^2 q8_0 (8192 tokens, 40 layers, 1 clip).
  cpu_baseline  the CPU oracle (a C restatement of ggml's CPU semantics, not ggml) on this host's cores:
                the whole 24-block clip, 1 warmup + 3 measured runs, mean (the reference's CPU protocol,
                docs/benchmarks.md:41-53), with the host CPU model and core counts from lscpu.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jepa.cpp_amd", "python"))

METRIC = "clips/s ViT-L 16f q8_0/q4_K on 1 MI355X; GEMM MFMA util %; p50 latency"
# algorithmic work per clip (2 ops per multiply-add): linear GEMMs 2*N*(4D^2 + 2DF)*L, attention 4*N^2*D*L
N_TOK, D, F, L, H = 2048, 1024, 4096, 24, 16
GEMM_OPS = 2 * N_TOK * (4 * D * D + 2 * D * F) * L          # 1.237e12
ATTN_FLOP = 4 * N_TOK * N_TOK * D * L                         # 0.412e12
PATCH_FLOP = 2 * N_TOK * 1536 * D
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 (the q8 GEMMs are priced against it)
PEAK_F16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_model(name):
    from jepa_amd import forge
    t0 = time.time()
    path = forge.cached_model(forge.CONFIGS[name])
    log(f"bench: model {name} ready in {time.time() - t0:.1f} s ({path})")
    return path


def time_forward(path, x_host, steps, warmup, kernel_pass=True):
    import numpy as np
    import torch
    from jepa_amd import _lib

    m = _lib.Model(path, device=0)
    ctx = _lib.Context(m)
    B, C, T, Hh, W = x_host.shape
    rows = m.token_grid(T, Hh, W)
    xin = torch.from_numpy(np.ascontiguousarray(x_host)).to("cuda")
    out = torch.empty((B * rows, m.dim), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    for _ in range(warmup):
        ctx.encode_device(xin.data_ptr(), x_host.shape, out.data_ptr(), out.numel())
    torch.cuda.synchronize()
    per_step = []
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.encode_device(xin.data_ptr(), x_host.shape, out.data_ptr(), out.numel())
        per_step.append(ctx.last_compute_ms)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    res = {"elapsed_s": elapsed, "device_ms": per_step, "rows": rows}
    # wall time of the host-buffer API (jepa_encode: H2D + forward + D2H), the PCIe-inclusive rate
    walls = []
    for _ in range(min(steps, 10)):
        t1 = time.perf_counter()
        ctx.encode(x_host)
        walls.append((time.perf_counter() - t1) * 1e3)
    res["host_api_ms"] = walls
    if kernel_pass:
        ctx.set_kernel_timing(True)
        ctx.reset_kernel_stats()
        for _ in range(steps):
            ctx.encode_device(xin.data_ptr(), x_host.shape, out.data_ptr(), out.numel())
        torch.cuda.synchronize()
        stats = {}
        classes = ["patchify", "patch_embed", "layernorm", "gemm_q8", "gemm_q4_0", "gemm_q4k", "gemm_f16", "attention", "quantize"]
        classes += [f"{g}.{r}" for g in ("gemm_q8", "gemm_q4_0", "gemm_q4k", "gemm_f16") for r in ("qkv", "out", "up", "down")]
        for cls in classes:
            n, ms = ctx.kernel_stats(cls)
            if n:
                stats[cls] = {"launches": n, "total_ms": ms, "avg_ms": ms / n, "per_step_ms": ms / steps}
        res["kernels"] = stats
        ctx.set_kernel_timing(False)
    ctx.close()
    m.close()
    return res


def forward_roofline(cfg, items, frames, rows, ms_per_step):
    """Whole-forward roofline of one step: the time the forward would take at the dense peaks with every
    contraction on its unit and nothing else (linear GEMMs on int8 for block-quantized weights or f16,
    attention and patch embedding on f16), against the measured step. Block-causal attention (LeVJEPA)
    counts its visible keys only (53.1 % of the 3137 x 3137 clip)."""
    d, f, nl = cfg.embed_dim, cfg.ffn_dim, cfg.n_layer
    gemm = 2.0 * rows * (4 * d * d + 2 * d * f) * nl * items
    attn = 4.0 * rows * rows * d * nl * items * (0.531 if cfg.attn_mode == "block_causal" else 1.0)
    pdim = 3 * cfg.patch * cfg.patch * (cfg.tubelet if frames > 1 else 1)   # one frame: the image patch embedding
    patch = 2.0 * rows * pdim * d * items
    gpeak = PEAK_F16_TFLOPS if cfg.ftype == "f16" else PEAK_INT8_TOPS
    t_min = gemm / (gpeak * 1e12) + (attn + patch) / (PEAK_F16_TFLOPS * 1e12)
    return {"t_min_ms": round(t_min * 1e3, 4), "frac": round(t_min * 1e3 / ms_per_step, 4),
            "gemm_op": gemm, "attn_flop": attn, "gemm_peak": gpeak}


# the other encoder configurations: (batch, frames, size) of one step and what one item is
CONFIG_SHAPES = {"vits16_f16": (1, 1, 224, "images"), "vitb16_2_1_q8_0": (8, 1, 384, "images"),
                 "vitg16_q8_0": (1, 64, 256, "clips"), "levjepa_vitl16_q8_0": (1, 16, 224, "clips"),
                 "vitl16_q8_0": (4, 16, 256, "clips")}   # the headline model, 4 clips per call (serving throughput)


def time_config(name, steps, warmup):
    """Rate of one of CONFIG_SHAPES: up to 20 device-resident forwards after a few warm ones."""
    import numpy as np
    from jepa_amd import forge, inputs
    if name not in CONFIG_SHAPES:
        log(f"bench: unknown configuration {name}")
        return None
    b, t, sz, unit = CONFIG_SHAPES[name]
    pc = make_model(name)
    xc = inputs.make_input(b, t, sz, sz, seed=1234)
    log(f"bench: timing {name}")
    st = max(3, min(steps, 20))
    rc = time_forward(pc, xc, st, max(2, min(warmup, 3)), kernel_pass=False)
    mps = rc["elapsed_s"] / st * 1e3
    return {"value": round(b * st / rc["elapsed_s"], 3), "unit": f"{unit}/s", "items_per_step": b,
            "tokens_per_item": rc["rows"], "ms_per_step": round(mps, 4),
            "p50_ms": round(float(np.median(rc["device_ms"])), 4), "steps": st,
            "forward_roofline": forward_roofline(forge.CONFIGS[name], b, t, rc["rows"], mps)}


def time_extra(name, steps):
    """Device time of one call of a row next to the encoder, median over `steps` calls after one warm call."""
    import ctypes as C
    import numpy as np
    import torch
    from jepa_amd import _lib, gguf
    rng = np.random.default_rng(5)
    if name in ("head", "predictor"):
        path = make_model("vitl16_ssv2_q8_0" if name == "head" else "vitl16_pred_q8_0")
        m = _lib.Model(path, device=0)
        ctx = _lib.Context(m)
        enc = rng.standard_normal((2048, 1024)).astype(np.float32)
        ms = []
        if name == "head":
            x = torch.from_numpy(enc).cuda()
            pooled = torch.zeros(1024, device="cuda")
            logits = torch.zeros(m.n_classes, device="cuda")
            torch.cuda.synchronize()
            for i in range(steps + 1):
                ctx.head_device(x.data_ptr(), 2048, pooled.data_ptr(), logits.data_ptr())
                if i:
                    ms.append(ctx.last_compute_ms)
            n_bytes = 2 * 2048 * 1024 * 4
            return {"workload": "V-JEPA 2 ViT-L SSv2 attentive-pool head: 3 pooler blocks over 2048 tokens, cross-attention, "
                                "MLP, 174 classes, q8_0", "p50_ms": round(float(np.median(ms)), 4), "calls": steps,
                    "pool_attention_bytes": n_bytes}
        perm = rng.permutation(2048)
        for i in range(steps + 1):
            ctx.predict(enc, perm[:1024], perm[1024:])
            if i:
                ms.append(ctx.last_compute_ms)
        return {"workload": "V-JEPA 2 ViT-L masked predictor: 12 blocks 384 wide, 12 heads of 32, 1024 context + 1024 "
                            "target rows, q8_0", "p50_ms": round(float(np.median(ms)), 4), "calls": steps}
    if name == "quantizer":
        n = 64 << 20
        x = (torch.randn(n, device="cuda") * 0.02).contiguous()
        out = {}
        for tname, gt in (("q8_0", gguf.GGML_Q8_0), ("q4_k", gguf.GGML_Q4_K)):
            y = torch.empty(gguf.row_bytes(gt, n), dtype=torch.uint8, device="cuda")
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            _lib.lib().jepa_amd_quantize_rows(0, gt, x.data_ptr(), n, y.data_ptr())
            torch.cuda.synchronize()
            ms = []
            for _ in range(max(3, steps // 4)):
                ev0.record()
                _lib.lib().jepa_amd_quantize_rows(0, gt, x.data_ptr(), n, y.data_ptr())
                ev1.record()
                torch.cuda.synchronize()
                ms.append(ev0.elapsed_time(ev1))
            t = float(np.median(ms))
            out[tname] = {"ms_per_64Mi_values": round(t, 3), "Gvalues/s": round(n / (t * 1e-3) / 1e9, 2),
                          "read_GB/s": round(n * 4 / (t * 1e-3) / 1e9, 1)}
        return out
    log(f"bench: unknown extra {name}")
    return None


def step_ceiling():
    """ns per 32x32x32 step of one SIMD for the q8_0 GEMM's inner step from registers alone
    (jepa_amd_gemm_step_probe), and the int8 rate it allows over all SIMDs."""
    import ctypes as C
    from jepa_amd import _lib
    L = _lib.lib()
    simds = 4 * 256
    out = {}
    names = {0: "whole_step", 1: "mfma_half_only", 2: "valu_half_only", 3: "halves_in_separate_waves"}
    for wps in (2, 4):
        for mode in (0, 1, 2, 3):
            ns = C.c_double(0)
            if L.jepa_amd_gemm_step_probe(0, mode, wps, 20000, C.byref(ns)) != 0 or ns.value <= 0:
                log(f"bench: step probe mode {mode} failed: {_lib.error_text()}")
                return None
            tops = 65536.0 / (ns.value * 1e-9) * simds / 1e12
            out[f"{names[mode]}_{wps}_waves_per_simd"] = {"ns_per_step": round(ns.value, 2), "tops": round(tops, 1),
                                                         "frac_of_int8_peak": round(tops / PEAK_INT8_TOPS, 4)}
    return out


def host_cpu():
    """Model name, sockets and physical cores of this host (lscpu), for the CPU baseline's record."""
    import subprocess
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {k.strip(): v.strip() for k, v in (ln.split(":", 1) for ln in out.splitlines() if ":" in ln)}
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info = {"model": kv.get("Model name", ""), "sockets": sockets, "physical_cores": sockets * per,
                "logical_cpus": int(kv.get("CPU(s)", "0") or 0)}
    except Exception as e:          # lscpu missing: report what Python knows
        info = {"model": "", "error": str(e)}
    info["affinity_cpus"] = len(os.sched_getaffinity(0))
    return info


def cpu_baseline(path, x_host):
    """The oracle on the host cores, the reference's CPU protocol: one ViT-L/16 16f q8_0 clip through all
    24 blocks, 1 warmup + 3 measured runs, mean. The thread count is the CPU share this process is given
    ($OMP_NUM_THREADS, capped by its affinity), not the whole host."""
    from oracle import oracle as O
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    threads = int(os.environ.get("ORACLE_THREADS", min(share, len(os.sched_getaffinity(0)))))
    os.environ["ORACLE_THREADS"] = str(threads)
    O.build()
    runs = []
    for i in range(4):
        t0 = time.perf_counter()
        O.encode(path, x_host, 1, N_TOK, D)
        runs.append(time.perf_counter() - t0)
        log(f"bench: CPU baseline run {i} ({'warmup' if i == 0 else 'measured'}): {runs[-1]:.2f} s")
    mean_s = sum(runs[1:]) / 3
    return {"value": round(1.0 / mean_s, 5), "unit": "clips/s", "cores": threads, "kind": "port",
            "ms_per_clip": round(mean_s * 1e3, 1), "runs_s": [round(t, 3) for t in runs], "host": host_cpu(),
            "sample": f"oracle (C restatement of ggml's CPU semantics, not ggml; OpenMP, {threads} threads) on one whole "
                      f"ViT-L/16 16f q8_0 clip (2048 tokens, 24 blocks): 1 warmup + 3 measured, mean {mean_s:.2f} s/clip",
            "published_reference": "jepa-bench (ggml CPU) 794.1 ms/clip = 1.26 clips/s on a 96-core Threadripper PRO 7995WX at "
                                   "32 threads (reference docs/benchmarks.md:103)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-q4k", action="store_true", help="skip the q4_K line")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--configs", default="vits16_f16,vitb16_2_1_q8_0,vitg16_q8_0",
                    help="also time these encoder configurations (comma list; default: vits16_f16, vitb16_2_1_q8_0, "
                         "vitg16_q8_0; also levjepa_vitl16_q8_0, vitl16_q8_0 = the headline model with 4 clips per call; "
                         "'' for none)")
    ap.add_argument("--extras", default="",
                    help="also time the rows next to the encoder (comma list: head = ViT-L SSv2 attentive-pool head on "
                         "2048 tokens; predictor = ViT-L masked predictor, 1024 context + 1024 target rows; quantizer = "
                         "the q8_0 / q4_K block quantizers over 64 Mi weights)")
    ap.add_argument("--configs-only", action="store_true",
                    help="time only the --configs configurations (no headline line; for per-configuration profiles)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run the library's plain copy kernel over this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the encoder has no multi-GPU path; clips are "
              "independent, so N GPUs would run N independent replicas). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from jepa_amd import forge, inputs

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.configs_only:
        res = {}
        for name in [c for c in args.configs.split(",") if c]:
            res[name] = time_config(name, args.steps, args.warmup)
        print(json.dumps({"configs": res}), flush=True)
        return
    x = inputs.make_input(1, 16, 256, 256, seed=1234)          # jepa-bench's seeded pixels
    path = make_model("vitl16_q8_0")
    log("bench: timing q8_0")
    r = time_forward(path, x, args.steps, args.warmup)
    dev_ms = np.array(r["device_ms"])
    ms_per_step = r["elapsed_s"] / args.steps * 1e3
    value = args.steps / r["elapsed_s"]
    k = r.get("kernels", {})
    gq = k.get("gemm_q8")
    roof = None
    if gq:
        launches_per_clip = gq["launches"] / args.steps
        ops_per_launch = GEMM_OPS / launches_per_clip
        achieved = ops_per_launch / (gq["avg_ms"] * 1e-3) / 1e12
        traffic = None
        tf = os.path.join(ROOT, "profiles", "gemm_q8_vitl16_counters.json")
        if os.path.exists(tf):
            with open(tf) as f:
                traffic = json.load(f).get("hbm_bytes_per_launch")    # rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic,
                "kernel": "gemm_q8 (q8_0 x q8_0 GEMMs: qkv, out, fc1, fc2)", "avg_launch_ms": round(gq["avg_ms"], 5),
                "ops_per_launch": ops_per_launch, "peak_note": "int8 dense 5.0 POP/s; block sums on v_mfma_i32_32x32x32_i8, per-32-block f32 scale epilogue on the VALU"}
    extra = {}
    # the ceiling of the q8_0 GEMM's arithmetic on this chip: its inner step (int8 MFMA block sum, f16
    # scale-product MFMA, 16 conversions + 16 fmas) timed from registers alone, whole step per wave
    # (the kernels' form) and split into MFMA-only and VALU-only waves (overlap across waves)
    ceil = step_ceiling()
    if ceil and roof:
        best = ceil["whole_step_2_waves_per_simd"]
        roof["step_ceiling_tops"] = best["tops"]
        roof["frac_of_step_ceiling"] = round(roof["achieved"] / best["tops"], 4)
        extra["gemm_step_ceiling"] = ceil
    att = k.get("attention")
    if att:
        extra["attention_roofline"] = {"bound": "mfma", "achieved": round(ATTN_FLOP / (att["per_step_ms"] * 1e-3) / 1e12, 2),
                                       "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(ATTN_FLOP / (att["per_step_ms"] * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
                                       "avg_launch_ms": round(att["avg_ms"], 5)}
    extra["kernel_ms_per_clip"] = {c: round(v["per_step_ms"], 4) for c, v in k.items()}
    extra["forward_roofline"] = forward_roofline(forge.CONFIGS["vitl16_q8_0"], 1, 16, N_TOK, ms_per_step)
    if not args.no_q4k:
        p4 = make_model("vitl16_q4_k")
        log("bench: timing q4_K")
        r4 = time_forward(p4, x, args.steps, args.warmup, kernel_pass=True)
        g4 = r4.get("kernels", {}).get("gemm_q4k")
        q4 = {"value": round(args.steps / r4["elapsed_s"], 3), "unit": "clips/s",
              "ms_per_step": round(r4["elapsed_s"] / args.steps * 1e3, 4),
              "p50_ms": round(float(np.median(r4["device_ms"])), 4)}
        if g4:
            ach = GEMM_OPS / (g4["per_step_ms"] * 1e-3) / 1e12
            q4["gemm_roofline"] = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                                   "frac": round(ach / PEAK_INT8_TOPS, 4)}
        q4["forward_roofline"] = forward_roofline(forge.CONFIGS["vitl16_q4_k"], 1, 16, N_TOK, q4["ms_per_step"])
        extra["q4_k"] = q4
    for name in [c for c in args.configs.split(",") if c]:
        r_c = time_config(name, args.steps, args.warmup)
        if r_c is not None:
            extra.setdefault("configs", {})[name] = r_c
    for name in [e for e in args.extras.split(",") if e]:
        res = time_extra(name, max(5, min(args.steps, 20)))
        if res is not None:
            extra.setdefault("extras", {})[name] = res
    if args.copy_mib > 0:
        # a copy of known size: FETCH_SIZE / WRITE_SIZE of k_copy_f32 calibrate the counters
        import ctypes as C
        from jepa_amd import _lib
        n = args.copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        ms = C.c_double(0)
        _lib.lib().jepa_amd_copy(0, src.data_ptr(), dst.data_ptr(), n, 3, C.byref(ms))
        extra["copy_calibration"] = {"bytes_read": n * 4, "bytes_written": n * 4, "ms": round(ms.value, 4),
                                     "GB/s": round(2 * n * 4 / (ms.value * 1e-3) / 1e9, 1)}
    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline (oracle)")
        cpu = cpu_baseline(path, x)
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "clips/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "dtype_note": "q8_0 weight and activation codes on int8 MFMA (exact int32 block sums), f32 per-block scale "
                      "epilogue and residual stream, f16 attention operands",
        "data": "synthetic (jepa-bench seeded pixels, random-init N(0,0.02) weights)",
        "config": {"workload": "V-JEPA 2 ViT-L/16 encoder, 16 frames 256x256 (2048 tokens), 24 layers, D 1024, 16 heads, "
                               "q8_0, batch 1 clip, device-resident input/output", "global_batch": 1, "seq_len": N_TOK,
                   "parallelism": "single GPU"},
        "p50_ms": round(float(np.median(dev_ms)), 4), "mean_ms": round(float(dev_ms.mean()), 4),
        "min_ms": round(float(dev_ms.min()), 4),
        "host_api_p50_ms": round(float(np.median(r["host_api_ms"])), 4),
        "roofline": roof, "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
