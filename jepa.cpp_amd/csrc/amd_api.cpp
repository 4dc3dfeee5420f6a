// amd_api.cpp - entry points of include/jepa_amd.h (device-resident encode, kernel timing, single-kernel hooks).
#include "../../include/jepa_amd.h"
#include "model.h"
#include "kernels.h"
#include "preprocess.h"
#include "rope3d.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

// scoped device + stream for the synchronous hooks
struct dev_scope {
    int prev = 0;
    hipStream_t s = nullptr;
    bool ok = false;
    std::vector<void *> allocs;
    explicit dev_scope(int device) {
        hipGetDevice(&prev);
        if (!dev_check(device)) return;
        if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
            jepa_log("jepa: cannot use HIP device %d\n", device);
            return;
        }
        ok = true;
    }
    void * alloc(size_t bytes) {
        std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
        void * p = nullptr;
        if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) { jepa_log("jepa: hipMalloc(%zu) failed\n", bytes); return nullptr; }
        allocs.push_back(p);
        return p;
    }
    int finish() {
        const hipError_t e = hipStreamSynchronize(s);
        const hipError_t l = hipGetLastError();
        if (e != hipSuccess || l != hipSuccess) {
            jepa_log("jepa: kernel failed: %s\n", hipGetErrorString(e != hipSuccess ? e : l));
            return -1;
        }
        return 0;
    }
    ~dev_scope() {
        if (s) hipStreamSynchronize(s);
        std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
        for (void * p : allocs) hipFree(p);
        if (s) hipStreamDestroy(s);
        hipSetDevice(prev);
    }
};

// split-K scratch for n_rows-row GEMMs, counters zeroed
bool alloc_split(dev_scope & d, gemm_split_ws & sw, int64_t n_rows) {
    gemm_split_ws_size(n_rows, &sw.part_floats, &sw.cnt_n);
    sw.part = (float *) d.alloc((size_t) sw.part_floats * 4);
    sw.cnt = (int *) d.alloc((size_t) sw.cnt_n * 4);
    if (!sw.part || !sw.cnt) return false;
    launch_fill_zero(sw.cnt, (size_t) sw.cnt_n * 4, d.s);
    return true;
}

bool alloc_act(dev_scope & d, act_view & a, int fmt, int64_t M, int64_t K) {
    a.fmt = fmt;
    a.ld = K;
    a.q = d.alloc((size_t) M * K * 4);
    a.d = d.alloc((size_t) M * (K / 32) * 4 + 16);
    a.bsum = d.alloc((size_t) M * (K / 16) * 2 + 16);
    return a.q && a.d && a.bsum;
}

}  // namespace

extern "C" int64_t jepa_amd_encode_device(jepa_context * ctx, const float * in_dev, int n_batch, int n_chans, int n_frames,
                                          int height, int width, float * out_dev, int64_t out_cap) {
    if (!ctx || !in_dev || !out_dev) return -1;
    return encode_device(ctx, in_dev, n_batch, n_chans, n_frames, height, width, out_dev, out_cap, nullptr, 0);
}

extern "C" int jepa_amd_head_device(jepa_context * ctx, const float * x_dev, int64_t n_tokens, float * pooled_dev, float * logits_dev) {
    if (!ctx || !x_dev) return -1;
    return head_device(ctx, x_dev, n_tokens, pooled_dev, logits_dev);
}

extern "C" int64_t jepa_amd_encode_trace(jepa_context * ctx, const jepa_input * in, float * out, int64_t out_cap, float * trace,
                                         int64_t trace_cap) {
    if (!ctx || !in || !in->data || !out || !trace) return -1;
    jepa_model * m = ctx->model;
    int64_t n_items = 0;
    const int64_t R = encode_rows(m, in->n_batch, in->n_frames, in->height, in->width, &n_items);
    if (R <= 0) { jepa_log("jepa: input shape is not encodable by this model\n"); return -1; }
    const int64_t D = m->hp.enc.embed_dim, L = m->hp.enc.n_layer;
    if (out_cap < n_items * R * D || trace_cap < n_items * (L + 1) * R * D) { jepa_log("jepa: output / trace buffer too small\n"); return -1; }
    dev_scope d(ctx->device);
    if (!d.ok) return -1;
    const size_t n_in = (size_t) in->n_batch * in->n_chans * in->n_frames * in->height * in->width;
    float * din = (float *) d.alloc(n_in * 4);
    float * dout = (float *) d.alloc((size_t) n_items * R * D * 4);
    float * dtr = (float *) d.alloc((size_t) n_items * (L + 1) * R * D * 4);
    if (!din || !dout || !dtr) return -1;
    if (hipMemcpyAsync(din, in->data, n_in * 4, hipMemcpyHostToDevice, d.s) != hipSuccess || hipStreamSynchronize(d.s) != hipSuccess) return -1;
    const int64_t r = encode_device(ctx, din, in->n_batch, in->n_chans, in->n_frames, in->height, in->width, dout, n_items * R * D, dtr,
                                    n_items * (L + 1) * R * D);
    if (r < 0) return -1;
    // device trace is [layer][all rows]; the caller wants [item][layer][rows]
    std::vector<float> tmp((size_t) (L + 1) * n_items * R * D);
    if (hipMemcpyAsync(tmp.data(), dtr, tmp.size() * 4, hipMemcpyDeviceToHost, d.s) != hipSuccess ||
        hipMemcpyAsync(out, dout, (size_t) n_items * R * D * 4, hipMemcpyDeviceToHost, d.s) != hipSuccess ||
        hipStreamSynchronize(d.s) != hipSuccess)
        return -1;
    for (int64_t it = 0; it < n_items; it++)
        for (int64_t l = 0; l <= L; l++)
            memcpy(trace + ((it * (L + 1) + l) * R) * D, tmp.data() + ((l * n_items + it) * R) * D, (size_t) R * D * 4);
    return r;
}

extern "C" void jepa_amd_context_set_kernel_timing(jepa_context * ctx, bool on) { if (ctx) ctx->kernel_timing = on; }
extern "C" int jepa_amd_context_kernel_stats(const jepa_context * ctx, const char * cls, int64_t * n, double * ms) {
    if (!ctx || !cls) return -1;
    auto it = ctx->kstats.find(cls);
    if (n) *n = it == ctx->kstats.end() ? 0 : it->second.first;
    if (ms) *ms = it == ctx->kstats.end() ? 0.0 : it->second.second;
    return 0;
}
extern "C" void jepa_amd_context_reset_kernel_stats(jepa_context * ctx) { if (ctx) ctx->kstats.clear(); }
extern "C" void jepa_amd_context_set_graph(jepa_context * ctx, bool on) { if (ctx) ctx->use_graph = on; }
extern "C" void * jepa_amd_context_stream(const jepa_context * ctx) { return ctx ? (void *) ctx->stream : nullptr; }

extern "C" int jepa_amd_dequantize(int device, int gtype, const void * blocks, int64_t n_rows, int64_t n_cols, float * y) {
    if (!blocks || !y || n_rows <= 0 || n_cols <= 0) return -1;
    const type_traits tt = ggml_traits(gtype);
    if (!(gtype == T_Q8_0 || gtype == T_Q4_0 || gtype == T_Q4_K || gtype == T_F16 || gtype == T_F32) || n_cols % tt.blck) {
        jepa_log("jepa: jepa_amd_dequantize: type %d / %lld columns not supported\n", gtype, (long long) n_cols);
        return -1;
    }
    dev_scope d(device);
    if (!d.ok) return -1;
    launch_dequant_rows(gtype, blocks, n_rows, n_cols, y, d.s);
    return d.finish();
}

extern "C" int jepa_amd_rownorm(int device, const float * x, int64_t n_rows, int64_t n_cols, const float * w, const float * b, float eps,
                                int normalize, int out_type, void * out) {
    if (!x || !out || n_rows <= 0 || n_cols <= 0 || n_cols % 8 || n_cols > 2048) {
        jepa_log("jepa: jepa_amd_rownorm: bad arguments (rows of %lld; 8 | cols <= 2048)\n", (long long) n_cols);
        return -1;
    }
    int fmt;
    switch (out_type) {
        case T_F32: fmt = A_F32; break;
        case T_F16: fmt = A_F16; break;
        case T_Q8_0: fmt = A_Q8_0; if (n_cols % 32) return -1; break;
        case T_Q8_K: fmt = A_Q8_K; if (n_cols % 256) return -1; break;
        default: jepa_log("jepa: jepa_amd_rownorm: output type %d not supported\n", out_type); return -1;
    }
    dev_scope d(device);
    if (!d.ok) return -1;
    act_view a;
    if (fmt == A_F32 || fmt == A_F16) { a.fmt = fmt; a.q = out; a.ld = n_cols; }
    else if (!alloc_act(d, a, fmt, n_rows, n_cols)) return -1;
    launch_rownorm_quant(x, n_rows, n_cols, w, b, eps, normalize != 0, a, d.s);
    if (fmt == A_Q8_0 || fmt == A_Q8_K) launch_pack_act_blocks(a, n_rows, n_cols, out, d.s);
    return d.finish();
}

namespace {

// a dev_linear over ggml weight blocks in device memory (repacked into the GEMM's operand layout)
bool make_linear(dev_scope & d, const char * who, int wtype, const void * w, int64_t n_out, int64_t n_in, const float * bias,
                 dev_linear & L) {
    L.gtype = wtype; L.n_out = n_out; L.n_in = n_in; L.bias = (float *) bias;
    L.fmt = weight_format(wtype, n_in);
    if (L.fmt < 0) { jepa_log("jepa: %s: weight type %d not supported\n", who, wtype); return false; }
    if (L.fmt != W_F32 && (n_out % 128 || n_in % 64 || (L.fmt == W_Q4K && n_in % 256) || n_in > 2048 * 8)) {
        jepa_log("jepa: %s: [%lld x %lld] not supported by the MFMA GEMM (n_out %% 128, n_in %% 64)\n", who, (long long) n_out,
                 (long long) n_in);
        return false;
    }
    if (L.fmt == W_F32 || L.fmt == W_F16) {
        L.w = (void *) w;
        return true;
    }
    L.w = d.alloc(weight_code_bytes(L.fmt, n_out, n_in));
    if (L.fmt == W_Q32 || L.fmt == W_Q40) L.wd = d.alloc((size_t) n_out * (n_in / 32) * 2);
    else {
        L.wd = d.alloc((size_t) n_out * (n_in / 256) * 4);
        L.wmin = d.alloc((size_t) n_out * (n_in / 256) * 32);
    }
    if (!L.w || !L.wd || (L.fmt == W_Q4K && !L.wmin)) return false;
    launch_repack(wtype, w, n_out, n_in, L.w, L.wd, L.wmin, d.s);
    return true;
}

}  // namespace

extern "C" int jepa_amd_matmul(int device, int wtype, const void * w, int64_t n_out, int64_t n_in, const float * bias, const float * x,
                               int64_t n_rows, float * y, int reps, double * gemm_ms) {
    if (!w || !x || !y || n_out <= 0 || n_in <= 0 || n_rows <= 0) return -1;
    dev_scope d(device);
    if (!d.ok) return -1;
    dev_linear L;
    if (!make_linear(d, "jepa_amd_matmul", wtype, w, n_out, n_in, bias, L)) return -1;
    act_view a;
    if (!alloc_act(d, a, L.act(), n_rows, n_in)) return -1;
    launch_rownorm_quant(x, n_rows, n_in, nullptr, nullptr, 0.0f, false, a, d.s);
    gemm_split_ws sw;
    if (!alloc_split(d, sw, n_rows)) return -1;
    gemm_epi ep;
    ep.kind = EPI_F32;
    ep.y = y; ep.ldy = n_out; ep.rin = n_rows; ep.rout = n_rows; ep.pre = 0;
    hipEvent_t e0, e1;
    hipEventCreate(&e0); hipEventCreate(&e1);
    if (reps < 1) reps = 1;
    launch_gemm(L, a, n_rows, ep, d.s, &sw);   // warm-up (and the result when reps == 1)
    hipEventRecord(e0, d.s);
    for (int i = 0; i < reps; i++) launch_gemm(L, a, n_rows, ep, d.s, &sw);
    hipEventRecord(e1, d.s);
    const int rc = d.finish();
    float ms = 0;
    hipEventElapsedTime(&ms, e0, e1);
    if (gemm_ms) *gemm_ms = ms / reps;
    hipEventDestroy(e0); hipEventDestroy(e1);
    return rc;
}

extern "C" int jepa_amd_matmul_gelu(int device, int wtype, const void * w, int64_t n_out, int64_t n_in, const float * bias,
                                    const float * x, int64_t n_rows, int out_type, void * out, int reps, double * gemm_ms) {
    if (!w || !x || !out || n_out <= 0 || n_in <= 0 || n_rows <= 0) return -1;
    if (!(out_type == T_F32 || out_type == T_F16 || out_type == T_Q8_0 || out_type == T_Q8_K) ||
        (out_type == T_Q8_K && n_out % 256) || (out_type == T_F16 && wtype == T_F32)) {
        jepa_log("jepa: jepa_amd_matmul_gelu: output type %d not supported for weight type %d, n_out %lld\n", out_type, wtype,
                 (long long) n_out);
        return -1;
    }
    dev_scope d(device);
    if (!d.ok) return -1;
    dev_linear L;
    if (!make_linear(d, "jepa_amd_matmul_gelu", wtype, w, n_out, n_in, bias, L)) return -1;
    if (L.fmt == W_F32 && out_type != T_F32) {
        jepa_log("jepa: jepa_amd_matmul_gelu: f32 weights have the f32 epilogue only\n");
        return -1;
    }
    act_view a;
    if (!alloc_act(d, a, L.act(), n_rows, n_in)) return -1;
    launch_rownorm_quant(x, n_rows, n_in, nullptr, nullptr, 0.0f, false, a, d.s);
    gemm_epi ep;
    ep.ldy = n_out;
    act_view o;
    if (out_type == T_F32) { ep.kind = EPI_GELU_F32; ep.y = (float *) out; }
    else if (out_type == T_F16) { ep.kind = EPI_GELU_F16; ep.oh = out; }
    else {
        if (!alloc_act(d, o, out_type == T_Q8_0 ? A_Q8_0 : A_Q8_K, n_rows, n_out)) return -1;
        if (out_type == T_Q8_0) { ep.kind = EPI_GELU_Q8_0; ep.oq = o.q; ep.od = o.d; }
        else { ep.kind = EPI_GELU_Q8_K; ep.oh = o.q; ep.od = o.d; ep.ob = o.bsum; }
    }
    hipEvent_t e0, e1;
    hipEventCreate(&e0); hipEventCreate(&e1);
    if (reps < 1) reps = 1;
    gemm_split_ws sw;
    if (!alloc_split(d, sw, n_rows)) return -1;
    launch_gemm(L, a, n_rows, ep, d.s, &sw);   // warm-up (and the result when reps == 1)
    hipEventRecord(e0, d.s);
    for (int i = 1; i < reps; i++) launch_gemm(L, a, n_rows, ep, d.s, &sw);
    hipEventRecord(e1, d.s);
    if (out_type == T_Q8_0 || out_type == T_Q8_K) launch_pack_act_blocks(o, n_rows, n_out, out, d.s);
    const int rc = d.finish();
    float ms = 0;
    hipEventElapsedTime(&ms, e0, e1);
    if (gemm_ms) *gemm_ms = reps > 1 ? ms / (reps - 1) : 0.0;
    hipEventDestroy(e0); hipEventDestroy(e1);
    return rc;
}

extern "C" int jepa_amd_gemm_split(int split) { return gemm_force_split(split); }

extern "C" int jepa_amd_gemm_split_of(int wtype, int64_t n_out, int64_t n_in) {
    const int wf = weight_format(wtype, n_in);
    return wf < 0 ? 1 : gemm_split_for(wf, n_out, n_in);
}

extern "C" int jepa_amd_gemm_tile(int index) {
    if (gemm_force_tile(index) != 0) { jepa_log("jepa: jepa_amd_gemm_tile: no tile %d\n", index); return -1; }
    return 0;
}

extern "C" int jepa_amd_attention(int device, const float * qkv, int64_t n_items, int64_t n_tok, int n_head, int hd,
                                  const float * rope_c, const float * rope_s, int n_prefix, int64_t tokens_per_slot, int out_type,
                                  void * out) {
    if (!qkv || !out || n_items <= 0 || n_tok <= 0 || n_head <= 0 || n_prefix < 0 || tokens_per_slot < 0 ||
        n_tok > 0x40000000) return -1;
    if (!attention_supports(hd)) { jepa_log("jepa: jepa_amd_attention: head width %d (a multiple of 16 up to 128)\n", hd); return -1; }
    if (out_type != T_F32 && !((out_type == T_Q8_0 || out_type == T_F16) && (hd == 64 || hd == 32))) {
        jepa_log("jepa: jepa_amd_attention: output type %d for head width %d\n", out_type, hd);
        return -1;
    }
    dev_scope d(device);
    if (!d.ok) return -1;
    const int hds = attention_stored_width(hd);   // stored head width
    const int64_t R_pad = (n_tok + 127) / 128 * 128;
    const size_t bytes = (size_t) n_items * n_head * R_pad * hds * 2;
    void * q = d.alloc(bytes), * k = d.alloc(bytes), * vt = d.alloc(bytes);
    if (!q || !k || !vt) return -1;
    launch_fill_zero(q, bytes, d.s);
    launch_fill_zero(k, bytes, d.s);
    launch_fill_zero(vt, bytes, d.s);
    gemm_epi ep;
    ep.kind = EPI_QKV;
    ep.q = q; ep.k = k; ep.vt = vt; ep.rope_c = rope_c; ep.rope_s = rope_s;
    ep.n_head = n_head; ep.hd = hd; ep.hds = hds; ep.D = n_head * hd; ep.R = n_tok; ep.R_pad = R_pad;
    launch_qkv_split(qkv, n_items * n_tok, (int64_t) 3 * n_head * hd, ep, d.s);
    act_view o;
    const int64_t rows = n_items * n_tok, D = (int64_t) n_head * hd;
    if (out_type == T_F32) {
        o.fmt = A_F32; o.q = out; o.ld = D;
    } else if (out_type == T_F16) {
        o.fmt = A_F16; o.q = out; o.ld = D;
    } else {
        o.fmt = A_Q8_0; o.ld = D;
        o.q = d.alloc((size_t) rows * D);
        o.d = d.alloc((size_t) rows * (D / 32) * 2);
        if (!o.q || !o.d) return -1;
    }
    launch_attention(q, k, vt, o, n_items, n_head, hd, n_tok, R_pad, 1.0f / sqrtf((float) hd), n_prefix, tokens_per_slot, d.s);
    if (out_type == T_Q8_0) launch_pack_act_blocks(o, rows, D, out, d.s);
    return d.finish();
}

extern "C" int jepa_amd_quantize_rows(int device, int gtype, const float * x, int64_t n, void * out) {
    if (!x || !out || n < 0) return -1;
    dev_scope d(device);
    if (!d.ok) return -1;
    if (!launch_quantize_rows(gtype, x, n, out, d.s)) {
        jepa_log("jepa: jepa_amd_quantize_rows: type %d with %lld values is not a quantizer target\n", gtype, (long long) n);
        return -1;
    }
    return d.finish();
}

extern "C" int jepa_amd_mfma_probe(int device, const float * a, const float * b, float * dd) {
    if (!a || !b || !dd) return -1;
    dev_scope d(device);
    if (!d.ok) return -1;
    float * da = (float *) d.alloc(32 * 16 * 4), * db = (float *) d.alloc(16 * 32 * 4), * dc = (float *) d.alloc(32 * 32 * 4);
    if (!da || !db || !dc) return -1;
    hipMemcpy(da, a, 32 * 16 * 4, hipMemcpyHostToDevice);
    hipMemcpy(db, b, 16 * 32 * 4, hipMemcpyHostToDevice);
    launch_mfma_probe(da, db, dc, d.s);
    if (d.finish() != 0) return -1;
    return hipMemcpy(dd, dc, 32 * 32 * 4, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}

extern "C" int jepa_amd_gemm_step_probe(int device, int mode, int waves_per_simd, int iters, double * ns_per_step) {
    if (mode < 0 || mode > 3 || waves_per_simd < 1 || waves_per_simd > 4 || iters < 1 || iters > 1000000 || !ns_per_step) return -1;
    dev_scope d(device);
    if (!d.ok) return -1;
    int dev = 0, n_cu = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0) n_cu = 256;
    float * sink = (float *) d.alloc((size_t) n_cu * 256 * waves_per_simd * 4);
    if (!sink) return -1;
    launch_step_probe(mode, waves_per_simd, iters, n_cu, sink, d.s);   // warm
    hipEvent_t e0, e1;
    hipEventCreate(&e0); hipEventCreate(&e1);
    hipEventRecord(e0, d.s);
    launch_step_probe(mode, waves_per_simd, iters, n_cu, sink, d.s);
    hipEventRecord(e1, d.s);
    const int rc = d.finish();
    float ms = 0;
    hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0); hipEventDestroy(e1);
    // one workgroup per CU, waves_per_simd waves on each of its 4 SIMDs, 2 * iters (half or whole) steps each;
    // a whole step is counted once per wave of modes 0-2 and once per pair of waves of mode 3
    const double steps_per_simd = 2.0 * iters * waves_per_simd / (mode == 3 ? 2.0 : 1.0);
    *ns_per_step = (double) ms * 1e6 / steps_per_simd;
    return rc;
}

extern "C" int jepa_amd_copy(int device, const float * src, float * dst, int64_t n, int reps, double * ms) {
    if (!src || !dst || n <= 0) return -1;
    dev_scope d(device);
    if (!d.ok) return -1;
    if (reps < 1) reps = 1;
    hipEvent_t e0, e1;
    hipEventCreate(&e0); hipEventCreate(&e1);
    launch_copy_f32(src, dst, n, d.s);
    hipEventRecord(e0, d.s);
    for (int i = 0; i < reps; i++) launch_copy_f32(src, dst, n, d.s);
    hipEventRecord(e1, d.s);
    const int rc = d.finish();
    float t = 0;
    hipEventElapsedTime(&t, e0, e1);
    if (ms) *ms = t / reps;
    hipEventDestroy(e0); hipEventDestroy(e1);
    return rc;
}

extern "C" int jepa_amd_preprocess_frames_device(int device, const jepa_preprocess_params * p, const uint8_t * frames, int n_frames, int h,
                                                 int w, float * out, int64_t out_cap, int * out_h, int * out_w) {
    if (!p || !frames || !out || n_frames <= 0 || h <= 0 || w <= 0) return -1;
    pre_plan g;
    if (!pre_plan_for(p, h, w, g)) return -1;
    const int64_t need = (int64_t) 3 * n_frames * g.crop * g.crop;
    if (out_cap < need) {
        jepa_log("jepa: jepa_amd_preprocess_frames_device: output holds %lld floats, %lld needed\n", (long long) out_cap, (long long) need);
        return -1;
    }
    dev_scope d(device);
    if (!d.ok) return -1;
    void * scratch = d.alloc(preprocess_scratch_bytes(p, g, n_frames, h, w));
    if (!scratch) return -1;
    if (!launch_preprocess(p, g, frames, n_frames, h, w, out, scratch, d.s)) {
        jepa_log("jepa: jepa_amd_preprocess_frames_device: launch failed\n");
        return -1;
    }
    if (out_h) *out_h = g.crop;
    if (out_w) *out_w = g.crop;
    return d.finish();
}

extern "C" int jepa_amd_preprocess_frames_device_noalloc(int device, const jepa_preprocess_params * p, const uint8_t * frames, int n_frames,
                                                         int h, int w, float * out, int64_t out_cap, int * out_h, int * out_w, void * stream) {
    if (!p || !frames || !out || n_frames <= 0 || h <= 0 || w <= 0) return -1;
    pre_plan g;
    if (!pre_plan_for(p, h, w, g)) return -1;
    const int64_t need = (int64_t) 3 * n_frames * g.crop * g.crop;
    if (out_cap < need) {
        jepa_log("jepa: jepa_amd_preprocess_frames_device_noalloc: output holds %lld floats, %lld needed\n", (long long) out_cap,
                 (long long) need);
        return -1;
    }
    const size_t bytes = preprocess_scratch_bytes(p, g, n_frames, h, w);
    if (bytes > PRE_NOALLOC_SCRATCH_BYTES) {
        jepa_log("jepa: jepa_amd_preprocess_frames_device_noalloc: %d frames of %dx%d need %.1f MiB of scratch, over the %zu MiB "
                 "this entry point has (use jepa_amd_preprocess_frames_device, or fewer frames per call)\n",
                 n_frames, h, w, (double) bytes / 1048576.0, PRE_NOALLOC_SCRATCH_BYTES >> 20);
        return -1;
    }
    if (!dev_check(device)) return -1;
    int prev = 0;
    hipGetDevice(&prev);
    if (hipSetDevice(device) != hipSuccess) {
        jepa_log("jepa: cannot use HIP device %d\n", device);
        return -1;
    }
    int rc = -1;
    void * scratch = preprocess_static_scratch(device);
    if (scratch) {
        hipStream_t s = (hipStream_t) stream;
        if (!launch_preprocess(p, g, frames, n_frames, h, w, out, scratch, s)) {
            jepa_log("jepa: jepa_amd_preprocess_frames_device_noalloc: launch failed: %s\n", hipGetErrorString(hipGetLastError()));
        } else {
            if (out_h) *out_h = g.crop;
            if (out_w) *out_w = g.crop;
            rc = 0;
        }
    }
    hipSetDevice(prev);
    return rc;
}

extern "C" int jepa_amd_rope_tables(int head_dim, int grid_t, int grid_h, int grid_w, int variant, int interpolate, int train_h,
                                    int train_w, float theta, const int32_t * ids, int64_t n_rows, int signed_sin, float * cos_out,
                                    float * sin_out) {
    if (head_dim <= 0 || grid_t <= 0 || grid_h <= 0 || grid_w <= 0 || n_rows <= 0 || !cos_out || !sin_out || (variant != 0 && variant != 1)) {
        jepa_log("jepa: jepa_amd_rope_tables: bad arguments (head_dim %d, grid %dx%dx%d, %lld rows, variant %d)\n", head_dim, grid_t,
                 grid_h, grid_w, (long long) n_rows, variant);
        return -1;
    }
    const int64_t n_grid = (int64_t) grid_t * grid_h * grid_w;
    if (!ids && n_rows > n_grid) {
        jepa_log("jepa: jepa_amd_rope_tables: %lld rows but the grid has %lld tokens\n", (long long) n_rows, (long long) n_grid);
        return -1;
    }
    for (int64_t r = 0; ids && r < n_rows; r++)
        if (ids[r] < 0 || ids[r] >= n_grid) {
            jepa_log("jepa: jepa_amd_rope_tables: id %d is outside the %lld-token grid\n", ids[r], (long long) n_grid);
            return -1;
        }
    rope3d_params p;
    p.grid_t = grid_t; p.grid_h = grid_h; p.grid_w = grid_w;
    p.head_dim = head_dim;
    p.theta = theta;
    p.interpolate = interpolate != 0;
    p.train_grid_h = train_h; p.train_grid_w = train_w;
    p.variant = variant;
    std::vector<float> c, s;
    rope3d_tables(p, ids, n_rows, c, s, signed_sin != 0);
    memcpy(cos_out, c.data(), c.size() * sizeof(float));
    memcpy(sin_out, s.data(), s.size() * sizeof(float));
    return 0;
}
