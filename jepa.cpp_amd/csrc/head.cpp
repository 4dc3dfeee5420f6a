// head.cpp - the attentive-pool head (V-JEPA 2 video classifiers) on one HIP device, and the
// jepa_head / jepa_head_ex entry points (reference src/jepa.cpp:1026-1112).
//
// Sequence (reference src/jepa.cpp:1034-1075), on one sequence of N encoder rows:
//   head.blk.{i}: the encoder's pre-LN block without RoPE (full attention over the N rows)
//   LN_kv(x) -> codes | K GEMM, V GEMM (f32 rows [N][D]; the LN is on the keys / values only)
//   q0 = head.query (raw) -> codes | q GEMM -> q [D]
//   pool attention: y = softmax(q K^T / sqrt(hd)) V + q0          (no output projection)
//   y += ffn_down(gelu(ffn_up(LN2 y)))                               (the block MLP kernels, 1 row)
//   logits = cls(y)                                                  (no final norm)
// The blocks and GEMMs are the encoder's kernels; the one-row GEMMs run the same MFMA tiles with
// the rows past the first masked, so every output has the encoder's summation order.
#include "forward.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace {

bool head_supported(const jepa_model * m) {
    const enc_hparams & e = m->hp.enc;
    if (!m->hp.has_head || m->hp.head_kind != "attentive_pool" || !m->head.cls.w) {
        jepa_log("jepa: jepa_head: model '%s' has no attentive-pool head\n", m->hp.name.c_str());
        return false;
    }
    if (e.head_dim() != 64) {
        jepa_log("jepa: jepa_head: head_dim %d is not supported by the attention kernels (64 only)\n", e.head_dim());
        return false;
    }
    if (e.embed_dim % 128 != 0 || e.embed_dim > 2048) {
        jepa_log("jepa: jepa_head: embed_dim %d is not a multiple of 128 up to 2048\n", e.embed_dim);
        return false;
    }
    if (e.act != ACT_GELU_ERF) {
        jepa_log("jepa: jepa_head: only the gelu_erf activation is implemented on this path\n");
        return false;
    }
    auto ffn_ok = [](int64_t F) { return F <= 2048 || F % 256 == 0; };
    for (const dev_layer & L : m->head.blocks)
        if (!ffn_ok(L.up.n_out)) { jepa_log("jepa: jepa_head: head block FFN width %lld is not supported\n", (long long) L.up.n_out); return false; }
    if (!ffn_ok(m->head.up.n_out)) {
        jepa_log("jepa: jepa_head: head MLP width %lld is not supported\n", (long long) m->head.up.n_out);
        return false;
    }
    return true;
}

bool ensure_head_workspace(jepa_context * ctx, int64_t N) {
    const jepa_model * m = ctx->model;
    const enc_hparams & e = m->hp.enc;
    fwd_workspace * w = ctx->hws.get();
    if (w && w->model == m && w->R == N) return true;
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
    ctx->hws.reset(new fwd_workspace());
    w = ctx->hws.get();
    w->model = m;
    const dev_head & h = m->head;
    int64_t F = h.up.n_out;
    for (const dev_layer & L : h.blocks) F = std::max<int64_t>(F, L.up.n_out);
    const int64_t D = e.embed_dim;
    w->hpart_n = pool_attention_part_floats(N, e.n_head);
    const bool ok = ws_alloc_blocks(*w, 1, N, D, F, e.n_head, enc_blk_shape(m).hds, ctx->stream) && ws_alloc(*w, (void **) &w->hq, (size_t) D * 4) &&
                    ws_alloc(*w, (void **) &w->hy, (size_t) D * 4) && ws_alloc(*w, (void **) &w->hlog, (size_t) h.cls.n_out * 4) &&
                    ws_alloc(*w, (void **) &w->hpart, (size_t) w->hpart_n * 4);
    if (!ok || hipStreamSynchronize(ctx->stream) != hipSuccess) { ctx->hws.reset(); return false; }
    return true;
}

// one-row (or N-row) linear with f32 output rows y [rows][W.n_out]
void linear_f32(const dev_linear & W, const float * x, int64_t rows, int64_t D, float * y, fwd_workspace & w, hipStream_t s, ktimer & kt,
                const char * what) {
    w.actA.fmt = W.act();
    kt.run("quantize", [&] { launch_rownorm_quant(x, rows, D, nullptr, nullptr, 0.0f, false, w.actA, s); }, what);
    gemm_epi ep;
    ep.kind = EPI_F32; ep.y = y; ep.ldy = W.n_out;
    kt.run(gemm_class(W), [&] { launch_gemm(W, w.actA, rows, ep, s, &w.split); }, what);
}

// the head on the N rows already in the head workspace's x; pooled token in w.hy, logits in w.hlog
int head_run(jepa_context * ctx, int64_t N, bool with_logits) {
    const jepa_model * m = ctx->model;
    const enc_hparams & e = m->hp.enc;
    const dev_head & h = m->head;
    fwd_workspace & w = *ctx->hws;
    hipStream_t s = ctx->stream;
    const int64_t D = e.embed_dim;
    const int H = e.n_head, hd = e.head_dim();
    ktimer kt{ctx};
    bool ok = true;
    hipEventRecord(ctx->ev0, s);
    const blk_shape bs = enc_blk_shape(m);
    for (const dev_layer & L : h.blocks) enqueue_block(bs, L, w, 1, N, nullptr, nullptr, 0, 0, s, kt);
    // cross-attention: K and V from LN_kv(x) (one set of codes when both weights take the same input format)
    float * Kf = w.attn, * Vf = w.out;
    w.actA.fmt = h.k.act();
    kt.run("layernorm", [&] { launch_rownorm_quant(w.x, N, D, h.ln_kv_w, h.ln_kv_b, e.ln_eps, true, w.actA, s); });
    {
        gemm_epi ep;
        ep.kind = EPI_F32; ep.y = Kf; ep.ldy = D;
        kt.run(gemm_class(h.k), [&] { launch_gemm(h.k, w.actA, N, ep, s, &w.split); }, "k");
    }
    if (h.v.act() != h.k.act()) {
        w.actA.fmt = h.v.act();
        kt.run("layernorm", [&] { launch_rownorm_quant(w.x, N, D, h.ln_kv_w, h.ln_kv_b, e.ln_eps, true, w.actA, s); });
    }
    {
        gemm_epi ep;
        ep.kind = EPI_F32; ep.y = Vf; ep.ldy = D;
        kt.run(gemm_class(h.v), [&] { launch_gemm(h.v, w.actA, N, ep, s, &w.split); }, "v");
    }
    linear_f32(h.q, h.query, 1, D, w.hq, w, s, kt, "q");
    kt.run("pool_attention", [&] {
        ok = launch_pool_attention(w.hq, Kf, Vf, N, D, H, hd, 1.0f / sqrtf((float) hd), h.query, w.hy, w.hpart, w.hpart_n, s);
    });
    enqueue_mlp(h.up, h.down, h.ln2_w, h.ln2_b, e.ln_eps, nullptr, w.hy, 1, D, w, s, kt);
    if (with_logits) linear_f32(h.cls, w.hy, 1, D, w.hlog, w, s, kt, "cls");
    hipEventRecord(ctx->ev1, s);
    const hipError_t err = hipStreamSynchronize(s);
    if (!ok || err != hipSuccess) {
        jepa_log("jepa: jepa_head: device execution failed: %s\n", hipGetErrorString(err));
        return -1;
    }
    float ms = 0;
    hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1);
    ctx->last_compute_ms = ms;
    kt.collect();
    return (int) h.cls.n_valid;
}

bool head_check_rows(const jepa_model * m, int64_t N) {
    if (N <= 0 || N > JEPA_LIMIT_N_TOKENS) {
        jepa_log("jepa: jepa_head: %lld tokens is out of range\n", (long long) N);
        return false;
    }
    return head_supported(m);
}

}  // namespace

int head_device(jepa_context * ctx, const float * x_dev, int64_t N, float * pooled_dev, float * logits_dev) {
    if (!head_check_rows(ctx->model, N) || hipSetDevice(ctx->device) != hipSuccess || !ensure_head_workspace(ctx, N)) return -1;
    fwd_workspace & w = *ctx->hws;
    const int64_t D = ctx->model->hp.enc.embed_dim;
    if (hipMemcpyAsync(w.x, x_dev, (size_t) N * D * 4, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess) return -1;
    const int C = head_run(ctx, N, logits_dev != nullptr);
    if (C < 0) return -1;
    if ((pooled_dev && hipMemcpyAsync(pooled_dev, w.hy, (size_t) D * 4, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess) ||
        (logits_dev && hipMemcpyAsync(logits_dev, w.hlog, (size_t) C * 4, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess) ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) return -1;
    return C;
}

// reference include/jepa.h:122-145, src/jepa.cpp:1077-1112, 1309-1311: encoder rows from the host,
// outputs malloc'd (the caller frees them with jepa_output_free); nothing is returned on failure
extern "C" int jepa_head_ex(jepa_context * ctx, const jepa_output * enc, jepa_output * pooled, jepa_output * logits) {
    if (!ctx || !enc || !enc->data || enc->n_tokens <= 0) return -1;
    const jepa_model * m = ctx->model;
    if (!head_supported(m)) return -1;
    if (enc->dim != m->hp.enc.embed_dim) {
        jepa_log("jepa: jepa_head: encoder rows are %lld wide, expected %d\n", (long long) enc->dim, m->hp.enc.embed_dim);
        return -1;
    }
    const int64_t D = enc->dim, N = enc->n_tokens;
    if (N > JEPA_LIMIT_N_TOKENS) {
        jepa_log("jepa: jepa_head: %lld x %lld tokens do not fit in memory\n", (long long) N, (long long) D);
        return -1;
    }
    if (!head_check_rows(m, N) || hipSetDevice(ctx->device) != hipSuccess || !ensure_head_workspace(ctx, N)) return -1;
    fwd_workspace & w = *ctx->hws;
    if (hipMemcpyAsync(w.x, enc->data, (size_t) N * D * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess) {
        jepa_log("jepa: input upload failed\n");
        return -1;
    }
    const int C = head_run(ctx, N, logits != nullptr);
    if (C < 0) return -1;
    float * hp = nullptr, * hl = nullptr;
    if (pooled && !(hp = (float *) malloc((size_t) D * 4))) return -1;
    if (logits && !(hl = (float *) malloc((size_t) std::max(C, 1) * 4))) { free(hp); return -1; }
    if ((hp && hipMemcpyAsync(hp, w.hy, (size_t) D * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess) ||
        (hl && hipMemcpyAsync(hl, w.hlog, (size_t) C * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess) ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        jepa_log("jepa: output download failed\n");
        free(hp); free(hl);
        return -1;
    }
    if (pooled) { pooled->data = hp; pooled->n_tokens = 1; pooled->dim = D; }
    if (logits) { logits->data = hl; logits->n_tokens = 1; logits->dim = C; }
    return 0;
}

extern "C" int jepa_head(jepa_context * ctx, const jepa_output * enc, jepa_output * out) { return jepa_head_ex(ctx, enc, nullptr, out); }
