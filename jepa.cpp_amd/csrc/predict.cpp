// predict.cpp - the V-JEPA 2 / 2.1 masked predictor on one HIP device, and jepa_predict /
// jepa_predict_ex / jepa_predict_mod (reference src/predictor.cpp:23-285).
//
// Sequence (reference src/predictor.cpp:56-133), rows = context ids then target ids:
//   context rows -> codes | pred.embed GEMM (+ bias, + modality vector)        -> x[0, n_ctx)
//     (2.1 ViT-g/G: pred.embed.0 GEMM + GELU -> codes | pred.embed.2 GEMM)
//   mask token row (+ modality vector)                                        -> x[n_ctx, n_ctx + n_tgt)
//   pred.blk.{i}: pre-LN blocks, 3-D RoPE from the token ids on q and k, full attention; the
//                 12 heads of 32 are stored 64 wide (zero upper half) for the head-64 attention kernel
//   pred.norm on the target rows -> codes | pred.proj GEMM                   -> out [n_tgt][out_dim]
// The LayerNorm epsilon of the blocks and the final norm is the encoder's (src/predictor.cpp:101-104).
#include "forward.h"
#include "rope3d.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

bool pred_supported(const jepa_model * m) {
    const pred_hparams & p = m->hp.pred;
    if (!m->hp.has_pred) {
        jepa_log("jepa: jepa_predict: '%s' has no predictor\n", m->hp.name.c_str());
        return false;
    }
    if (p.kind != "masked") {
        jepa_log("jepa: jepa_predict: predictor kind '%s' is not the masked predictor%s\n", p.kind.c_str(),
                 p.kind == "lewm" ? " (use jepa_lewm_predict)" : p.kind == "ac" ? " (use jepa_ac_predict)" : "");
        return false;
    }
    if (m->pred.blocks.size() != (size_t) p.n_layer || !m->pred.proj.w) {
        jepa_log("jepa: jepa_predict: the predictor of '%s' was not loaded\n", m->hp.name.c_str());
        return false;
    }
    const int hd = p.head_dim_eff();
    if ((hd != 32 && hd != 64) || p.n_head * hd != p.embed_dim) {
        jepa_log("jepa: jepa_predict: %d heads of %d in a %d-wide predictor are not supported (heads of 32 or 64 filling the width)\n",
                 p.n_head, hd, p.embed_dim);
        return false;
    }
    if (p.embed_dim % 128 != 0 || (p.embed_dim > 2048 && p.embed_dim % 256 != 0)) {
        jepa_log("jepa: jepa_predict: predictor width %d is not supported by the row kernels\n", p.embed_dim);
        return false;
    }
    if (p.act != ACT_GELU_ERF) {
        jepa_log("jepa: jepa_predict: only the gelu_erf activation is implemented on this path\n");
        return false;
    }
    return true;
}

blk_shape pred_shape(const jepa_model * m) {
    const pred_hparams & p = m->hp.pred;
    blk_shape b;
    b.D = p.embed_dim; b.H = p.n_head; b.hd = p.head_dim_eff(); b.hds = 64; b.eps = m->hp.enc.ln_eps;
    return b;
}

// reference src/predictor.cpp:23-49: ids are decoded on (grid_t, grid, grid), grid_t from the largest id
rope3d_params pred_rope(const jepa_model * m, int64_t max_id) {
    const enc_hparams & e = m->hp.enc;
    const pred_hparams & p = m->hp.pred;
    rope3d_params rp;
    const int grid = p.grid_size > 0 ? p.grid_size : e.grid_size();
    rp.grid_h = rp.grid_w = grid;
    const int64_t per_frame = (int64_t) grid * grid;
    rp.grid_t = per_frame > 0 ? (int) std::min<int64_t>(max_id / per_frame + 1, INT32_MAX) : 0;
    rp.head_dim = p.head_dim_eff();
    rp.theta = e.rope_theta;
    rp.interpolate = p.rope_interpolate;
    rp.train_grid_h = rp.train_grid_w = p.rope_ref_grid;
    if (!p.rope_freq_layout.empty()) rp.variant = p.rope_freq_layout == "interleaved" ? 1 : 0;
    else rp.variant = m->hp.family == FAM_VJEPA2_1 ? 1 : 0;
    return rp;
}

bool ensure_pred_workspace(jepa_context * ctx, int n_ctx, int n_tgt) {
    const jepa_model * m = ctx->model;
    const pred_hparams & p = m->hp.pred;
    fwd_workspace * w = ctx->pws.get();
    if (w && w->model == m && w->n_ctx == n_ctx && w->n_tgt == n_tgt) return true;
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
    ctx->pws.reset(new fwd_workspace());
    w = ctx->pws.get();
    w->model = m;
    w->n_ctx = n_ctx; w->n_tgt = n_tgt;
    const dev_pred & pr = m->pred;
    const blk_shape b = pred_shape(m);
    const int64_t N = (int64_t) n_ctx + n_tgt, De = m->hp.enc.embed_dim;
    int64_t F = p.ffn_dim;
    for (const dev_layer & L : pr.blocks) F = std::max<int64_t>(F, L.up.n_out);
    if (pr.embed0.w) F = std::max<int64_t>(F, pr.embed0.n_out);
    const bool ok = ws_alloc_blocks(*w, 1, N, b.D, F, b.H, b.hds, ctx->stream) &&
                    ws_alloc(*w, (void **) &w->pin, (size_t) std::max(n_ctx, 1) * De * 4) &&
                    ws_alloc_act(*w, w->actC, std::max(n_ctx, 1), De) &&
                    ws_alloc(*w, (void **) &w->pout, (size_t) n_tgt * pr.proj.n_out * 4) &&
                    ws_alloc(*w, (void **) &w->rope_c, (size_t) N * b.hd * 4) && ws_alloc(*w, (void **) &w->rope_s, (size_t) N * b.hd * 4);
    if (!ok || hipStreamSynchronize(ctx->stream) != hipSuccess) { ctx->pws.reset(); return false; }
    return true;
}

// the predictor on the context rows already in w.pin; target rows into w.pout
int pred_run(jepa_context * ctx, const int32_t * ids, int n_ctx, int n_tgt, int mask_index, int modality) {
    const jepa_model * m = ctx->model;
    const pred_hparams & p = m->hp.pred;
    const dev_pred & pr = m->pred;
    fwd_workspace & w = *ctx->pws;
    hipStream_t s = ctx->stream;
    const blk_shape b = pred_shape(m);
    const int64_t N = (int64_t) n_ctx + n_tgt, Dp = b.D, De = m->hp.enc.embed_dim;
    int64_t max_id = 0;
    for (int64_t i = 0; i < N; i++) max_id = std::max<int64_t>(max_id, ids[i]);
    const rope3d_params rp = pred_rope(m, max_id);
    if (rp.grid_t <= 0 || rp.grid_t > JEPA_LIMIT_N_FRAMES) {
        jepa_log("jepa: jepa_predict: token id %lld puts the predictor grid at %d temporal slices (grid %dx%d, limit %d) - the ids "
                 "are not positions on this model's grid\n", (long long) max_id, rp.grid_t, rp.grid_h, rp.grid_w, JEPA_LIMIT_N_FRAMES);
        return -1;
    }
    const float * mod = nullptr;
    if (p.modality_embed) {
        const bool image = modality == 2;
        mod = image ? pr.mod_img : pr.mod_video;
        if (!mod) {
            jepa_log("jepa: jepa_predict: jepa.pred.modality_embed is set but pred.mod_embed_%s is missing\n", image ? "img" : "video");
            return -1;
        }
    }
    std::vector<float> c, sn;
    rope3d_tables(rp, ids, N, c, sn, true);
    ktimer kt{ctx};
    hipEventRecord(ctx->ev0, s);
    bool ok = hipMemcpyAsync(w.rope_c, c.data(), c.size() * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
              hipMemcpyAsync(w.rope_s, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, s) == hipSuccess;
    // 1. context rows -> predictor width (+ modality vector)
    if (n_ctx > 0) {
        const dev_linear & last = pr.embed0.w ? pr.embed2 : pr.embed;
        gemm_epi ep;
        ep.kind = EPI_F32; ep.y = w.x; ep.ldy = Dp; ep.addvec = mod;
        if (pr.embed0.w) {
            w.actC.fmt = pr.embed0.act();
            kt.run("quantize", [&] { launch_rownorm_quant(w.pin, n_ctx, De, nullptr, nullptr, 0.0f, false, w.actC, s); }, "embed");
            w.actB.fmt = pr.embed2.act();
            enqueue_gemm_gelu(pr.embed0, w.actC, n_ctx, w.actB, w, s, kt, "embed0");
            kt.run(gemm_class(last), [&] { launch_gemm(last, w.actB, n_ctx, ep, s, &w.split); }, "embed2");
        } else {
            w.actC.fmt = last.act();
            kt.run("quantize", [&] { launch_rownorm_quant(w.pin, n_ctx, De, nullptr, nullptr, 0.0f, false, w.actC, s); }, "embed");
            kt.run(gemm_class(last), [&] { launch_gemm(last, w.actC, n_ctx, ep, s, &w.split); }, "embed");
        }
    }
    // 2. mask token rows (+ modality vector): row mask_index mod the declared count
    {
        const int64_t n_mask = p.n_mask_tokens > 0 ? p.n_mask_tokens : pr.n_mask_rows;
        int64_t idx = n_mask > 0 ? mask_index % n_mask : 0;
        if (idx < 0) idx += n_mask;
        kt.run("cls", [&] { launch_cls_rows(w.x + (int64_t) n_ctx * Dp, pr.mask_tokens + idx * Dp, mod, n_tgt, 1, Dp, s); });
    }
    // 3. blocks with 3-D RoPE from the ids
    for (const dev_layer & L : pr.blocks) enqueue_block(b, L, w, 1, N, w.rope_c, w.rope_s, 0, 0, s, kt);
    // 4. final norm of the target rows, projection
    w.actA.fmt = pr.proj.act();
    kt.run("layernorm", [&] {
        launch_rownorm_quant(w.x + (int64_t) n_ctx * Dp, n_tgt, Dp, pr.norm_w, pr.norm_b, b.eps, true, w.actA, s);
    });
    {
        gemm_epi ep;
        ep.kind = EPI_F32; ep.y = w.pout; ep.ldy = pr.proj.n_out;
        kt.run(gemm_class(pr.proj), [&] { launch_gemm(pr.proj, w.actA, n_tgt, ep, s, &w.split); }, "proj");
    }
    hipEventRecord(ctx->ev1, s);
    const hipError_t err = hipStreamSynchronize(s);
    if (!ok || err != hipSuccess) {
        jepa_log("jepa: jepa_predict: device execution failed: %s\n", hipGetErrorString(err));
        return -1;
    }
    float ms = 0;
    hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1);
    ctx->last_compute_ms = ms;
    kt.collect();
    return (int) pr.proj.n_out;
}

// shared checks of both entry points (reference src/predictor.cpp:140-178)
bool pred_check(const jepa_context * ctx, int n_context, int n_target, const int32_t * ids, int64_t enc_rows) {
    const jepa_model * m = ctx->model;
    const pred_hparams & p = m->hp.pred;
    if (n_target <= 0 || n_context < 0) {
        jepa_log("jepa: jepa_predict: need n_target > 0 and n_context >= 0 (got %d / %d)\n", n_target, n_context);
        return false;
    }
    const int64_t n_rows = (int64_t) n_context + n_target;
    const double need = (double) n_rows * (3.0 * p.embed_dim + (double) p.ffn_dim + 8.0 * p.embed_dim) * sizeof(float);
    const size_t budget = ctx->max_graph_bytes ? ctx->max_graph_bytes : JEPA_DEFAULT_MAX_GRAPH_BYTES;
    if (need >= (double) budget) {
        jepa_log("jepa: jepa_predict: %lld context + %lld target rows need about %.1f MiB of activations, over the %.1f MiB limit - "
                 "raise $JEPA_MAX_GRAPH_MIB or predict fewer tokens per call\n", (long long) n_context, (long long) n_target,
                 need / 1048576.0, (double) budget / 1048576.0);
        return false;
    }
    for (int64_t i = 0; i < n_rows; i++)
        if (ids[i] < 0) { jepa_log("jepa: jepa_predict: negative token id %d\n", ids[i]); return false; }
    for (int i = 0; i < n_context; i++)
        if (ids[i] >= enc_rows) {
            jepa_log("jepa: jepa_predict: context id %d is outside the encoder output (%lld rows)\n", ids[i], (long long) enc_rows);
            return false;
        }
    return true;
}

// AUTO: one temporal slice of the predictor grid with an image modality vector is the 2.1 image path
int resolve_modality(const jepa_model * m, const std::vector<int32_t> & ids, int modality) {
    if (modality != JEPA_MODALITY_AUTO) return modality;
    int64_t max_id = 0;
    for (int32_t v : ids) max_id = std::max<int64_t>(max_id, v);
    return (pred_rope(m, max_id).grid_t == 1 && m->pred.mod_img) ? JEPA_MODALITY_IMAGE : JEPA_MODALITY_VIDEO;
}

std::vector<int32_t> make_ids(const int32_t * context_idx, int n_context, const int32_t * target_idx, int n_target) {
    std::vector<int32_t> ids((size_t) n_context + n_target);
    for (int i = 0; i < n_context; i++) ids[(size_t) i] = context_idx ? context_idx[i] : i;
    for (int i = 0; i < n_target; i++) ids[(size_t) n_context + i] = target_idx ? target_idx[i] : i;
    return ids;
}

}  // namespace

extern "C" int jepa_predict_mod(jepa_context * ctx, const jepa_output * enc, const int32_t * context_idx, int n_context,
                                const int32_t * target_idx, int n_target, int mask_index, int modality, jepa_output * out) {
    if (!ctx || !enc || !enc->data || !out) return -1;
    const jepa_model * m = ctx->model;
    if (!pred_supported(m)) return -1;
    if (modality != JEPA_MODALITY_AUTO && modality != JEPA_MODALITY_VIDEO && modality != JEPA_MODALITY_IMAGE) {
        jepa_log("jepa: jepa_predict: unknown modality %d (JEPA_MODALITY_AUTO/VIDEO/IMAGE)\n", modality);
        return -1;
    }
    const int64_t De = m->hp.enc.embed_dim;
    if (enc->dim != De) {
        jepa_log("jepa: jepa_predict: encoder output has dim %lld, model embed_dim is %lld\n", (long long) enc->dim, (long long) De);
        return -1;
    }
    if (enc->n_tokens <= 0) {
        jepa_log("jepa: jepa_predict: the encoder output holds %lld rows\n", (long long) enc->n_tokens);
        return -1;
    }
    if (n_target <= 0 || n_context < 0) {
        pred_check(ctx, n_context, n_target, nullptr, 0);   // logs the reason
        return -1;
    }
    const std::vector<int32_t> ids = make_ids(context_idx, n_context, target_idx, n_target);
    if (!pred_check(ctx, n_context, n_target, ids.data(), enc->n_tokens)) return -1;
    modality = resolve_modality(m, ids, modality);
    if (hipSetDevice(ctx->device) != hipSuccess || !ensure_pred_workspace(ctx, n_context, n_target)) return -1;
    fwd_workspace & w = *ctx->pws;
    // gather the context rows (src/predictor.cpp:187-191), one upload
    if (n_context > 0) {
        std::vector<float> rows((size_t) n_context * De);
        for (int i = 0; i < n_context; i++) memcpy(rows.data() + (size_t) i * De, enc->data + (size_t) ids[(size_t) i] * De, (size_t) De * 4);
        if (hipMemcpyAsync(w.pin, rows.data(), rows.size() * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            jepa_log("jepa: input upload failed\n");
            return -1;
        }
    }
    const int od = pred_run(ctx, ids.data(), n_context, n_target, mask_index, modality);
    if (od < 0) return -1;
    float * data = (float *) malloc((size_t) n_target * od * 4);
    if (!data) return -1;
    if (hipMemcpyAsync(data, w.pout, (size_t) n_target * od * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        jepa_log("jepa: output download failed\n");
        free(data);
        return -1;
    }
    out->data = data;
    out->n_tokens = n_target;
    out->dim = od;
    return 0;
}

// the historical entry point: video modality (src/predictor.cpp:272-279)
extern "C" int jepa_predict_ex(jepa_context * ctx, const jepa_output * enc, const int32_t * context_idx, int n_context,
                               const int32_t * target_idx, int n_target, int mask_index, jepa_output * out) {
    return jepa_predict_mod(ctx, enc, context_idx, n_context, target_idx, n_target, mask_index, JEPA_MODALITY_VIDEO, out);
}

// mask_index 1 is the HF / Meta default (src/predictor.cpp:281-285)
extern "C" int jepa_predict(jepa_context * ctx, const jepa_output * enc, const int32_t * context_idx, int n_context,
                            const int32_t * target_idx, int n_target, jepa_output * out) {
    return jepa_predict_ex(ctx, enc, context_idx, n_context, target_idx, n_target, 1, out);
}
