// forward.cpp - encoder forward on one HIP device: workspace, kernel sequence, hipGraph replay.
//
// The sequence is the reference's graph (src/jepa.cpp:444-471 block, 586-627 image encoder,
// 846-895 video encoder) with producer/consumer fusion:
//   patchify -> patch-embed GEMM (+bias, +modality / +pos, CLS row)          = x (f32 residual stream)
//   per block: LN1 -> q8 codes | qkv GEMM + bias + 3-D RoPE -> Q, K, V^T (f16)
//              flash attention -> f32 | codes | out GEMM + bias (* ls1) + residual into x
//              LN2 -> codes | up GEMM + bias + GELU(erf) -> codes of the down GEMM's input
//              down GEMM + bias (* ls2) + residual into x
//   final LN -> f32 output rows
// The whole sequence for one input shape is captured once into a hipGraph and replayed.
#include "forward.h"
#include "rope3d.h"

#include <algorithm>
#include <cinttypes>
#include <cmath>
#include <cstring>

#define HIP_OK(expr) \
    do { hipError_t e_ = (expr); if (e_ != hipSuccess) { jepa_log("jepa: %s failed: %s\n", #expr, hipGetErrorString(e_)); return false; } } while (0)

jepa_context::jepa_context() = default;

jepa_context::~jepa_context() {
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
    hipSetDevice(device);
    ws.reset();
    if (io_in) hipFree(io_in);
    if (io_out) hipFree(io_out);
    if (ev0) hipEventDestroy(ev0);
    if (ev1) hipEventDestroy(ev1);
    if (stream) hipStreamDestroy(stream);
}

bool video_shape_for(const jepa_model * m, int n_frames, int height, int width, video_shape & vs, bool log) {
    const enc_hparams & e = m->hp.enc;
    const int P = e.patch_size;
    if (P <= 0 || n_frames <= 0 || height <= 0 || width <= 0) return false;
    if (height % P != 0 || width % P != 0) {
        if (log) jepa_log("jepa: input %dx%d is not a multiple of the patch size %d\n", height, width, P);
        return false;
    }
    vs.image_path = false;
    vs.tubelet = e.tubelet_size > 0 ? e.tubelet_size : 1;
    if (n_frames == 1 && e.image_patch_embed && m->patch_img.w) { vs.image_path = true; vs.tubelet = 1; }   // src/jepa.cpp:771-775
    if (n_frames % vs.tubelet != 0) {
        if (log) jepa_log("jepa: %d frames is not a multiple of the tubelet size %d (an image has to be fed to this model as a %d-frame clip, i.e. repeated)\n",
                          n_frames, vs.tubelet, vs.tubelet);
        return false;
    }
    vs.gt = n_frames / vs.tubelet;
    vs.gh = height / P;
    vs.gw = width / P;
    vs.n_prefix = (e.cls_token ? 1 : 0) + e.n_registers;
    vs.n_tokens = (int64_t) vs.gt * vs.gh * vs.gw;
    vs.patch_dim = (int64_t) e.in_chans * vs.tubelet * P * P;
    const dev_linear & pe = vs.image_path ? m->patch_img : m->patch;
    if (!pe.w || pe.n_in != vs.patch_dim) {
        if (log) jepa_log("jepa: patch embedding %s takes rows of %lld values, this shape needs %lld\n",
                          vs.image_path ? "enc.patch_embed_img.weight" : "enc.patch_embed.weight", pe.w ? (long long) pe.n_in : 0LL,
                          (long long) vs.patch_dim);
        return false;
    }
    return true;
}

int64_t encode_rows(const jepa_model * m, int n_batch, int n_frames, int height, int width, int64_t * n_items) {
    const enc_hparams & e = m->hp.enc;
    if (is_video_family(m->hp.family)) {
        video_shape vs;
        if (!video_shape_for(m, n_frames, height, width, vs, false)) return 0;
        if (n_items) *n_items = n_batch;
        return vs.n_rows();
    }
    if (is_image_family(m->hp.family)) {
        if (e.patch_size <= 0 || height % e.patch_size || width % e.patch_size) return 0;
        if (n_items) *n_items = (int64_t) n_batch * n_frames;
        return (int64_t) (height / e.patch_size) * (width / e.patch_size) + (e.cls_token ? 1 : 0) + e.n_registers;
    }
    return 0;
}

bool ws_alloc(fwd_workspace & w, void ** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    if (hipMalloc(p, bytes) != hipSuccess) {
        jepa_log("jepa: hipMalloc of %.1f MiB for the forward workspace failed\n", bytes / 1048576.0);
        return false;
    }
    w.allocs.push_back(*p);
    return true;
}

bool ws_alloc_act(fwd_workspace & w, act_view & a, int64_t rows, int64_t K) {
    a.ld = K;
    return ws_alloc(w, &a.q, (size_t) rows * K * 4) &&   // f32 worst case (A_F32)
           ws_alloc(w, &a.d, (size_t) rows * std::max<int64_t>(K / 32 * 2, K / 256 * 4) + 16) &&
           ws_alloc(w, &a.bsum, (size_t) rows * (K / 16) * 2 + 16);
}

bool ws_alloc_blocks(fwd_workspace & w, int64_t n_items, int64_t R, int64_t D, int64_t F, int H, int hds, hipStream_t s) {
    w.R = R;
    w.R_pad = (R + 127) / 128 * 128;
    const int64_t rows = n_items * R, qkv = n_items * H * w.R_pad * hds * 2;
    const bool ok = ws_alloc(w, (void **) &w.x, (size_t) rows * D * 4) && ws_alloc_act(w, w.actA, rows, D) && ws_alloc_act(w, w.actB, rows, F) &&
                    ws_alloc(w, &w.Q, (size_t) qkv) && ws_alloc(w, &w.Kt, (size_t) qkv) && ws_alloc(w, &w.Vt, (size_t) qkv) &&
                    ws_alloc(w, (void **) &w.attn, (size_t) rows * D * 4) && ws_alloc(w, (void **) &w.ff, (size_t) rows * F * 4) &&
                    ws_alloc(w, (void **) &w.out, (size_t) rows * D * 4);
    if (!ok) return false;
    gemm_split_ws_size(rows, &w.split.part_floats, &w.split.cnt_n);
    // clips are batched into one forward here, where the reference runs a graph per clip: f16 split-K
    // by tile count would make a clip's rounding depend on how many clips share the call
    w.split.f16_by_tiles = !w.video;
    if (!ws_alloc(w, (void **) &w.split.part, (size_t) w.split.part_floats * 4) ||
        !ws_alloc(w, (void **) &w.split.cnt, (size_t) w.split.cnt_n * 4)) return false;
    launch_fill_zero(w.split.cnt, (size_t) w.split.cnt_n * 4, s);
    // Q/K/V^T padding rows are read by the attention kernel: zero them once (never written again)
    launch_fill_zero(w.Q, (size_t) qkv, s);
    launch_fill_zero(w.Kt, (size_t) qkv, s);
    launch_fill_zero(w.Vt, (size_t) qkv, s);
    return true;
}

blk_shape enc_blk_shape(const jepa_model * m) {
    const enc_hparams & e = m->hp.enc;
    blk_shape b;
    b.D = e.embed_dim; b.H = e.n_head; b.hd = e.head_dim(); b.hds = attention_stored_width(b.hd); b.eps = e.ln_eps;
    return b;
}

const char * gemm_class(const dev_linear & W) {
    switch (W.fmt) { case W_F16: return "gemm_f16"; case W_Q32: return "gemm_q8"; case W_Q40: return "gemm_q4_0"; case W_Q4K: return "gemm_q4k"; default: return "gemm_f32"; }
}

void enqueue_gemm_gelu(const dev_linear & W, const act_view & x, int64_t rows, act_view & out, fwd_workspace & w, hipStream_t s,
                       ktimer & kt, const char * what) {
    const int64_t F = W.n_out;
    gemm_epi ep;
    ep.ldy = F;
    const bool mfma = W.fmt != W_F32;
    if (mfma && out.fmt == A_Q8_0) { ep.kind = EPI_GELU_Q8_0; ep.oq = out.q; ep.od = out.d; }
    else if (mfma && out.fmt == A_Q8_K && F % 256 == 0) { ep.kind = EPI_GELU_Q8_K; ep.oh = out.q; ep.od = out.d; ep.ob = out.bsum; }
    else if (mfma && out.fmt == A_F16) { ep.kind = EPI_GELU_F16; ep.oh = out.q; }
    else { ep.kind = EPI_GELU_F32; ep.y = w.ff; }
    kt.run(gemm_class(W), [&] { launch_gemm(W, x, rows, ep, s, &w.split); }, what);
    if (ep.kind == EPI_GELU_F32)
        kt.run("quantize", [&] { launch_rownorm_quant(w.ff, rows, F, nullptr, nullptr, 0.0f, false, out, s); }, "ff");
}

void enqueue_mlp(const dev_linear & up, const dev_linear & down, const float * ln_w, const float * ln_b, float eps, const float * ls,
                 float * x, int64_t rows, int64_t D, fwd_workspace & w, hipStream_t s, ktimer & kt) {
    w.actA.fmt = up.act();
    kt.run("layernorm", [&] { launch_rownorm_quant(x, rows, D, ln_w, ln_b, eps, true, w.actA, s); });
    w.actB.fmt = down.act();
    enqueue_gemm_gelu(up, w.actA, rows, w.actB, w, s, kt, "up");
    gemm_epi ep;
    ep.kind = EPI_RESID; ep.y = x; ep.ldy = D; ep.ls = ls;
    kt.run(gemm_class(down), [&] { launch_gemm(down, w.actB, rows, ep, s, &w.split); }, "down");
}

void enqueue_block(const blk_shape & b, const dev_layer & L, fwd_workspace & w, int64_t n_items, int64_t R, const float * rope_c,
                   const float * rope_s, int n_prefix, int64_t slot_rows, hipStream_t s, ktimer & kt) {
    const int64_t D = b.D, rows = n_items * R;
    const int H = b.H, hd = b.hd;
    // attention half
    {
        gemm_epi ep;
        ep.kind = EPI_QKV;
        ep.q = w.Q; ep.k = w.Kt; ep.vt = w.Vt;
        ep.rope_c = rope_c; ep.rope_s = rope_s;
        ep.n_head = H; ep.hd = hd; ep.hds = b.hds; ep.D = (int) D; ep.R = R; ep.R_pad = w.R_pad;
        if (!L.qkv_separate) {
            w.actA.fmt = L.qkv.act();
            kt.run("layernorm", [&] { launch_rownorm_quant(w.x, rows, D, L.ln1_w, L.ln1_b, b.eps, true, w.actA, s); });
            kt.run(gemm_class(L.qkv), [&] { launch_gemm(L.qkv, w.actA, rows, ep, s, &w.split); }, "qkv");
        } else {
            // q, k, v one by one (reference src/jepa.cpp:408-414), each on ln1 in its own activation
            // format (the LayerNorm runs again only when the format changes)
            int fmt = -1;
            for (int i = 0; i < 3; i++) {
                const dev_linear & P = L.qkv_part[i];
                if (P.act() != fmt) {
                    fmt = P.act();
                    w.actA.fmt = P.act();
                    kt.run("layernorm", [&] { launch_rownorm_quant(w.x, rows, D, L.ln1_w, L.ln1_b, b.eps, true, w.actA, s); });
                }
                ep.col0 = (int64_t) i * D;
                kt.run(gemm_class(P), [&] { launch_gemm(P, w.actA, rows, ep, s, &w.split); }, "qkv");
            }
        }
    }
    w.actA.fmt = L.out.act();
    if ((w.actA.fmt == A_Q8_0 || w.actA.fmt == A_F16) && (hd == 64 || hd == 32)) {
        // the attention epilogue writes the out-projection's q8_0 or f16 input directly
        kt.run("attention", [&] {
            launch_attention(w.Q, w.Kt, w.Vt, w.actA, n_items, H, hd, R, w.R_pad, 1.0f / sqrtf((float) hd), n_prefix, slot_rows, s);
        });
    } else {
        act_view o;
        o.fmt = A_F32; o.q = w.attn; o.ld = D;
        kt.run("attention", [&] {
            launch_attention(w.Q, w.Kt, w.Vt, o, n_items, H, hd, R, w.R_pad, 1.0f / sqrtf((float) hd), n_prefix, slot_rows, s);
        });
        kt.run("quantize", [&] { launch_rownorm_quant(w.attn, rows, D, nullptr, nullptr, 0.0f, false, w.actA, s); }, "attn");
    }
    {
        gemm_epi ep;
        ep.kind = EPI_RESID; ep.y = w.x; ep.ldy = D; ep.ls = L.ls1;
        kt.run(gemm_class(L.out), [&] { launch_gemm(L.out, w.actA, rows, ep, s, &w.split); }, "out");
    }
    // MLP half
    enqueue_mlp(L.up, L.down, L.ln2_w, L.ln2_b, b.eps, L.ls2, w.x, rows, D, w, s, kt);
}

namespace {

// bytes the workspace needs for n items of R rows (the $JEPA_MAX_GRAPH_MIB guard)
double workspace_bytes(const jepa_model * m, int64_t n_items, int64_t R, int64_t Np, int64_t K) {
    const enc_hparams & e = m->hp.enc;
    const double rows = (double) n_items * (double) R;
    const double D = e.embed_dim, F = e.ffn_dim;
    return rows * (D * 4 * 4 + D * 4 + F * 4 * 2 + 3 * D * 2) + (double) n_items * Np * K * 4;
}

bool ensure_workspace(jepa_context * ctx, int n_items, int n_chans, int n_frames, int height, int width) {
    const jepa_model * m = ctx->model;
    const enc_hparams & e = m->hp.enc;
    fwd_workspace * w = ctx->ws.get();
    if (w && w->model == m && w->n_items == n_items && w->n_chans == n_chans && w->n_frames == n_frames && w->height == height &&
        w->width == width)
        return true;
    ctx->ws.reset(new fwd_workspace());
    w = ctx->ws.get();
    w->model = m;
    w->n_items = n_items; w->n_chans = n_chans; w->n_frames = n_frames; w->height = height; w->width = width;
    w->video = is_video_family(m->hp.family);
    const int P = e.patch_size;
    if (w->video) {
        video_shape vs;
        if (!video_shape_for(m, n_frames, height, width, vs, true)) { ctx->ws.reset(); return false; }
        w->image_path = vs.image_path;
        w->tubelet = vs.tubelet;
        w->Np = vs.n_tokens;
        w->prefix = vs.n_prefix;
        w->K = vs.patch_dim;
    } else {
        w->tubelet = 1;
        w->Np = (int64_t) (height / P) * (width / P);
        w->prefix = (e.cls_token ? 1 : 0) + e.n_registers;
        w->K = (int64_t) e.in_chans * P * P;
    }
    const int64_t D = e.embed_dim, F = e.ffn_dim, H = e.n_head, hd = e.head_dim();
    const dev_linear & pe = w->image_path ? m->patch_img : m->patch;
    const bool ok = ws_alloc(*w, &w->clip, (size_t) n_items * n_chans * (w->video ? n_frames : 1) * height * width * 4) &&
                    ws_alloc(*w, &w->patches, (size_t) n_items * w->Np * w->K * (pe.fmt == W_F32 ? 4 : 2)) &&
                    ws_alloc_blocks(*w, n_items, w->Np + w->prefix, D, F, (int) H, enc_blk_shape(m).hds, ctx->stream);
    if (!ok) { ctx->ws.reset(); return false; }
    if (w->video) {
        rope3d_params rp;
        rp.grid_t = w->n_frames / w->tubelet; rp.grid_h = height / P; rp.grid_w = width / P;
        rp.head_dim = (int) hd;
        rp.theta = e.rope_theta;
        rp.variant = e.rope_freq_layout == "interleaved" ? 1 : 0;   // src/jepa.cpp:810-815
        rp.interpolate = e.rope_interpolate;
        rp.train_grid_h = rp.train_grid_w = e.rope_ref_grid;
        std::vector<float> c, s;
        rope3d_tables(rp, nullptr, w->Np, c, s, true);
        if (w->prefix > 0) {   // prefix rows are not rotated: identity rows (src/jepa.cpp:960-966)
            c.insert(c.begin(), (size_t) w->prefix * hd, 1.0f);
            s.insert(s.begin(), (size_t) w->prefix * hd, 0.0f);
        }
        if (!ws_alloc(*w, (void **) &w->rope_c, c.size() * 4) || !ws_alloc(*w, (void **) &w->rope_s, s.size() * 4)) { ctx->ws.reset(); return false; }
        if (hipMemcpyAsync(w->rope_c, c.data(), c.size() * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
            hipMemcpyAsync(w->rope_s, s.data(), s.size() * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            jepa_log("jepa: RoPE table upload failed\n");
            ctx->ws.reset();
            return false;
        }
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) { jepa_log("jepa: workspace initialisation failed\n"); ctx->ws.reset(); return false; }
    return true;
}

// Enqueue the forward of the workspace's shape on ctx->stream. in: NCTHW f32 of n_items; out: [rows][D].
void enqueue_forward(jepa_context * ctx, const float * in, float * out, float * trace, ktimer & kt) {
    const jepa_model * m = ctx->model;
    const enc_hparams & e = m->hp.enc;
    fwd_workspace & w = *ctx->ws;
    hipStream_t s = ctx->stream;
    const int64_t n_items = w.n_items, R = w.R, D = e.embed_dim, rows = n_items * R;
    const dev_linear & pe = w.image_path ? m->patch_img : m->patch;

    kt.run("patchify", [&] {
        launch_patchify(in, w.patches, pe.fmt != W_F32, n_items, w.n_chans, w.n_frames, w.height, w.width, e.patch_size, w.tubelet,
                        w.video, s);
    });
    {
        act_view pa;
        pa.fmt = pe.act();
        pa.q = w.patches;
        pa.ld = w.K;
        gemm_epi ep;
        ep.kind = EPI_F32;
        ep.y = w.x; ep.ldy = D;
        ep.rin = w.Np; ep.rout = R; ep.pre = w.prefix;
        if (w.video && e.modality_embed) ep.addvec = w.image_path ? m->mod_img : m->mod_video;
        if (!w.video && m->pos_embed) ep.addrows = m->pos_embed;
        kt.run("patch_embed", [&] { launch_gemm(pe, pa, n_items * w.Np, ep, s, &w.split); });
        // CLS and register rows in front: image families add their position rows; the video families
        // give them no position (reference src/jepa.cpp:598-608, 865-880)
        if (w.prefix > 0)
            kt.run("cls", [&] {
                launch_prefix_rows(w.x, e.cls_token ? m->cls_token : nullptr, m->reg_tokens, e.n_registers,
                                   w.video ? nullptr : m->pos_embed, n_items, R, D, s);
            });
    }
    if (trace) launch_copy_f32(w.x, trace, rows * D, s);
    // block-causal attention (levjepa): temporal slots of gh*gw patch rows after the prefix rows
    const int64_t slot_rows = e.attn_mode == "block_causal" ? (int64_t) (w.height / e.patch_size) * (w.width / e.patch_size) : 0;
    const int n_prefix = (int) w.prefix;
    const blk_shape bs = enc_blk_shape(m);
    for (int l = 0; l < e.n_layer; l++) {
        enqueue_block(bs, m->layers[(size_t) l], w, n_items, R, w.rope_c, w.rope_s, n_prefix, slot_rows, s, kt);
        if (trace) launch_copy_f32(w.x, trace + (int64_t) (l + 1) * rows * D, rows * D, s);
    }
    act_view o;
    o.fmt = A_F32; o.q = out; o.ld = D;
    kt.run("layernorm", [&] { launch_rownorm_quant(w.x, rows, D, m->norm_w, m->norm_b, e.ln_eps, true, o, s); });
}

bool check_supported(const jepa_model * m) {
    const enc_hparams & e = m->hp.enc;
    if (!is_video_family(m->hp.family) && !is_image_family(m->hp.family)) {
        jepa_log("jepa: jepa_encode: family '%s' is not implemented on this path\n", m->hp.family_str.c_str());
        return false;
    }
    if (e.n_head * e.head_dim() != e.embed_dim || !attention_supports(e.head_dim())) {
        jepa_log("jepa: jepa_encode: head_dim %d (embed_dim %d / %d heads) is not supported by the attention kernels "
                 "(a multiple of 16 up to 128)\n", e.head_dim(), e.embed_dim, e.n_head);
        return false;
    }
    if (e.embed_dim % 256 != 0 && e.embed_dim % 128 != 0) {
        jepa_log("jepa: jepa_encode: embed_dim %d is not a multiple of 128\n", e.embed_dim);
        return false;
    }
    if (e.embed_dim > 2048 || (e.ffn_dim > 2048 && e.ffn_dim % 256 != 0)) {
        jepa_log("jepa: jepa_encode: embed_dim %d is above the 2048 the row kernels hold\n", e.embed_dim);
        return false;
    }
    if (e.act != ACT_GELU_ERF) {
        jepa_log("jepa: jepa_encode: only the gelu_erf activation is implemented on this path\n");
        return false;
    }
    if (e.attn_mode != "full" && !(e.attn_mode == "block_causal" && is_video_family(m->hp.family))) {
        jepa_log("jepa: jepa_encode: attn_mode '%s' is not implemented on this path\n", e.attn_mode.c_str());
        return false;
    }
    return true;
}

}  // namespace

int64_t encode_device(jepa_context * ctx, const float * in_dev, int n_batch, int n_chans, int n_frames, int height, int width,
                      float * out_dev, int64_t out_cap, float * trace_dev, int64_t trace_cap) {
    jepa_model * m = ctx->model;
    const enc_hparams & e = m->hp.enc;
    if (!check_supported(m)) return -1;
    if (n_chans != e.in_chans) { jepa_log("jepa: input has %d channels, model expects %d\n", n_chans, e.in_chans); return -1; }
    int64_t n_items = 0;
    const int64_t R = encode_rows(m, n_batch, n_frames, height, width, &n_items);
    if (R <= 0) {
        if (is_video_family(m->hp.family)) { video_shape vs; video_shape_for(m, n_frames, height, width, vs, true); }
        else jepa_log("jepa: input %dx%d is not a multiple of the patch size %d\n", height, width, e.patch_size);
        return -1;
    }
    const bool video = is_video_family(m->hp.family);
    if (!video && m->pos_embed && m->pos_rows != R) {
        jepa_log("jepa: token grid %dx%d (+%d prefix) = %lld tokens does not match enc.pos_embed (%lld rows); "
                 "position-table interpolation is not implemented yet - feed a %dx%d input\n",
                 height / e.patch_size, width / e.patch_size, (e.cls_token ? 1 : 0) + e.n_registers, (long long) R, (long long) m->pos_rows, e.img_size,
                 e.img_size);
        return -1;
    }
    const int64_t D = e.embed_dim;
    if (out_cap < n_items * R * D) { jepa_log("jepa: output buffer holds %lld floats, %lld needed\n", (long long) out_cap, (long long) (n_items * R * D)); return -1; }
    // items per pass: the context's batch cap, shrunk to the memory budget
    int64_t bmax = ctx->max_batch > 0 ? ctx->max_batch : JEPA_DEFAULT_MAX_BATCH;
    bmax = std::min<int64_t>(bmax, n_items);
    const size_t budget = ctx->max_graph_bytes ? ctx->max_graph_bytes : JEPA_DEFAULT_MAX_GRAPH_BYTES;
    video_shape vs;
    int64_t Np = R, K = (int64_t) e.in_chans * e.patch_size * e.patch_size;
    if (video && video_shape_for(m, n_frames, height, width, vs, false)) { Np = vs.n_tokens; K = vs.patch_dim; }
    while (bmax > 1 && workspace_bytes(m, bmax, R, Np, K) > (double) budget) bmax /= 2;
    if (workspace_bytes(m, 1, R, Np, K) > (double) budget) {
        jepa_log("jepa: one %lld-row item of '%s' needs about %.1f MiB of device activations, over the %.1f MiB limit - raise "
                 "$JEPA_MAX_GRAPH_MIB or feed a shorter or smaller input\n", (long long) R, m->hp.name.c_str(),
                 workspace_bytes(m, 1, R, Np, K) / 1048576.0, budget / 1048576.0);
        return -1;
    }
    if (trace_dev && trace_cap < n_items * (e.n_layer + 1) * R * D) { jepa_log("jepa: trace buffer too small\n"); return -1; }
    if (trace_dev) bmax = n_items;   // one pass, so the trace layout is [layer][all rows]
    if (hipSetDevice(ctx->device) != hipSuccess) { jepa_log("jepa: hipSetDevice(%d) failed\n", ctx->device); return -1; }

    const int64_t frames_per_item = video ? n_frames : 1;
    const int64_t in_per_item = (int64_t) n_chans * frames_per_item * height * width;
    double total_ms = 0;
    for (int64_t base = 0; base < n_items; base += bmax) {
        const int nb = (int) std::min<int64_t>(bmax, n_items - base);
        // image families are laid out [items][C][1][H][W] for the patchify kernel (gathered below
        // when the caller's input has several frames per batch entry)
        {
            std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
            if (!ensure_workspace(ctx, nb, n_chans, video ? n_frames : 1, height, width)) return -1;
        }
        fwd_workspace & w = *ctx->ws;
        // image families: item `it` is the (b, t) slice; slices of one chunk must be contiguous in
        // memory for the patchify kernel, which indexes ((b*C + c)*T + f): pass the whole input and
        // offset by whole (b) groups when T == 1, otherwise gather into the staging clip.
        const float * src = in_dev;
        int64_t base_items = base;
        if (!video && n_frames > 1) {
            // gather items [base, base+nb) into w.clip as [nb][C][1][H][W]
            for (int64_t j = 0; j < nb; j++) {
                const int64_t it = base + j, b = it / n_frames, t = it % n_frames;
                for (int c = 0; c < n_chans; c++) {
                    const float * p = in_dev + (((b * n_chans + c) * n_frames + t) * height) * width;
                    if (hipMemcpyAsync((float *) w.clip + ((j * n_chans + c) * (int64_t) height) * width, p, (size_t) height * width * 4,
                                       hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess) {
                        jepa_log("jepa: input gather failed\n");
                        return -1;
                    }
                }
            }
            src = (const float *) w.clip;
            base_items = 0;
        } else {
            src = in_dev + base_items * in_per_item;
        }
        float * dst = out_dev + base * R * D;
        ktimer kt{ctx};
        hipEventRecord(ctx->ev0, ctx->stream);
        if (trace_dev || ctx->kernel_timing || !ctx->use_graph) {
            enqueue_forward(ctx, src, dst, trace_dev, kt);
        } else {
            if (!w.graph_ok || w.g_in != src || w.g_out != dst) {
                std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
                if (w.exec) { hipGraphExecDestroy(w.exec); w.exec = nullptr; }
                w.graph_ok = false;
                hipGraph_t graph = nullptr;
                bool cap = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal) == hipSuccess;
                if (cap) {
                    enqueue_forward(ctx, src, dst, nullptr, kt);
                    cap = hipStreamEndCapture(ctx->stream, &graph) == hipSuccess && graph &&
                          hipGraphInstantiate(&w.exec, graph, nullptr, nullptr, 0) == hipSuccess;
                    if (graph) hipGraphDestroy(graph);
                }
                if (!cap) {
                    // capture is an optimisation: fall back to direct launches (same kernels)
                    hipGetLastError();
                    ctx->use_graph = false;
                    enqueue_forward(ctx, src, dst, nullptr, kt);
                } else {
                    w.graph_ok = true;
                    w.g_in = src;
                    w.g_out = dst;
                }
            }
            if (w.graph_ok && hipGraphLaunch(w.exec, ctx->stream) != hipSuccess) {
                jepa_log("jepa: hipGraphLaunch failed\n");
                return -1;
            }
        }
        hipEventRecord(ctx->ev1, ctx->stream);
        const hipError_t st = hipEventSynchronize(ctx->ev1);
        if (st != hipSuccess) { jepa_log("jepa: forward failed on device %d: %s\n", ctx->device, hipGetErrorString(st)); return -1; }
        const hipError_t le = hipGetLastError();
        if (le != hipSuccess) { jepa_log("jepa: kernel launch failed: %s\n", hipGetErrorString(le)); return -1; }
        float ms = 0;
        hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1);
        total_ms += ms;
        kt.collect();
    }
    ctx->last_compute_ms = total_ms;
    ctx->last_batch = video ? 1 : (int) bmax;
    return R;
}

// Host-input path: upload, run, download (used by jepa_encode).
int64_t encode_host(jepa_context * ctx, const jepa_input * in, float * out_host, int64_t out_cap) {
    jepa_model * m = ctx->model;
    if (!check_supported(m)) return -1;
    const size_t n_in = (size_t) in->n_batch * in->n_chans * in->n_frames * in->height * in->width;
    int64_t n_items = 0;
    const int64_t R = encode_rows(m, in->n_batch, in->n_frames, in->height, in->width, &n_items);
    if (R <= 0) return encode_device(ctx, nullptr, in->n_batch, in->n_chans, in->n_frames, in->height, in->width, nullptr, 0, nullptr, 0);
    const size_t n_out = (size_t) n_items * R * m->hp.enc.embed_dim;
    if ((int64_t) n_out > out_cap) return -1;
    if (hipSetDevice(ctx->device) != hipSuccess) return -1;
    // persistent I/O buffers: stable pointers let the captured graph be replayed call after call
    std::unique_lock<std::recursive_mutex> lk(jepa_hip_mutex());
    if (ctx->io_in_cap < n_in * 4) {
        if (ctx->io_in) hipFree(ctx->io_in);
        ctx->io_in = nullptr; ctx->io_in_cap = 0;
        if (hipMalloc(&ctx->io_in, n_in * 4) != hipSuccess) { jepa_log("jepa: hipMalloc(input %.1f MiB) failed\n", n_in * 4 / 1048576.0); return -1; }
        ctx->io_in_cap = n_in * 4;
    }
    if (ctx->io_out_cap < n_out * 4) {
        if (ctx->io_out) hipFree(ctx->io_out);
        ctx->io_out = nullptr; ctx->io_out_cap = 0;
        if (hipMalloc(&ctx->io_out, n_out * 4) != hipSuccess) { jepa_log("jepa: hipMalloc(output %.1f MiB) failed\n", n_out * 4 / 1048576.0); return -1; }
        ctx->io_out_cap = n_out * 4;
    }
    lk.unlock();
    float * din = (float *) ctx->io_in, * dout = (float *) ctx->io_out;
    int64_t r = -1;
    if (hipMemcpyAsync(din, in->data, n_in * 4, hipMemcpyHostToDevice, ctx->stream) == hipSuccess) {
        r = encode_device(ctx, din, in->n_batch, in->n_chans, in->n_frames, in->height, in->width, dout, (int64_t) n_out, nullptr, 0);
        if (r > 0 && (hipMemcpyAsync(out_host, dout, n_out * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
                      hipStreamSynchronize(ctx->stream) != hipSuccess)) {
            jepa_log("jepa: output download failed\n");
            r = -1;
        }
    } else {
        jepa_log("jepa: input upload failed\n");
    }
    return r;
}
