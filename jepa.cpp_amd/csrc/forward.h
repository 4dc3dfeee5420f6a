// forward.h - the encoder's device workspace, the per-kernel timer and the transformer block that
// the encoder (forward.cpp) and the attentive-pool head (head.cpp) both enqueue.
#pragma once
#include "model.h"
#include "kernels.h"

#include <string>
#include <vector>

struct fwd_workspace {
    // shape the buffers and the captured graph were made for
    int n_items = 0, n_chans = 0, n_frames = 0, height = 0, width = 0;
    int64_t R = 0, Np = 0, R_pad = 0, K = 0, prefix = 0;
    bool image_path = false, video = false;
    int tubelet = 1;
    const jepa_model * model = nullptr;
    // buffers
    std::vector<void *> allocs;
    void * clip = nullptr;       // f32 input (host-input path)
    void * patches = nullptr;    // f16 or f32 patch rows
    float * x = nullptr;         // residual stream
    act_view actA, actB;         // GEMM inputs (LN outputs / attention output codes; up-GEMM output codes)
    void * Q = nullptr, * Kt = nullptr, * Vt = nullptr;
    float * attn = nullptr, * ff = nullptr, * out = nullptr;
    float * rope_c = nullptr, * rope_s = nullptr;
    gemm_split_ws split;         // split-K GEMM scratch (counters zeroed once, left zero by every launch)
    // attentive-pool head (head.cpp): query projection, pooled token, padded logits, pool partials
    float * hq = nullptr, * hy = nullptr, * hlog = nullptr, * hpart = nullptr;
    int64_t hpart_n = 0;
    // masked predictor (predict.cpp): context rows in, target rows out, context embedding input codes
    int n_ctx = 0, n_tgt = 0;
    float * pin = nullptr, * pout = nullptr;
    act_view actC;
    // graph
    hipGraphExec_t exec = nullptr;
    const float * g_in = nullptr; float * g_out = nullptr;
    bool graph_ok = false;

    void release() {
        if (exec) { hipGraphExecDestroy(exec); exec = nullptr; }
        for (void * p : allocs) hipFree(p);
        allocs.clear();
        graph_ok = false;
    }
    ~fwd_workspace() { release(); }
};

struct ktimer {   // optional per-kernel-class event timing (jepa_amd_context_set_kernel_timing)
    jepa_context * ctx;
    struct rec { std::string name, detail; hipEvent_t a, b; };
    std::vector<rec> evs;
    // the launch counts under `name` and, when given, also under "name.detail" (e.g. gemm_q8.qkv)
    template <typename F> void run(const char * name, F && f, const char * detail = nullptr) {
        if (!ctx->kernel_timing) { f(); return; }
        hipEvent_t a, b;
        hipEventCreate(&a); hipEventCreate(&b);
        hipEventRecord(a, ctx->stream);
        f();
        hipEventRecord(b, ctx->stream);
        evs.push_back({name, detail ? std::string(name) + "." + detail : std::string(), a, b});
    }
    void collect() {
        for (auto & e : evs) {
            hipEventSynchronize(e.b);
            float ms = 0;
            hipEventElapsedTime(&ms, e.a, e.b);
            for (const std::string * k : {&e.name, &e.detail}) {
                if (k->empty()) continue;
                auto & st = ctx->kstats[*k];
                st.first += 1;
                st.second += ms;
            }
            hipEventDestroy(e.a);
            hipEventDestroy(e.b);
        }
        evs.clear();
    }
};

// shape of a transformer block: width, heads, head width, stored head width of Q / K / V^T (64 for
// 32-wide heads, see gemm_epi::hds), LayerNorm epsilon
struct blk_shape {
    int64_t D = 0;
    int H = 0, hd = 0, hds = 0;
    float eps = 1e-6f;
};
blk_shape enc_blk_shape(const jepa_model * m);

const char * gemm_class(const dev_linear & W);
// a device buffer owned by the workspace (freed with it); logs and returns false on failure
bool ws_alloc(fwd_workspace & w, void ** p, size_t bytes);
// GEMM input buffers of `rows` rows of K values in any activation format
bool ws_alloc_act(fwd_workspace & w, act_view & a, int64_t rows, int64_t K);
// the residual-stream / block buffers of n_items x R rows: x, actA (D), actB (F), Q / K / V^T
// (H heads stored hds wide, zero-padded to R_pad rows), attn, ff, out and the split-K scratch, for
// blocks of width D, FFN F
bool ws_alloc_blocks(fwd_workspace & w, int64_t n_items, int64_t R, int64_t D, int64_t F, int H, int hds, hipStream_t s);
// out = codes of gelu(x W^T + b) in the input format of the linear that consumes them (`out.fmt`),
// through the GEMM's fused GELU + quantize epilogue (or f32 + the quantizer: w.ff holds rows x n_out)
void enqueue_gemm_gelu(const dev_linear & W, const act_view & x, int64_t rows, act_view & out, fwd_workspace & w, hipStream_t s,
                       ktimer & kt, const char * what);
// MLP half of a block on the residual rows x [rows][D] (any f32 stream of the workspace's row count or
// fewer): x += down(gelu(up(LN(x)))) [* ls], through w.actA / w.actB / w.ff
void enqueue_mlp(const dev_linear & up, const dev_linear & down, const float * ln_w, const float * ln_b, float eps, const float * ls,
                 float * x, int64_t rows, int64_t D, fwd_workspace & w, hipStream_t s, ktimer & kt);
// One pre-LN transformer block on the workspace's residual stream w.x [n_items * R][D]
// (reference src/jepa.cpp:444-471): x += out(attn(rope(qkv(LN1 x)))) [* ls1]; x += down(gelu(up(LN2 x))) [* ls2].
// rope_c / rope_s null: no rotation; slot_rows > 0: block-causal attention after n_prefix rows.
void enqueue_block(const blk_shape & b, const dev_layer & L, fwd_workspace & w, int64_t n_items, int64_t R, const float * rope_c,
                   const float * rope_s, int n_prefix, int64_t slot_rows, hipStream_t s, ktimer & kt);
