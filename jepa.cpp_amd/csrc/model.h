// model.h - internal model / context structures of libjepa (MI355X encoder path).
//
// The hparams mirror the jepa.* GGUF schema the reference parses (src/jepa-internal.h:103-140,
// src/jepa-gguf.cpp:254-596); weights live on one HIP device in layouts chosen for the kernels
// (see dev_linear), not in ggml's.
#pragma once
#include "../../include/jepa.h"
#include "common.h"
#include "gguf.h"

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

// reference src/jepa-internal.h:92-101 (range limits on untrusted metadata)
#define JEPA_LIMIT_EMBED_DIM   65536
#define JEPA_LIMIT_N_LAYER      1024
#define JEPA_LIMIT_N_HEAD       1024
#define JEPA_LIMIT_FFN_DIM   1048576
#define JEPA_LIMIT_PATCH_SIZE    1024
#define JEPA_LIMIT_IMG_SIZE     65536
#define JEPA_LIMIT_N_FRAMES     65536
#define JEPA_LIMIT_IN_CHANS      1024
#define JEPA_LIMIT_N_TOKENS   4194304

#define JEPA_DEFAULT_MAX_BATCH 32
#define JEPA_DEFAULT_MAX_GRAPH_BYTES ((size_t) 8 << 30)

enum family_id { FAM_UNKNOWN = 0, FAM_IJEPA, FAM_VJEPA, FAM_VJEPA2, FAM_VJEPA2_1, FAM_LEVJEPA, FAM_HFVIT, FAM_LEWM, FAM_HJEPA };
enum act_id { ACT_GELU_ERF = 0, ACT_GELU_TANH, ACT_SILU, ACT_RELU };

struct enc_hparams {
    int   embed_dim = 0, n_layer = 0, n_head = 0, ffn_dim = 0;
    int   patch_size = 16, tubelet_size = 1, img_size = 224, n_frames = 1, in_chans = 3;
    float ln_eps = 1e-6f;
    act_id act = ACT_GELU_ERF;
    std::string pos_type;
    float rope_theta = 10000.0f;
    bool  rope_interpolate = false;
    std::string rope_freq_layout;
    int   rope_ref_grid = 0;
    bool  cls_token = false;
    int   n_registers = 0;
    bool  qkv_fused = true;
    bool  modality_embed = false, image_patch_embed = false, layer_scale = false;
    std::string attn_mode = "full";
    bool  has_proj = false;
    int head_dim() const { return n_head > 0 ? embed_dim / n_head : 0; }
    int grid_size() const { return patch_size > 0 ? img_size / patch_size : 0; }
};

struct pre_hparams {
    float mean[3] = {0.485f, 0.456f, 0.406f};
    float std[3]  = {0.229f, 0.224f, 0.225f};
    int   resize_short = 224, crop = 224;
    std::string resample = "bilinear", resize_mode = "shortest_edge";
    float rescale = 1.0f / 255.0f;
};

// jepa.pred.* of the masked predictor (reference src/jepa-internal.h:142-173, src/jepa-gguf.cpp:379-440)
struct pred_hparams {
    std::string kind;              // masked | ac | lewm
    int   embed_dim = 0, n_layer = 0, n_head = 0, ffn_dim = 0, head_dim = 0;
    int   n_mask_tokens = 0, out_dim = 0, grid_size = 0, rope_ref_grid = 0;
    std::string rope_freq_layout;
    bool  rope_interpolate = false, modality_embed = false;
    act_id act = ACT_GELU_ERF;
    int head_dim_eff() const { return head_dim > 0 ? head_dim : (n_head > 0 ? embed_dim / n_head : 0); }
};

struct hparams {
    std::string arch, name, family_str, modality;
    uint32_t file_type = 0;
    family_id family = FAM_UNKNOWN;
    enc_hparams enc;
    pre_hparams pre;
    bool has_pred = false, has_head = false;
    std::string pred_kind, head_kind;
    pred_hparams pred;
    int n_classes = 0, n_pool_layers = 0;
    std::vector<std::string> labels;
};

// Weight formats on the device. Quantized matrices are repacked once at load into the operand
// layout of the GEMM kernel plus their scales: q8_0 as int8 codes for the int8 MFMA; q4_0 and q4_K
// stay 4-bit (codes regrouped for an in-register unpack; q4_K's scales and mins split out) and are
// unpacked in the GEMM for the int8 MFMA. q4_0 rows whose length is not a multiple of 128 (one
// 64-column LDS stage of 4-bit codes would be 32 bytes) are expanded to int8 codes q - 8 instead.
enum wfmt {
    W_F32 = 0, W_F16 = 1,
    W_Q32 = 2,   // int8 codes, f16 scale per 32 (q8_0; q4_0 rows not a multiple of 128)
    W_Q4K = 3,   // q4_K, 4-bit
    W_Q40 = 4,   // q4_0, 4-bit codes, f16 scale per 32
};

// device format of a ggml weight type for rows of n_in values; -1: no GEMM for the type
inline int weight_format(int gtype, int64_t n_in) {
    switch (gtype) {
        case T_F32: return W_F32;
        case T_F16: return W_F16;
        case T_Q8_0: return W_Q32;
        case T_Q4_0: return n_in % 128 == 0 ? W_Q40 : W_Q32;
        case T_Q4_K: return W_Q4K;
        default: return -1;
    }
}

// bytes of the code array dev_linear::w of a quantized format (q4_K: codes, then its sub-block scales)
inline size_t weight_code_bytes(int fmt, int64_t n_out, int64_t n_in) {
    if (fmt == W_Q32) return (size_t) n_out * n_in;
    if (fmt == W_Q40) return (size_t) n_out * (n_in / 2);
    return (size_t) n_out * (n_in / 2) + (size_t) n_out * (n_in / 256) * 8;
}
// Activation formats consumed by the GEMM (what the producer of a linear's input writes).
enum afmt { A_F32 = 0, A_F16 = 1, A_Q8_0 = 2, A_Q8_K = 3 };

struct dev_linear {
    int      gtype = -1;          // ggml type in the file
    int      fmt = W_F32;
    int64_t  n_out = 0, n_in = 0;
    int64_t  n_valid = 0;         // outputs in the file (n_out is rounded up to 128 for the head's linears)
    void *   w = nullptr;         // [n_out][n_in]: f32 (W_F32), int8 (W_Q32), f16 (W_F16); W_Q40: 4-bit codes
                                  // [n_out][n_in/2]; W_Q4K: 4-bit codes [n_out][n_in/2] followed by the 6-bit
                                  // sub-block scales [n_out][n_in/256][8]
    void *   wd = nullptr;        // W_Q32, W_Q40: f16 d [n_out][n_in/32]; W_Q4K: u32 (f16 d | f16 dmin << 16) [n_in/256][n_out]
    void *   wmin = nullptr;      // W_Q4K: f16 mins [n_out][n_in/256][16] (m_{k/2}, k = 0..15)
    float *  bias = nullptr;      // [n_out] or null
    afmt act() const {
        switch (fmt) { case W_F32: return A_F32; case W_F16: return A_F16; case W_Q32: case W_Q40: return A_Q8_0; default: return A_Q8_K; }
    }
};

struct dev_layer {
    float * ln1_w = nullptr, * ln1_b = nullptr, * ln2_w = nullptr, * ln2_b = nullptr;
    float * ls1 = nullptr, * ls2 = nullptr;
    dev_linear qkv, out, up, down;
    // separate attn_q / attn_k / attn_v whose dtypes take different activation formats (f16 beside
    // q8_0, q4_K beside q8_0, ...): three linears run one by one, as the reference runs them; qkv unused
    bool qkv_separate = false;
    dev_linear qkv_part[3];
};

// attentive-pool head (reference src/jepa.cpp:1026-1075, tensors docs/gguf-schema.md:121-137)
struct dev_head {
    std::vector<dev_layer> blocks;   // head.blk.{i}
    float * query = nullptr;         // [D] raw query token
    float * ln_kv_w = nullptr, * ln_kv_b = nullptr, * ln2_w = nullptr, * ln2_b = nullptr;
    dev_linear q, k, v, up, down, cls;   // cls: n_out rounded up to 128, n_valid = n_classes
};

// masked predictor (reference src/predictor.cpp:56-133)
struct dev_pred {
    dev_linear embed;                // pred.embed: encoder width -> predictor width
    dev_linear embed0, embed2;       // or the 2-layer MLP pred.embed.0 / .2 (V-JEPA 2.1 ViT-g/G)
    float * mask_tokens = nullptr;   // [n_mask_rows][Dp]
    int64_t n_mask_rows = 0;
    float * mod_video = nullptr, * mod_img = nullptr;
    float * norm_w = nullptr, * norm_b = nullptr;
    std::vector<dev_layer> blocks;   // pred.blk.{i}
    dev_linear proj;                 // pred.proj: predictor width -> out_dim
};

struct jepa_model {
    std::string path;
    hparams hp;
    std::vector<std::pair<std::string, std::string>> raw_kv;
    int device = 0;                 // HIP device ordinal the weights live on
    size_t n_bytes_weights = 0;     // device bytes of the repacked weights
    size_t n_bytes_file = 0;        // tensor bytes in the file
    // encoder
    dev_linear patch, patch_img;
    float * pos_embed = nullptr; int64_t pos_rows = 0;
    float * cls_token = nullptr;
    float * reg_tokens = nullptr;   // [n_registers][D]
    float * mod_img = nullptr, * mod_video = nullptr;
    float * norm_w = nullptr, * norm_b = nullptr;
    std::vector<dev_layer> layers;
    dev_head head;                   // loaded when jepa.head.kind = attentive_pool
    dev_pred pred;                   // loaded when jepa.pred.kind = masked
    std::vector<void *> allocations;   // every device allocation, freed with the model
};

struct fwd_workspace;   // forward.cpp

struct jepa_context {
    jepa_model * model = nullptr;
    jepa_context_params params{};
    int n_threads = 1;
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_compute_ms = 0;
    int max_batch = 0, last_batch = 1;
    size_t max_graph_bytes = 0;
    bool prec_f32 = true;
    bool use_graph = true;           // capture the forward into a hipGraph and replay it
    std::unique_ptr<fwd_workspace> ws;
    std::unique_ptr<fwd_workspace> hws;   // jepa_head's buffers, made for the last token count
    std::unique_ptr<fwd_workspace> pws;   // jepa_predict's buffers, made for the last context + target count
    void * io_in = nullptr, * io_out = nullptr;   // device copies of jepa_encode's host input / output
    size_t io_in_cap = 0, io_out_cap = 0;
    // per-kernel timing (jepa_amd_context_set_kernel_timing)
    bool kernel_timing = false;
    std::map<std::string, std::pair<int64_t, double>> kstats;
    jepa_context();
    ~jepa_context();
};

// ---- loader (loader.cpp) ----
const char * jepa_file_type_name_u32(uint32_t ft);
family_id family_from_string(const std::string & s);

// ---- devices (device.cpp) ----
int  dev_count();
bool dev_check(int device);        // logs when the device does not exist
int  dev_resolve(int requested);   // -1 -> 0 (this library computes on a GPU)
int  device_from_env();

// ---- encoder shapes (forward.cpp) ----
struct video_shape {
    int tubelet = 1, gt = 0, gh = 0, gw = 0;
    bool image_path = false;
    int n_prefix = 0;
    int64_t n_tokens = 0;    // patch tokens
    int64_t patch_dim = 0;
    int64_t n_rows() const { return n_tokens + n_prefix; }
};
bool video_shape_for(const jepa_model * m, int n_frames, int height, int width, video_shape & vs, bool log);
bool is_video_family(family_id f);
bool is_image_family(family_id f);

// Run the encoder on a device-resident NCTHW clip/batch. in_dev: [n_batch*C*T*H*W] f32.
// out_dev: [rows_total, D] f32 (device). Returns rows per item or -1. Records last_compute_ms.
int64_t encode_device(jepa_context * ctx, const float * in_dev, int n_batch, int n_chans, int n_frames,
                      int height, int width, float * out_dev, int64_t out_cap_floats,
                      float * trace_dev, int64_t trace_cap_floats);
// Rows per item and item count for an input shape (0 when not encodable).
int64_t encode_rows(const jepa_model * m, int n_batch, int n_frames, int height, int width, int64_t * n_items);
// jepa_encode's path: host input -> device -> forward -> host output rows. Returns rows per item or -1.
int64_t encode_host(jepa_context * ctx, const jepa_input * in, float * out_host, int64_t out_cap);
// Attentive-pool head on device-resident encoder rows x_dev [n_tokens][D] f32: pooled_dev [D] and
// logits_dev [n_classes] (device, either may be null). Returns n_classes or -1. Records last_compute_ms.
int head_device(jepa_context * ctx, const float * x_dev, int64_t n_tokens, float * pooled_dev, float * logits_dev);
