/*
 * jepa.h - C API of the MI355X encoder library (libjepa.so).
 *
 * Declaration-compatible with aselimc/jepa.cpp include/jepa.h (v0.5.0): every struct has the same
 * fields in the same order and every entry point has the same name, argument types and return
 * type, so a caller compiled against that header (tools/jepa-bench.cpp, tools/jepa-embed.cpp, the
 * ctypes binding in python/src/jepa_cpp/_api.py) links against this library unchanged.
 *
 * What is implemented on the GPU: the ViT encoder forward of the image families (hfvit / ijepa /
 * lewm encoder part) and of the video families (vjepa2 / vjepa2_1 / levjepa), i.e. jepa_encode, the
 * attentive-pool head (jepa_head, jepa_head_ex), the masked predictor (jepa_predict, _ex, _mod), the
 * preprocessing entry points and image loading (PNG, PPM / PGM, baseline JPEG), plus the model
 * loader, introspection, device selection, pooling and diagnostics. Entry points that belong to the
 * other subsystems of the reference (LeWM and V-JEPA 2-AC world models, H-JEPA, planners, the LeWM
 * projector) are exported so that callers link, and return -1 / NULL / 0 with a message in
 * jepa_error_text().
 *
 * Conventions shared with the reference (include/jepa.h:612-647): a jepa_model is immutable after
 * load and may be shared; a jepa_context belongs to one thread; failures return -1 or NULL and the
 * reason is written to stderr and to a thread-local buffer read by jepa_error_text(); passing NULL
 * to any entry point is defined (an error or a no-op).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* opaque handles - reference include/jepa.h:11-12 */
typedef struct jepa_model   jepa_model;
typedef struct jepa_context jepa_context;

/* K/V dtype inside attention - reference include/jepa.h:14 */
enum { JEPA_KV_AUTO = 0, JEPA_KV_F16 = 1, JEPA_KV_F32 = 2 };

/* reference include/jepa.h:16-23 (same fields, same order) */
typedef struct {
    int   n_threads;      /* CPU threads of the oracle path; ignored on the GPU */
    bool  use_flash_attn; /* true: fused attention kernel (the only GPU path) */
    bool  verbose;
    int   flash_kv;       /* JEPA_KV_*; the GPU kernel always holds K/V in f16 */
} jepa_context_params;

/* reference include/jepa.h:26-29: NCTHW float32, already normalized */
typedef struct {
    const float * data;
    int n_batch, n_chans, n_frames, height, width;
} jepa_input;

/* reference include/jepa.h:31-35: malloc'd rows, freed with jepa_free */
typedef struct {
    float * data;
    int64_t n_tokens;
    int64_t dim;
} jepa_output;

/* ---- lifecycle: reference include/jepa.h:38-45 ---- */
jepa_context_params jepa_context_default_params(void);
jepa_model   * jepa_model_load(const char * gguf_path, bool verbose);
void           jepa_model_free(jepa_model * model);
jepa_context * jepa_context_new(jepa_model * model, jepa_context_params params);
void           jepa_context_free(jepa_context * ctx);
int            jepa_context_n_threads(const jepa_context * ctx);
/* Device time (ms, hipEvents on the context stream) of the forward of the last jepa_encode call:
 * the reference's "graph compute" window, i.e. without host patchify, uploads and downloads. */
double         jepa_context_last_compute_ms(const jepa_context * ctx);

/* ---- introspection: reference include/jepa.h:48-67 ---- */
const char * jepa_model_family(const jepa_model * model);
const char * jepa_model_name(const jepa_model * model);
int          jepa_model_embed_dim(const jepa_model * model);
int          jepa_model_patch_size(const jepa_model * model);
int          jepa_model_tubelet_size(const jepa_model * model);
int          jepa_model_img_size(const jepa_model * model);
int          jepa_model_n_frames(const jepa_model * model);
int          jepa_model_n_layer(const jepa_model * model);
int          jepa_model_n_head(const jepa_model * model);
bool         jepa_model_has_cls(const jepa_model * model);
int          jepa_model_n_registers(const jepa_model * model);
int          jepa_model_n_prefix_tokens(const jepa_model * model);
bool         jepa_model_has_predictor(const jepa_model * model);
bool         jepa_model_has_head(const jepa_model * model);
bool         jepa_model_has_projector(const jepa_model * model);
int          jepa_model_n_classes(const jepa_model * model);
const char * jepa_model_label(const jepa_model * model, int idx);
int          jepa_model_file_type(const jepa_model * model);
const char * jepa_model_file_type_name(const jepa_model * model);
size_t       jepa_model_n_bytes(const jepa_model * model);

/* ---- preprocessing: reference include/jepa.h:70-103 ---- */
enum { JEPA_RESAMPLE_BILINEAR = 0, JEPA_RESAMPLE_BICUBIC = 1 };
enum { JEPA_RESIZE_SHORTEST_EDGE = 0, JEPA_RESIZE_SQUASH = 1 };

typedef struct {
    float mean[3];
    float std[3];
    int   resize_short;
    int   crop;
    int   resample;       /* JEPA_RESAMPLE_* */
    int   resize_mode;    /* JEPA_RESIZE_* */
    float rescale;
    bool  fused_norm;
} jepa_preprocess_params;

/* Returns the model's jepa.pre.* values (used by jepa-bench to normalise synthetic pixels). */
jepa_preprocess_params jepa_preprocess_default_params(const jepa_model * model);
/* Image decoding / resizing is not part of this library: these return NULL with a message. */
float * jepa_preprocess_image_file(const jepa_model * model, const char * path, int * out_h, int * out_w);
float * jepa_preprocess_image_rgb(const jepa_model * model, const uint8_t * rgb, int h, int w, int * out_h, int * out_w);
float * jepa_preprocess_frames_rgb(const jepa_model * model, const uint8_t * const * frames, int n_frames, int h, int w, int * out_h, int * out_w);
float * jepa_preprocess_image_rgb_ex(const jepa_preprocess_params * p, const uint8_t * rgb, int h, int w, int * out_h, int * out_w);
float * jepa_preprocess_frames_rgb_ex(const jepa_preprocess_params * p, const uint8_t * const * frames, int n_frames, int h, int w, int * out_h, int * out_w);
uint8_t * jepa_load_image_rgb(const char * path, int * h, int * w);
void jepa_resize_antialias_u8(const uint8_t * src, int h, int w, int c, uint8_t * dst, int out_h, int out_w, int resample);
void    jepa_free(void * p);

/* ---- inference: reference include/jepa.h:105-127 ---- */
/* Encoder forward -> [n_tokens, embed_dim] after the final norm (reference src/jepa.cpp:1183-1224). */
int jepa_encode(jepa_context * ctx, const jepa_input * in, jepa_output * out);
int jepa_pool_mean(const jepa_model * model, const jepa_output * enc, jepa_output * out);
int jepa_pool_cls(const jepa_model * model, const jepa_output * enc, jepa_output * out);
int jepa_lewm_project(jepa_context * ctx, const jepa_output * enc, jepa_output * out);
int jepa_lewm_project_rows(jepa_context * ctx, const float * cls_rows, int n_rows, jepa_output * out);
int jepa_head(jepa_context * ctx, const jepa_output * enc, jepa_output * out);
int jepa_predict(jepa_context * ctx, const jepa_output * enc,
                 const int32_t * context_idx, int n_context,
                 const int32_t * target_idx,  int n_target, jepa_output * out);

/* ---- video encoders / head: reference include/jepa.h:134-150 ---- */
int64_t jepa_token_grid(const jepa_model * model, int n_frames, int height, int width, int * gt, int * gh, int * gw);
int jepa_head_ex(jepa_context * ctx, const jepa_output * enc, jepa_output * pooled, jepa_output * logits);
void jepa_softmax(const float * logits, int n, float * probs);
int  jepa_top_k(const float * logits, int n, int k, int32_t * idx);

/* ---- misc: reference include/jepa.h:153-154 ---- */
const char * jepa_version(void);
void jepa_print_system_info(void);

/* ---- predictors & world models: reference include/jepa.h:161-273 (not implemented here) ---- */
int jepa_predict_ex(jepa_context * ctx, const jepa_output * enc,
                    const int32_t * context_idx, int n_context,
                    const int32_t * target_idx,  int n_target,
                    int mask_index, jepa_output * out);
enum { JEPA_MODALITY_AUTO = 0, JEPA_MODALITY_VIDEO = 1, JEPA_MODALITY_IMAGE = 2 };
int jepa_predict_mod(jepa_context * ctx, const jepa_output * enc,
                     const int32_t * context_idx, int n_context,
                     const int32_t * target_idx,  int n_target,
                     int mask_index, int modality, jepa_output * out);
int jepa_lewm_n_frames(const jepa_model * model);
int jepa_lewm_action_dim(const jepa_model * model);
int jepa_lewm_predict(jepa_context * ctx, const float * embs, const float * actions,
                      int n_frames, jepa_output * out);
int jepa_lewm_rollout(jepa_context * ctx, const float * embs, int n_seed,
                      const float * actions, int n_steps, float * out);
int jepa_hjepa_n_levels(const jepa_model * model);
int jepa_hjepa_embed_dim(const jepa_model * model, int level);
int jepa_hjepa_action_dim(const jepa_model * model, int level);
int jepa_hjepa_action_embed_dim(const jepa_model * model, int level);
int jepa_hjepa_stride(const jepa_model * model, int level);
int jepa_hjepa_n_frames(const jepa_model * model, int level);
int jepa_hjepa_proprio_dim(const jepa_model * model);
int jepa_hjepa_raw_action_dim(const jepa_model * model);
int jepa_hjepa_frameskip(const jepa_model * model);
int jepa_hjepa_norm_stats(const jepa_model * model, const char * column, float * mean, float * std, int capacity);
int jepa_hjepa_action_prior(const jepa_model * model, int level, float * out, int capacity);
int jepa_hjepa_embed(jepa_context * ctx, const float * cls_rows, const float * proprio, int n_rows, jepa_output * out);
int jepa_hjepa_lift(jepa_context * ctx, int level, const float * below, int n_rows, jepa_output * out);
int jepa_hjepa_action_embed(jepa_context * ctx, int level, const float * actions, int n_rows, jepa_output * out);
int jepa_hjepa_action_encode(jepa_context * ctx, int level, const float * below_act_emb, int n_rows, jepa_output * out);
int jepa_hjepa_predict(jepa_context * ctx, int level, const float * states, const float * actions,
                       int n_frames, jepa_output * out);
int jepa_hjepa_rollout(jepa_context * ctx, int level, const float * states, int n_seed,
                       const float * actions, int n_steps, int history, float * out);

/* ---- H-JEPA planning: reference include/jepa.h:283-373 (not implemented here) ---- */
#define JEPA_HJEPA_MAX_PLAN_LEVELS 8

typedef struct jepa_hjepa_level_plan {
    int   horizon;
    int   pre_decay_horizon;
    int   n_samples;
    int   n_steps;
    float lr, weight_decay;
    float var_scale;
    float action_noise;
    float action_clip_sigma;
    int   min_its;
    int   early_stop_patience;
    float early_stop_rel_delta;
    int   cost_last_n;
    float intermediate_cost_weight;
    float action_cost_weight;
    int   num_subgoals;
    int   horizon_one_goal_upper;
} jepa_hjepa_level_plan;
jepa_hjepa_level_plan jepa_hjepa_level_plan_default(void);

typedef void (*jepa_randn_fn)(void * user, float * out, size_t n);

typedef struct jepa_hjepa_goal {
    const float * states;
    int           n_states;
    int           level;
    int           dense;
    const float * actions;
} jepa_hjepa_goal;

int jepa_hjepa_plan_cost(jepa_context * ctx, int level, const float * state, const jepa_hjepa_goal * goal,
                         const jepa_hjepa_level_plan * plan, const float * actions, int n_samples,
                         int horizon, float * costs, float * grad);
int jepa_hjepa_solve(jepa_context * ctx, int level, const float * state, const jepa_hjepa_goal * goal,
                     const jepa_hjepa_level_plan * plan, jepa_randn_fn randn, void * randn_user,
                     float * actions, float * states, float * cost, int * iters);
int jepa_hjepa_horizons(const jepa_model * model, const jepa_hjepa_level_plan * levels, int n_levels,
                        int replanning_interval, int eval_budget, int steps_taken, int * horizons);

typedef struct jepa_hjepa_plan_info {
    int   planned[JEPA_HJEPA_MAX_PLAN_LEVELS];
    int   goal_level[JEPA_HJEPA_MAX_PLAN_LEVELS];
    int   iters[JEPA_HJEPA_MAX_PLAN_LEVELS];
    float cost[JEPA_HJEPA_MAX_PLAN_LEVELS];
} jepa_hjepa_plan_info;

int jepa_hjepa_plan(jepa_context * ctx, const float * const * states, const float * const * goals,
                    const jepa_hjepa_level_plan * levels, int n_levels, jepa_randn_fn randn,
                    void * randn_user, float * actions, jepa_hjepa_plan_info * info);

/* ---- V-JEPA 2-AC world model: reference include/jepa.h:386-523 (not implemented here) ---- */
int  jepa_ac_tokens_per_frame(const jepa_model * model);
int  jepa_ac_action_dim(const jepa_model * model);
int  jepa_ac_state_dim(const jepa_model * model);
int  jepa_ac_max_frames(const jepa_model * model);
bool jepa_ac_normalize_reps(const jepa_model * model);
void jepa_ac_normalize(const jepa_model * model, float * rows, int64_t n_rows, int64_t dim);
int jepa_ac_predict(jepa_context * ctx, const float * context, int n_frames, int n_batch,
                    const float * actions, const float * states, jepa_output * out);
int jepa_ac_predict_all(jepa_context * ctx, const float * context, int n_frames, int n_batch,
                        const float * actions, const float * states, jepa_output * out);
int jepa_ac_rollout(jepa_context * ctx, const float * context, int n_seed, const float * seed_states,
                    const float * actions, const float * states, int n_cand, int horizon, float * out);
int jepa_ac_rollout_ex(jepa_context * ctx, const float * context, int n_seed,
                       const float * seed_actions, const float * seed_states,
                       const float * actions, const float * states,
                       int n_cand, int horizon, float * out);

typedef struct jepa_ac_context jepa_ac_context;
jepa_ac_context * jepa_ac_context_new(jepa_context * ctx, const float * latents, int n_frames,
                                      const float * actions, const float * states);
void jepa_ac_context_free(jepa_ac_context * handle);
int  jepa_ac_context_n_frames(const jepa_ac_context * handle);
int  jepa_ac_context_capacity(const jepa_ac_context * handle);
int  jepa_ac_context_update(jepa_ac_context * handle, const float * latents, const float * action,
                            const float * state);
int  jepa_ac_context_trim(jepa_ac_context * handle, int n_keep);
int  jepa_ac_rollout_cached(jepa_context * ctx, jepa_ac_context * handle,
                            const float * actions, const float * states,
                            int n_cand, int horizon, float * out);

typedef struct {
    int   samples;
    int   topk;
    int   cem_steps;
    int   horizon;
    float maxnorm;
    float gripper_clamp;
    float momentum_mean, momentum_std;
    float momentum_mean_gripper, momentum_std_gripper;
    float round_gripper;
    uint32_t seed;
} jepa_ac_cem_params;

jepa_ac_cem_params jepa_ac_cem_default_params(void);
int jepa_ac_plan(jepa_context * ctx, jepa_ac_context * handle, const float * goal,
                 const jepa_ac_cem_params * params, const float * noise,
                 float * out_actions, float * out_energy);
void jepa_ac_next_state(const jepa_model * model, const float * state, const float * action, float * out);
void jepa_ac_energy(const float * pred, const float * goal, int n_batch, int64_t n_rows, int64_t dim,
                    float * out);

/* ---- encoder batching: reference include/jepa.h:539-544 ---- */
void jepa_context_set_max_batch(jepa_context * ctx, int n);
int  jepa_context_max_batch(const jepa_context * ctx);
int  jepa_context_last_batch(const jepa_context * ctx);

/* ---- devices: reference include/jepa.h:554-594 ---- */
/* device -1 = the default device (HIP device 0; this library has no CPU backend, so the reference's
 * "cpu" choice also lands on device 0), >= 0 = the n-th HIP device. */
typedef struct {
    bool verbose;
    int  device;
} jepa_model_params;

/* device from $JEPA_DEVICE: "cpu" | "cuda:N" | "gpu:N" | "hip:N" | "N" (reference src/jepa.cpp:107-132) */
jepa_model_params jepa_model_default_params(void);
jepa_model * jepa_model_load_ex(const char * gguf_path, const jepa_model_params * params);

int          jepa_device_count(void);
const char * jepa_device_name(int device);         /* "HIP0", ... */
const char * jepa_device_description(int device);  /* the HIP device name, e.g. "AMD Instinct MI355X" */
void         jepa_device_memory(int device, size_t * free_bytes, size_t * total_bytes);

int          jepa_model_device(const jepa_model * model);
const char * jepa_model_device_name(const jepa_model * model);
bool         jepa_model_is_gpu(const jepa_model * model);

/* Accumulation is always f32 on this GPU path; the flag is kept and reported for callers. */
void jepa_context_set_mul_mat_prec_f32(jepa_context * ctx, bool on);
bool jepa_context_mul_mat_prec_f32(const jepa_context * ctx);

/* ---- diagnostics capture: reference include/jepa.h:609-610 ---- */
void         jepa_error_reset(void);
const char * jepa_error_text(void);

#ifdef __cplusplus
}
#endif
