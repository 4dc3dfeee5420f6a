// stubs.cpp - entry points of include/jepa.h outside the encoder path.
//
// The reference exports these for its world models (LeWM, V-JEPA 2-AC), H-JEPA, planners and the
// LeWM projector (reference include/jepa.h:69-103, 118-127, 161-523). They are exported here so that
// callers such as tools/jepa-bench.cpp link unchanged; each one reports that it is not part of this
// library and returns its error value. (The attentive-pool head, the masked predictor and image
// decoding are implemented: head.cpp, predict.cpp, image_io.cpp.)
#include "model.h"

#include <cstring>

namespace {
int nope(const char * fn) {
    jepa_log("jepa: %s is not implemented by this library (encoder path only)\n", fn);
    return -1;
}
}  // namespace

#define NOPE_INT(fn) return nope(fn)
#define NOPE_PTR(fn) do { nope(fn); return nullptr; } while (0)

extern "C" {



int jepa_lewm_project(jepa_context *, const jepa_output *, jepa_output *) { NOPE_INT("jepa_lewm_project"); }
int jepa_lewm_project_rows(jepa_context *, const float *, int, jepa_output *) { NOPE_INT("jepa_lewm_project_rows"); }

int jepa_lewm_n_frames(const jepa_model *) { return 0; }
int jepa_lewm_action_dim(const jepa_model *) { return 0; }
int jepa_lewm_predict(jepa_context *, const float *, const float *, int, jepa_output *) { NOPE_INT("jepa_lewm_predict"); }
int jepa_lewm_rollout(jepa_context *, const float *, int, const float *, int, float *) { NOPE_INT("jepa_lewm_rollout"); }

int jepa_hjepa_n_levels(const jepa_model *) { return 0; }
int jepa_hjepa_embed_dim(const jepa_model *, int) { return 0; }
int jepa_hjepa_action_dim(const jepa_model *, int) { return 0; }
int jepa_hjepa_action_embed_dim(const jepa_model *, int) { return 0; }
int jepa_hjepa_stride(const jepa_model *, int) { return 0; }
int jepa_hjepa_n_frames(const jepa_model *, int) { return 0; }
int jepa_hjepa_proprio_dim(const jepa_model *) { return 0; }
int jepa_hjepa_raw_action_dim(const jepa_model *) { return 0; }
int jepa_hjepa_frameskip(const jepa_model *) { return 0; }
int jepa_hjepa_norm_stats(const jepa_model *, const char *, float *, float *, int) { return 0; }
int jepa_hjepa_action_prior(const jepa_model *, int, float *, int) { return 0; }
int jepa_hjepa_embed(jepa_context *, const float *, const float *, int, jepa_output *) { NOPE_INT("jepa_hjepa_embed"); }
int jepa_hjepa_lift(jepa_context *, int, const float *, int, jepa_output *) { NOPE_INT("jepa_hjepa_lift"); }
int jepa_hjepa_action_embed(jepa_context *, int, const float *, int, jepa_output *) { NOPE_INT("jepa_hjepa_action_embed"); }
int jepa_hjepa_action_encode(jepa_context *, int, const float *, int, jepa_output *) { NOPE_INT("jepa_hjepa_action_encode"); }
int jepa_hjepa_predict(jepa_context *, int, const float *, const float *, int, jepa_output *) { NOPE_INT("jepa_hjepa_predict"); }
int jepa_hjepa_rollout(jepa_context *, int, const float *, int, const float *, int, int, float *) { NOPE_INT("jepa_hjepa_rollout"); }

jepa_hjepa_level_plan jepa_hjepa_level_plan_default(void) {
    // the reference's documented defaults (include/jepa.h:311-312)
    jepa_hjepa_level_plan p;
    memset(&p, 0, sizeof(p));
    p.n_samples = 100; p.n_steps = 90; p.lr = 0.1f; p.weight_decay = 0.01f; p.var_scale = 1.0f;
    p.min_its = 30; p.early_stop_patience = 5; p.early_stop_rel_delta = 0.01f; p.cost_last_n = 1;
    p.intermediate_cost_weight = 1.0f; p.num_subgoals = 1;
    return p;
}
int jepa_hjepa_plan_cost(jepa_context *, int, const float *, const jepa_hjepa_goal *, const jepa_hjepa_level_plan *, const float *, int, int,
                         float *, float *) { NOPE_INT("jepa_hjepa_plan_cost"); }
int jepa_hjepa_solve(jepa_context *, int, const float *, const jepa_hjepa_goal *, const jepa_hjepa_level_plan *, jepa_randn_fn, void *,
                     float *, float *, float *, int *) { NOPE_INT("jepa_hjepa_solve"); }
int jepa_hjepa_horizons(const jepa_model *, const jepa_hjepa_level_plan *, int, int, int, int, int *) { NOPE_INT("jepa_hjepa_horizons"); }
int jepa_hjepa_plan(jepa_context *, const float * const *, const float * const *, const jepa_hjepa_level_plan *, int, jepa_randn_fn, void *,
                    float *, jepa_hjepa_plan_info *) { NOPE_INT("jepa_hjepa_plan"); }

int jepa_ac_tokens_per_frame(const jepa_model *) { return 0; }
int jepa_ac_action_dim(const jepa_model *) { return 0; }
int jepa_ac_state_dim(const jepa_model *) { return 0; }
int jepa_ac_max_frames(const jepa_model *) { return 0; }
bool jepa_ac_normalize_reps(const jepa_model *) { return false; }
void jepa_ac_normalize(const jepa_model *, float *, int64_t, int64_t) { nope("jepa_ac_normalize"); }
int jepa_ac_predict(jepa_context *, const float *, int, int, const float *, const float *, jepa_output *) { NOPE_INT("jepa_ac_predict"); }
int jepa_ac_predict_all(jepa_context *, const float *, int, int, const float *, const float *, jepa_output *) { NOPE_INT("jepa_ac_predict_all"); }
int jepa_ac_rollout(jepa_context *, const float *, int, const float *, const float *, const float *, int, int, float *) { NOPE_INT("jepa_ac_rollout"); }
int jepa_ac_rollout_ex(jepa_context *, const float *, int, const float *, const float *, const float *, const float *, int, int, float *) {
    NOPE_INT("jepa_ac_rollout_ex");
}
jepa_ac_context * jepa_ac_context_new(jepa_context *, const float *, int, const float *, const float *) { NOPE_PTR("jepa_ac_context_new"); }
void jepa_ac_context_free(jepa_ac_context *) {}
int jepa_ac_context_n_frames(const jepa_ac_context *) { return 0; }
int jepa_ac_context_capacity(const jepa_ac_context *) { return 0; }
int jepa_ac_context_update(jepa_ac_context *, const float *, const float *, const float *) { NOPE_INT("jepa_ac_context_update"); }
int jepa_ac_context_trim(jepa_ac_context *, int) { NOPE_INT("jepa_ac_context_trim"); }
int jepa_ac_rollout_cached(jepa_context *, jepa_ac_context *, const float *, const float *, int, int, float *) { NOPE_INT("jepa_ac_rollout_cached"); }
jepa_ac_cem_params jepa_ac_cem_default_params(void) {
    jepa_ac_cem_params p;
    memset(&p, 0, sizeof(p));
    return p;
}
int jepa_ac_plan(jepa_context *, jepa_ac_context *, const float *, const jepa_ac_cem_params *, const float *, float *, float *) {
    NOPE_INT("jepa_ac_plan");
}
void jepa_ac_next_state(const jepa_model *, const float *, const float *, float *) { nope("jepa_ac_next_state"); }
void jepa_ac_energy(const float *, const float *, int, int64_t, int64_t, float *) { nope("jepa_ac_energy"); }

}  // extern "C"
