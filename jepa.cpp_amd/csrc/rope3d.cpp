// rope3d.cpp - host RoPE tables (see rope3d.h; reference src/rope3d.cpp:9-134).
#include "rope3d.h"

#include <cmath>

int rope3d_axis_dim(int head_dim) { return 2 * ((head_dim / 3) / 2); }

namespace {

// (rescaled) coordinate of grid index `i` along one axis; t is never rescaled (reference
// src/rope3d.cpp:13-28, Meta's interpolate_rope)
float axis_pos(const rope3d_params & p, int axis, int i) {
    float v = (float) i;
    if (!p.interpolate) return v;
    if (axis == 1 && p.grid_h > 1) v = (v * (float) (p.train_grid_h - 1)) / (float) (p.grid_h - 1);
    if (axis == 2 && p.grid_w > 1) v = (v * (float) (p.train_grid_w - 1)) / (float) (p.grid_w - 1);
    return v;
}

}  // namespace

void rope3d_tables(const rope3d_params & p, const int32_t * ids, int64_t n_rows, std::vector<float> & c,
                   std::vector<float> & s, bool signed_sin) {
    const int D = p.head_dim, d = rope3d_axis_dim(D), half = d / 2;
    c.assign((size_t) n_rows * D, 1.0f);
    s.assign((size_t) n_rows * D, 0.0f);
    if (d == 0) return;
    std::vector<float> omega((size_t) half);
    for (int k = 0; k < half; k++) omega[(size_t) k] = 1.0f / powf(p.theta, (float) k / (float) half);
    const int dims[3] = {p.grid_t, p.grid_h, p.grid_w};
    // per-axis rows, cached by grid coordinate
    std::vector<float> ac[3], as[3];
    for (int a = 0; a < 3; a++) {
        ac[a].resize((size_t) dims[a] * d);
        as[a].resize((size_t) dims[a] * d);
        for (int i = 0; i < dims[a]; i++) {
            const float pos = axis_pos(p, a, i);
            for (int j = 0; j < d; j++) {
                const int k = p.variant == 0 ? (j % half) : (j / 2);
                const float ang = pos * omega[(size_t) k];
                ac[a][(size_t) i * d + j] = cosf(ang);
                as[a][(size_t) i * d + j] = sinf(ang);
            }
        }
    }
    const int64_t per_frame = (int64_t) p.grid_h * p.grid_w;
    for (int64_t r = 0; r < n_rows; r++) {
        const int64_t id = ids ? ids[r] : r;
        const int64_t idx[3] = {id / per_frame, (id % per_frame) / p.grid_w, id % p.grid_w};
        float * cr = &c[(size_t) r * D];
        float * sr = &s[(size_t) r * D];
        for (int a = 0; a < 3; a++)
            for (int j = 0; j < d; j++) {
                cr[a * d + j] = ac[a][(size_t) idx[a] * d + j];
                sr[a * d + j] = as[a][(size_t) idx[a] * d + j];
            }
        if (signed_sin)
            for (int j = 0; j < D; j += 2) sr[j] = -sr[j];
    }
}
