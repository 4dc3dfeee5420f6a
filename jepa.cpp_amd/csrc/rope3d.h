// rope3d.h - host tables of the V-JEPA 2 / 2.1 3-axis rotary embedding.
//
// Same tables as reference src/rope3d.cpp:9-134 (math spec src/rope3d.h:1-62): per-axis rotated
// width d = 2*((hd/3)/2); dims [0,d) rotate with the frame index, [d,2d) with the row, [2d,3d) with
// the column, the rest are identity (cos 1, sin 0); omega_k = 1/theta^(k/(d/2)) in float32;
// variant 0 (V-JEPA 2, "tiled") uses omega[j % (d/2)], variant 1 (V-JEPA 2.1, "interleaved")
// omega[j/2]; 2.1 interpolation rescales h, w by (ref-1)/(g-1) left to right in float32. The sine
// table carries the rotation's sign on even lanes, so the device applies out = x*C + swap(x)*S'.
#pragma once
#include <cstdint>
#include <vector>

struct rope3d_params {
    int   grid_t = 1, grid_h = 1, grid_w = 1;
    int   head_dim = 64;
    float theta = 10000.0f;
    bool  interpolate = false;
    int   train_grid_h = 0, train_grid_w = 0;
    int   variant = 0;
};

int rope3d_axis_dim(int head_dim);
// [n_rows, head_dim] tables; ids == nullptr means every token of the grid in T-major order
void rope3d_tables(const rope3d_params & p, const int32_t * ids, int64_t n_rows, std::vector<float> & cos_out,
                   std::vector<float> & sin_out, bool signed_sin = true);
