// preprocess.h - shared pieces of the host (preprocess.cpp) and device (preprocess.hip) preprocessing.
#pragma once
#include "../../include/jepa.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

// a shortest-edge resize whose intermediate would exceed this many pixels is refused (the aspect
// ratio, not the file size, makes it large; reference src/preprocess.cpp:195-200)
#define JEPA_PRE_MAX_PIXELS (64ll * 1024 * 1024)

// One axis of a separable uint8 resize, as a compressed-row table: output o reads the inputs
// lo[o], lo[o] + 1, ... with the integer taps taps[beg[o]] .. taps[beg[o + 1] - 1], accumulates
// 2^(shift-1) + sum(tap * pixel) in int32 and keeps clamp(acc >> shift, 0, 255). The rows have
// their own lengths (no padding), and the same arrays are uploaded for the device passes.
struct resample_axis {
    int n_in = 0, n_out = 0, shift = 0;
    std::vector<int32_t> lo;      // [n_out]
    std::vector<int32_t> beg;     // [n_out + 1]
    std::vector<int16_t> taps;    // [beg[n_out]]
    bool identity() const { return n_in == n_out; }
};
resample_axis resample_axis_for(int n_in, int n_out, int resample);

// geometry and normalisation of one preprocessing call
struct pre_plan {
    int rh = 0, rw = 0;        // resized size
    int crop = 0;              // output is crop x crop
    int oy = 0, ox = 0;        // crop pixel (y, x) = resized pixel (y + oy, x + ox), zero outside
    float inv = 255.0f;        // 1 / rescale
    bool fused = true;
    float mean[3] = {0, 0, 0}, stdv[3] = {1, 1, 1};   // fused: mean / rescale and std / rescale
};
bool pre_plan_for(const jepa_preprocess_params * p, int h, int w, pre_plan & g);

// normalised value of channel c of a uint8 pixel (the reference's two formulas, src/preprocess.cpp:283-287)
__host__ __device__ inline float pre_normalize_v(bool fused, float inv, float mean, float stdv, uint8_t v) {
    return fused ? ((float) v - mean) / stdv : ((float) v / inv - mean) / stdv;
}
inline float pre_normalize(const pre_plan & g, int c, uint8_t v) { return pre_normalize_v(g.fused, g.inv, g.mean[c], g.stdv[c], v); }

// device: n_frames HWC uint8 frames [n][h][w][3] (device memory) -> NCTHW floats [3][n][crop][crop]
// (device memory), equal bit for bit to jepa_preprocess_frames_rgb_ex. Tables are built on the host
// and uploaded into `scratch` (see preprocess_scratch_bytes). Returns false on a bad geometry.
size_t preprocess_scratch_bytes(const jepa_preprocess_params * p, const pre_plan & g, int n_frames, int h, int w);
bool launch_preprocess(const jepa_preprocess_params * p, const pre_plan & g, const uint8_t * frames, int n_frames, int h, int w,
                       float * out, void * scratch, hipStream_t s);

// The allocation-free variant's scratch: a static device array of this size on every GPU the library
// runs on (tap tables + the horizontal-pass image of all frames), and its device address on
// `device` (looked up once per device with that device current; nullptr on failure).
#define PRE_NOALLOC_SCRATCH_BYTES ((size_t) 32 << 20)
void * preprocess_static_scratch(int device);
