// rownorm_dev.h - one row of LayerNorm + output conversion per wave (the row kernel of misc.hip), in
// a load phase and a normalise / convert / store phase.
//
// A wave owns a row of D floats; lane l holds octets o = l + 64 i (8 consecutive values), so a q8_0
// block (32 values) is 4 adjacent lanes and a q8_K block (256) is 32 adjacent lanes.
//   LayerNorm = ggml_norm (mean, centred variance, both accumulated in double like ggml_float)
//   followed by * w and + b (reference src/jepa.cpp:356-361), then the output conversion:
//   A_Q8_0: d = amax/127 (f16), q = rne(x * 127/amax)        x86 quantize_row_q8_0; int8 codes
//   A_Q8_K: max = first largest-|x| value, iscale = -127/max, q = min(127, rne(iscale*x)),
//           d = 1/iscale (f32), bsums of 16                  quantize_row_q8_K_ref
//   A_F16 / A_F32: the values rounded to f16 / as they are
// The double sums of D floats are exact when every partial sum fits 53 bits: each value is a multiple
// of the unit in the last place of the smallest nonzero |x|, so that holds while max|x| / min|x| <
// 2^30 / D (2^20 at D = 1024; squares: the same bound on the squared values), and then their order
// (a DPP tree here, sequential in ggml) does not change them.
#pragma once
#include "kernels.h"
#include "quant_dev.h"

namespace rowln {

constexpr int MAXOCT = 4;   // D <= 2048 (octets per lane: 1, 2 or 4, by row length)

// Cross-lane moves through DPP (VALU, a few cycles) instead of ds_bpermute shuffles (an LDS round
// trip each). update_dpp(0, v, ...) gives 0 in lanes of rows the row mask leaves out.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_f64(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(0, p.x, CTRL, ROW_MASK, 0xF, false);
    r.y = __builtin_amdgcn_update_dpp(0, p.y, CTRL, ROW_MASK, 0xF, false);
    return __builtin_bit_cast(double, r);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E;                 // quad_perm [1,0,3,2], [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140, DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;

// Sum over the 64 lanes, returned to every lane: within rows of 16 by xor / mirror steps, then
// row 0 -> 1 and 2 -> 3 (row_bcast:15), rows 0+1 -> 3 (row_bcast:31); lane 63 holds the total.
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<DPP_XOR1>(v);
    v += dpp_f64<DPP_XOR2>(v);
    v += dpp_f64<DPP_HALF_MIRROR>(v);
    v += dpp_f64<DPP_MIRROR>(v);
    v += dpp_f64<DPP_BCAST15, 0xA>(v);
    v += dpp_f64<DPP_BCAST31, 0xC>(v);
    const int2 p = __builtin_bit_cast(int2, v);
    return __builtin_bit_cast(double, make_int2(__builtin_amdgcn_readlane(p.x, 63), __builtin_amdgcn_readlane(p.y, 63)));
}

// v_permlane16_swap: lanes of 16-lane rows 2r and 2r+1 exchange; r[0] is the even row's value and
// r[1] the odd row's, in both rows
__device__ __forceinline__ uint2 rows16_pair(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return make_uint2(r[0], r[1]);
}

// Over the 32 lanes of each half-wave, returned to all of them: the largest |x| (am) and, among the
// elements equal to it in magnitude, the first in element order, as key = 2 * index + sign bit.
__device__ __forceinline__ float half_max_f32(float v) {
    v = fmaxf(v, dpp_f32<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f32<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_MIRROR>(v));
    const uint2 r = rows16_pair(__float_as_uint(v));
    return fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t half_min_u32(uint32_t v) {
    v = min(v, dpp_u32<DPP_XOR1>(v));
    v = min(v, dpp_u32<DPP_XOR2>(v));
    v = min(v, dpp_u32<DPP_HALF_MIRROR>(v));
    v = min(v, dpp_u32<DPP_MIRROR>(v));
    const uint2 r = rows16_pair(v);
    return min(r.x, r.y);
}

__device__ __forceinline__ uint16_t f2hbits(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

// The lane's NOCT octets of one row (zero past the row's end)
template <int NOCT>
__device__ __forceinline__ void load_row(const float * xr, int64_t D, int lane, float (&v)[NOCT][8]) {
    const int n_oct = (int) (D / 8);
#pragma unroll
    for (int i = 0; i < NOCT; i++) {
        const int o = lane + 64 * i;
        if (o < n_oct) {
            const float4 a = *(const float4 *) (xr + 8 * o), c = *(const float4 *) (xr + 8 * o + 4);
            v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w; v[i][4] = c.x; v[i][5] = c.y; v[i][6] = c.z; v[i][7] = c.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[i][e] = 0.0f;
        }
    }
}

// the affine parameters of the lane's octets (1 / 0 where absent)
template <int NOCT>
__device__ __forceinline__ void load_affine(const float * w, const float * b, int64_t D, int lane, float (&gw)[NOCT][8],
                                            float (&gb)[NOCT][8]) {
    const int n_oct = (int) (D / 8);
#pragma unroll
    for (int i = 0; i < NOCT; i++) {
        const int o = lane + 64 * i;
        const bool live = o < n_oct;
        const float4 w0 = w && live ? *(const float4 *) (w + 8 * o) : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 w1 = w && live ? *(const float4 *) (w + 8 * o + 4) : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 b0 = b && live ? *(const float4 *) (b + 8 * o) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 b1 = b && live ? *(const float4 *) (b + 8 * o + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        gw[i][0] = w0.x; gw[i][1] = w0.y; gw[i][2] = w0.z; gw[i][3] = w0.w; gw[i][4] = w1.x; gw[i][5] = w1.y; gw[i][6] = w1.z; gw[i][7] = w1.w;
        gb[i][0] = b0.x; gb[i][1] = b0.y; gb[i][2] = b0.z; gb[i][3] = b0.w; gb[i][4] = b1.x; gb[i][5] = b1.y; gb[i][6] = b1.z; gb[i][7] = b1.w;
    }
}

// LayerNorm of the loaded row v in place: ggml_norm, then * w and + b where given
template <int NOCT>
__device__ __forceinline__ void normalize_row(float (&v)[NOCT][8], int64_t D, bool has_w, bool has_b, const float (&gw)[NOCT][8],
                                              const float (&gb)[NOCT][8], float eps, int lane) {
    const int n_oct = (int) (D / 8);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < NOCT; i++)
#pragma unroll
        for (int e = 0; e < 8; e++) s += (double) v[i][e];
    s = wave_sum_f64(s);
    const float mean = (float) s / (float) D;
    double s2 = 0.0;
#pragma unroll
    for (int i = 0; i < NOCT; i++) {
        const bool live = lane + 64 * i < n_oct;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float t = __fsub_rn(v[i][e], mean);
            v[i][e] = t;
            if (live) s2 += (double) __fmul_rn(t, t);
        }
    }
    s2 = wave_sum_f64(s2);
    const float var = (float) (s2 / (double) D);
    const float scale = 1.0f / sqrtf(__fadd_rn(var, eps));
#pragma unroll
    for (int i = 0; i < NOCT; i++) {
        const int o = lane + 64 * i;
        if (o >= n_oct) continue;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float t = __fmul_rn(v[i][e], scale);
            if (has_w) t = __fmul_rn(t, gw[i][e]);
            if (has_b) t = __fadd_rn(t, gb[i][e]);
            v[i][e] = t;
        }
    }
}

// LayerNorm (NORM) of the loaded row v, then the output conversion of row `row` of out
template <int OUT, bool NORM, int NOCT>
__device__ __forceinline__ void finish_row(float (&v)[NOCT][8], int64_t row, int64_t D, bool has_w, bool has_b,
                                           const float (&gw)[NOCT][8], const float (&gb)[NOCT][8], float eps, const act_view & out,
                                           int lane) {
    const int n_oct = (int) (D / 8);
    if constexpr (NORM) normalize_row<NOCT>(v, D, has_w, has_b, gw, gb, eps, lane);
#pragma unroll
    for (int i = 0; i < NOCT; i++) {
        const int o = lane + 64 * i;
        const bool live = o < n_oct;
        if (i * 64 >= n_oct) break;   // uniform across the wave
        if constexpr (OUT == A_F32) {
            if (live) {
                float * dst = (float *) out.q + row * D + 8 * o;
                *(float4 *) dst = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
                *(float4 *) (dst + 4) = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
            }
        } else if constexpr (OUT == A_F16) {
            if (live) {
                typedef _Float16 h8 __attribute__((ext_vector_type(8)));
                h8 hv;
#pragma unroll
                for (int e = 0; e < 8; e++) hv[e] = (_Float16) v[i][e];
                *(h8 *) ((_Float16 *) out.q + row * D + 8 * o) = hv;
            }
        } else if constexpr (OUT == A_Q8_0) {
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) am = fmaxf(am, fabsf(v[i][e]));
            am = fmaxf(am, dpp_f32<DPP_XOR1>(am));      // the 4 lanes of a 32-value block are one quad
            am = fmaxf(am, dpp_f32<DPP_XOR2>(am));
            const float d = am / 127.0f;
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            if (live) {
                uint32_t qb[2] = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    qb[e >> 2] |= q8_byte(v[i][e], id) << (8 * (e & 3));
                }
                *(uint2 *) ((int8_t *) out.q + row * D + 8 * o) = make_uint2(qb[0], qb[1]);
                if ((o & 3) == 0) ((uint16_t *) out.d)[row * (D / 32) + o / 4] = f2hbits(d);
            }
        } else {   // A_Q8_K
            // largest |x| of the 256-block, then the first element of that magnitude (its sign gives
            // the scale's sign): max over the half-wave, then min of 2 * index + sign
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) am = fmaxf(am, fabsf(v[i][e]));
            am = half_max_f32(am);
            uint32_t key = 0xffffffffu;
#pragma unroll
            for (int e = 7; e >= 0; e--)
                if (fabsf(v[i][e]) == am) key = 2u * (uint32_t) ((lane & 31) * 8 + e) + (__float_as_uint(v[i][e]) >> 31);
            key = half_min_u32(key);
            const float mx = (key & 1u) ? -am : am;
            float q[8];
            float d = 0.0f;
            if (am != 0.0f) {
                const float iscale = -127.0f / mx;
#pragma unroll
                for (int e = 0; e < 8; e++) q[e] = fminf(rintf(iscale * v[i][e]), 127.0f);
                d = 1.0f / iscale;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) q[e] = 0.0f;
            }
            float bs = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) bs += q[e];
            bs += dpp_f32<DPP_XOR1>(bs);   // the other 8 values of the 16-group
            if (live) {
                uint32_t qb[2] = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; e++) qb[e >> 2] |= ((uint32_t) (int) q[e] & 0xffu) << (8 * (e & 3));
                *(uint2 *) ((int8_t *) out.q + row * D + 8 * o) = make_uint2(qb[0], qb[1]);   // int8 codes
                if ((o & 31) == 0) ((float *) out.d)[row * (D / 256) + o / 32] = d;
                if ((o & 1) == 0) ((_Float16 *) out.bsum)[row * (D / 16) + o / 2] = (_Float16) bs;
            }
        }
    }
}

}  // namespace rowln
