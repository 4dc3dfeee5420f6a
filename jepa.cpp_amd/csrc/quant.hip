// quant.hip - weight quantizers on gfx950: f32 rows -> ggml q8_0 / q4_0 / q4_K blocks and f16, bit
// for bit what ggml's reference quantizers write (quantize_row_q8_0_ref / q4_0_ref / q4_K_ref of the
// ggml the reference pins; the tool that calls them is tools/jepa-quantize.cpp:159-173).
//
// Every rounding is the C code's: the file is built with -ffp-contract=off and correctly rounded
// division and square root, sums run sequentially in element order, nearest_int is the 1.5 * 2^23
// magic-number round-half-to-even, float -> f16 is the hardware's round-to-nearest-even conversion.
//   q8_0: one thread per 32-value block.
//   q4_0: one thread per 32-value block.
//   q4_K: eight lanes per 256-value super-block, one per 32-value sub-block: each runs the weighted
//         make_qkx2_quants search on its sub-block in registers, the eight exchange their scale and
//         min by lane shuffles (maxima are order-free), quantize them to 6 bits, re-fit their values,
//         and the even lane of each pair writes the 32 nibble bytes the pair shares.
#include "common.h"
#include "kernels.h"

namespace {

__device__ __forceinline__ int nearest_int(float v) {
    const float val = v + 12582912.0f;
    return (__float_as_int(val) & 0x007fffff) - 0x00400000;
}

// f32 -> f16 bits of a value already rounded to f32 (the C code rounds the f32 expression, then
// converts). The empty asm keeps the compiler from folding the producing multiply into the
// conversion (v_fma_mix with a +0 addend turns -0 into +0, and fuses away the f32 rounding).
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16) f);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

__global__ void k_quant_q8_0(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nblk) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const float * xb = x + b * 32;
    float v[32], amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) { v[j] = xb[j]; amax = fmaxf(amax, fabsf(v[j])); }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t * o = (uint16_t *) (y + b * 34);   // 34-byte blocks: 2-byte aligned
    o[0] = f2h(d);
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        const int q0 = (int) roundf(v[j] * id), q1 = (int) roundf(v[j + 1] * id);
        o[1 + j / 2] = (uint16_t) ((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

__global__ void k_quant_q4_0(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nblk) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const float * xb = x + b * 32;
    float v[32], amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        v[j] = xb[j];
        if (amax < fabsf(v[j])) { amax = fabsf(v[j]); mx = v[j]; }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t * o = (uint16_t *) (y + b * 18);
    o[0] = f2h(d);
    uint8_t q[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int t0 = (int) (v[j] * id + 8.5f), t1 = (int) (v[16 + j] * id + 8.5f);
        q[j] = (uint8_t) (min(15, t0) | (min(15, t1) << 4));
    }
#pragma unroll
    for (int j = 0; j < 16; j += 2) o[1 + j / 2] = (uint16_t) (q[j] | (q[j + 1] << 8));
}

// ggml make_qkx2_quants(32, 15, x, w, L, &the_min, Laux, rmin -1, rdelta 0.1, nstep 20, use_mad false),
// levels packed four per u32 (L[i] in byte i % 4 of Lw[i / 4])
__device__ __forceinline__ float qkx2_32(const float * x, const float * w, uint32_t * Lw, float * the_min) {
    constexpr int n = 32, nmax = 15, nstep = 20;
    constexpr float rmin = -1.0f, rdelta = 0.1f;
    float mn = x[0], mx = x[0], sum_w = w[0], sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
#pragma unroll
        for (int i = 0; i < n / 4; i++) Lw[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_error = 0;
#pragma unroll
    for (int i = 0; i < n / 4; i++) Lw[i] = 0;
#pragma unroll
    for (int i = 0; i < n; ++i) {
        const int l = max(0, min(nmax, nearest_int(iscale * (x[i] - mn))));
        Lw[i / 4] |= (uint32_t) l << (8 * (i % 4));
        const float diff = scale * l + mn - x[i];
        best_error += w[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        uint32_t La[n / 4];
#pragma unroll
        for (int i = 0; i < n / 4; i++) La[i] = 0;
#pragma unroll
        for (int i = 0; i < n; ++i) {
            const int l = max(0, min(nmax, nearest_int(iscale * (x[i] - mn))));
            La[i / 4] |= (uint32_t) l << (8 * (i % 4));
            const float wl = w[i] * l;
            sum_l += wl;
            sum_l2 += wl * l;
            sum_xl += wl * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
#pragma unroll
            for (int i = 0; i < n; ++i) {
                const float diff = this_scale * (float) ((La[i / 4] >> (8 * (i % 4))) & 0xff) + this_min - x[i];
                cur_error += w[i] * (diff * diff);
            }
            if (cur_error < best_error) {
#pragma unroll
                for (int i = 0; i < n / 4; i++) Lw[i] = La[i];
                best_error = cur_error;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

// lane j (0..7) of an aligned group of 8 handles sub-block j of super-block (global lane) / 8
__global__ __launch_bounds__(256) void k_quant_q4_K(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nsb) {
    const int64_t g = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t sbk = g >> 3;
    const int j = (int) (g & 7);
    const bool live = sbk < nsb;     // whole groups of 8 share liveness (nsb * 8 lanes are live)
    float v[32], w[32];
    const float * xs = x + (live ? sbk : 0) * 256 + 32 * j;
#pragma unroll
    for (int l = 0; l < 32; l++) v[l] = live ? xs[l] : 0.0f;
    float sum_x2 = 0;
#pragma unroll
    for (int l = 0; l < 32; ++l) sum_x2 += v[l] * v[l];
    const float av_x = sqrtf(sum_x2 / 32);
#pragma unroll
    for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(v[l]);
    uint32_t L[8];
    float the_min;
    const float scale = qkx2_32(v, w, L, &the_min);
    // maxima over the 8 sub-blocks (lanes of one group are aligned to 8 within the wave)
    float max_scale = scale > 0 ? scale : 0.0f, max_min = the_min > 0 ? the_min : 0.0f;
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        max_scale = fmaxf(max_scale, __shfl_xor(max_scale, o, 64));
        max_min = fmaxf(max_min, __shfl_xor(max_min, o, 64));
    }
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    uint8_t ls = (uint8_t) nearest_int(inv_scale * scale), lm = (uint8_t) nearest_int(inv_min * the_min);
    ls = ls < 63 ? ls : 63;
    lm = lm < 63 ? lm : 63;
    const uint16_t dh = f2h(max_scale / 63.0f), dmh = f2h(max_min / 63.0f);
    // the 12 packed scale bytes: lane j < 4 owns bytes j and j + 4, lane j >= 4 owns byte j + 4
    const int ls_hi = __shfl_xor((int) ls, 4, 64), lm_hi = __shfl_xor((int) lm, 4, 64);   // lane j < 4: sub-block j + 4
    // re-fit against the quantized scale and min (a zero scale keeps the search's levels)
    const float d = h2f(dh) * ls;
    if (d != 0.0f) {
        const float dm = h2f(dmh) * lm;
#pragma unroll
        for (int i = 0; i < 8; i++) L[i] = 0;
#pragma unroll
        for (int ii = 0; ii < 32; ++ii) {
            const int l = max(0, min(15, nearest_int((v[ii] + dm) / d)));
            L[ii / 4] |= (uint32_t) l << (8 * (ii % 4));
        }
    }
    // the odd sub-block of each pair supplies the high nibbles
    uint32_t hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) hi[i] = (uint32_t) __shfl_xor((int) L[i], 1, 64);
    if (!live) return;
    uint8_t * blk = y + sbk * 144;
    if (j == 0) {
        uint16_t * h = (uint16_t *) blk;   // 144-byte blocks: 4-byte aligned
        h[0] = dh;
        h[1] = dmh;
    }
    if (j < 4) {
        blk[4 + j] = (uint8_t) (ls | ((ls_hi >> 4) << 6));
        blk[4 + j + 4] = (uint8_t) (lm | ((lm_hi >> 4) << 6));
    } else {
        blk[4 + j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
    }
    if ((j & 1) == 0) {
        uint32_t * q = (uint32_t *) (blk + 16 + 16 * j);   // chunk j / 2: 32 bytes at 16 + 32 * (j / 2)
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = L[i] | (hi[i] << 4);
    }
}

__global__ void k_to_f16(const float * __restrict__ x, uint16_t * __restrict__ y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = f2h(x[i]);
}

int nblocks(int64_t n, int t) { return (int) ((n + t - 1) / t); }

}  // namespace

bool launch_quantize_rows(int dst_type, const float * x, int64_t n, void * y, hipStream_t s) {
    switch (dst_type) {
        case T_Q8_0:
            if (n % 32) return false;
            if (n) k_quant_q8_0<<<nblocks(n / 32, 256), 256, 0, s>>>(x, (uint8_t *) y, n / 32);
            return true;
        case T_Q4_0:
            if (n % 32) return false;
            if (n) k_quant_q4_0<<<nblocks(n / 32, 256), 256, 0, s>>>(x, (uint8_t *) y, n / 32);
            return true;
        case T_Q4_K:
            if (n % 256) return false;
            if (n) k_quant_q4_K<<<nblocks(n / 256 * 8, 256), 256, 0, s>>>(x, (uint8_t *) y, n / 256);
            return true;
        case T_F16:
            if (n) k_to_f16<<<nblocks(n, 256), 256, 0, s>>>(x, (uint16_t *) y, n);
            return true;
        default:
            return false;
    }
}
