/*
 * oracle.c - CPU restatement of jepa.cpp's encoder path with ggml CPU semantics (test infrastructure).
 *
 * See oracle.h for the scope. Reference citations are into aselimc/jepa.cpp; the ggml behaviour
 * restated here is that of ggml @36da5713 (v0.22.0) on x86 as described in the reference's docs
 * (docs/ggml-notes.md, docs/parity.md) and in ggml's public block layouts (ggml-common.h).
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp). Floating-point
 * contraction is off so every rounding is the one written here; FMAs are explicit (fmaf).
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK8_0 32
#define QK4_0 32
#define QK_K 256

typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;                 /* 34 B */
typedef struct { uint16_t d; uint8_t qs[QK4_0 / 2]; } blk_q4_0;            /* 18 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; } blk_q4_K;  /* 144 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } blk_q8_K;         /* 292 B */

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 block");
_Static_assert(sizeof(blk_q4_0) == 18, "q4_0 block");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K block");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K block");

/* ------------------------------------------------------------------------------------------------
 * IEEE binary16 <-> binary32, round to nearest even (what F16C's vcvtps2ph with imm 0 does, which is
 * ggml's GGML_FP32_TO_FP16 on x86). Written from the IEEE-754 definition.
 * ---------------------------------------------------------------------------------------------- */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0));
    }
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);   /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal half (or zero) */
        if (ax < 0x33000000u) return (uint16_t) sign;            /* < 2^-25 rounds to 0 (ties to even 0) */
        const uint32_t e = ax >> 23;               /* biased exponent, 102..112 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;            /* value = m * 2^(e-150); half ulp unit 2^-24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t) (sign | q);
    }
    /* normal range */
    uint32_t h = ((ax >> 13) - (112u << 10));      /* rebias exponent 127 -> 15 */
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t) (sign | h);
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {                                     /* subnormal: normalise */
            int sh = 0; uint32_t mm = m;
            while (!(mm & 0x400u)) { mm <<= 1; sh++; }
            x = sign | ((uint32_t) (113 - sh) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f; memcpy(&f, &x, 4);
    return f;
}

void or_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = or_fp32_to_fp16(x[i]); }
void or_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = or_fp16_to_fp32(x[i]); }

size_t or_row_size(int type, int64_t n) {
    switch (type) {
        case OR_F32:  return (size_t) n * 4;
        case OR_F16:  return (size_t) n * 2;
        case OR_Q8_0: return n % QK8_0 ? 0 : (size_t) (n / QK8_0) * sizeof(blk_q8_0);
        case OR_Q4_0: return n % QK4_0 ? 0 : (size_t) (n / QK4_0) * sizeof(blk_q4_0);
        case OR_Q4_K: return n % QK_K ? 0 : (size_t) (n / QK_K) * sizeof(blk_q4_K);
        case OR_Q8_K: return n % QK_K ? 0 : (size_t) (n / QK_K) * sizeof(blk_q8_K);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------
 * quantizers
 * ---------------------------------------------------------------------------------------------- */
/* ggml quantize_row_q8_0_ref: d = amax/127, id = 1/d, q = roundf(x*id) (half away from zero).
 * This is what ggml_quantize_chunk -> quantize_q8_0 writes into a q8_0 GGUF (tools/jepa-quantize.cpp:171). */
void or_quantize_q8_0_ref(const float * x, void * vb, int64_t n) {
    blk_q8_0 * y = (blk_q8_0 *) vb;
    for (int64_t i = 0; i < n / QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < QK8_0; j++) y[i].qs[j] = (int8_t) roundf(x[i * QK8_0 + j] * id);
    }
}

/* ggml quantize_row_q4_0_ref: d = max/-8 (max = the signed value of largest magnitude),
 * q = min(15, (int8)(x/d + 8.5)); low nibbles hold elements 0..15, high nibbles 16..31. */
void or_quantize_q4_0_ref(const float * x, void * vb, int64_t n) {
    blk_q4_0 * y = (blk_q4_0 *) vb;
    for (int64_t i = 0; i < n / QK4_0; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK4_0; j++) {
            const float v = x[i * QK4_0 + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < QK4_0 / 2; j++) {
            const float x0 = x[i * QK4_0 + j] * id;
            const float x1 = x[i * QK4_0 + QK4_0 / 2 + j] * id;
            int8_t t0 = (int8_t) (x0 + 8.5f), t1 = (int8_t) (x1 + 8.5f);
            const uint8_t q0 = (uint8_t) (t0 < 15 ? t0 : 15), q1 = (uint8_t) (t1 < 15 ? t1 : 15);
            y[i].qs[j] = (uint8_t) (q0 | (q1 << 4));
        }
    }
}

/* ggml nearest_int: round half to even through the 1.5*2^23 magic (valid for |v| < 2^22). */
static inline int nearest_int(float v) {
    float val = v + 12582912.0f;
    int32_t i; memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* 6-bit scale and min of sub-block j from the 12 packed q4_K scale bytes */
static inline void q4k_scale_min(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *d = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* ggml's make_qkx2_quants (ggml-quants.c of the ggml the reference pins, 36da5713 / v0.22.0; the
 * submodule is absent from the reference tree): an asymmetric 4-bit fit of n values with weights w.
 * Start from the min/max grid, then try nstep + 1 scales iscale = (rmin + rdelta*is + nmax)/(max-min):
 * for each, the weighted least-squares scale and min of the resulting levels (min clamped <= 0), kept
 * when its weighted squared error beats the best so far. Returns the scale, *the_min = -min. Every sum
 * runs sequentially in element order, in float32, as in ggml's scalar code. */
static float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                              uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t) (l < 0 ? 0 : l > nmax ? nmax : l);
        const float diff = scale * L[i] + min - x[i];
        best_error += weights[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : l > nmax ? nmax : l;
            Laux[i] = (uint8_t) l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
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
            for (int i = 0; i < n; ++i) {
                const float diff = this_scale * Laux[i] + this_min - x[i];
                cur_error += weights[i] * (diff * diff);
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* One make_qkx2_quants fit of n <= 256 values, exported so the tests can check the fit itself (the
 * q4_K block only keeps its 6-bit requantization). Returns -1 for n out of range. */
float or_make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                          float rmin, float rdelta, int nstep) {
    uint8_t Laux[256];
    if (n <= 0 || n > 256) return -1.0f;
    return make_qkx2_quants(n, nmax, x, weights, L, the_min, Laux, rmin, rdelta, nstep);
}

/* ggml quantize_row_q4_K_ref (same source as above): per 32-value sub-block, weights
 * av_x + |x| with av_x = sqrt(mean x^2), make_qkx2_quants(32, 15, rmin -1, rdelta 0.1, 20 steps);
 * the 8 scales and mins quantized to 6 bits against their maxima (d = max_scale/63, dmin =
 * max_min/63, f16), packed into the 12 scale bytes; then every value re-fitted against its quantized
 * scale and min (a sub-block whose quantized scale is 0 keeps the levels of the fit); nibbles hold
 * values j..j+31 (low) and j+32..j+63 (high) of each 64. This is what ggml_quantize_chunk writes for a
 * q4_K tensor without an importance matrix (tools/jepa-quantize.cpp:159-173). */
void or_quantize_q4_K(const float * x, void * vb, int64_t n) {
    blk_q4_K * y = (blk_q4_K *) vb;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const float * xb = x + i * QK_K;
        uint8_t L[QK_K], Laux[32];
        float weights[32], mins[QK_K / 32], scales[QK_K / 32];
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xb[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.0f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t) nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t) ((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t) ((lm >> 4) << 6);
            }
        }
        y[i].d = or_fp32_to_fp16(max_scale / 63.0f);
        y[i].dmin = or_fp32_to_fp16(max_min / 63.0f);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t sc, m;
            q4k_scale_min(j, y[i].scales, &sc, &m);
            const float d = or_fp16_to_fp32(y[i].d) * sc;
            if (!d) continue;
            const float dm = or_fp16_to_fp32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((xb[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : l > 15 ? 15 : l;
                L[32 * j + ii] = (uint8_t) l;
            }
        }
        for (int j = 0; j < QK_K; j += 64)
            for (int l = 0; l < 32; l++) y[i].qs[j / 2 + l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 4));
    }
}

/* Activation q8_0 as the x86 CPU backend computes it inside mul_mat (quantize_row_q8_0, AVX2 path):
 *   amax = max|x|, d = amax / 127 (stored f16), id = amax != 0 ? 127 / amax : 0,
 *   q = round-to-nearest-even(x * id)   (_mm256_round_ps(_MM_ROUND_NEAREST), then packs)        */
void or_quantize_q8_0_act(const float * x, void * vb, int64_t n) {
    blk_q8_0 * y = (blk_q8_0 *) vb;
    for (int64_t i = 0; i < n / QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / 127.0f;
        y[i].d = or_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < QK8_0; j++) {
            float v = rintf(x[i * QK8_0 + j] * id);           /* default rounding mode: half even */
            if (v > 127.0f) v = 127.0f;
            if (v < -128.0f) v = -128.0f;
            y[i].qs[j] = (int8_t) v;
        }
    }
}

/* Activation q8_K (quantize_row_q8_K_ref, which is what the x86 build uses):
 *   max = signed value of largest |x|, iscale = -127/max, q = min(127, nearest_int(iscale*x)),
 *   bsums = sums of 16 consecutive q, d = 1/iscale (f32). An all-zero block gives d = 0, q = 0. */
void or_quantize_q8_K_act(const float * x, void * vb, int64_t n) {
    blk_q8_K * y = (blk_q8_K *) vb;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const float * xb = x + i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) { memset(&y[i], 0, sizeof(blk_q8_K)); continue; }
        const float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t) s;
        }
        y[i].d = 1.0f / iscale;
    }
}


void or_dequantize(int type, const void * vb, float * y, int64_t n) {
    switch (type) {
        case OR_F32: memcpy(y, vb, (size_t) n * 4); return;
        case OR_F16: or_fp16_to_fp32_row((const uint16_t *) vb, y, n); return;
        case OR_Q8_0: {
            const blk_q8_0 * b = (const blk_q8_0 *) vb;
            for (int64_t i = 0; i < n / QK8_0; i++) {
                const float d = or_fp16_to_fp32(b[i].d);
                for (int j = 0; j < QK8_0; j++) y[i * QK8_0 + j] = b[i].qs[j] * d;
            }
            return;
        }
        case OR_Q4_0: {
            const blk_q4_0 * b = (const blk_q4_0 *) vb;
            for (int64_t i = 0; i < n / QK4_0; i++) {
                const float d = or_fp16_to_fp32(b[i].d);
                for (int j = 0; j < QK4_0 / 2; j++) {
                    y[i * QK4_0 + j]             = ((b[i].qs[j] & 0xF) - 8) * d;
                    y[i * QK4_0 + j + QK4_0 / 2] = ((b[i].qs[j] >> 4) - 8) * d;
                }
            }
            return;
        }
        case OR_Q4_K: {
            const blk_q4_K * b = (const blk_q4_K *) vb;
            for (int64_t i = 0; i < n / QK_K; i++) {
                const float d = or_fp16_to_fp32(b[i].d), dmin = or_fp16_to_fp32(b[i].dmin);
                const uint8_t * q = b[i].qs;
                float * yy = y + i * QK_K;
                for (int j = 0, is = 0; j < QK_K; j += 64, is += 2, q += 32) {
                    uint8_t sc, m;
                    q4k_scale_min(is, b[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = dmin * m;
                    q4k_scale_min(is + 1, b[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = dmin * m;
                    for (int l = 0; l < 32; l++) *yy++ = d1 * (q[l] & 0xF) - m1;
                    for (int l = 0; l < 32; l++) *yy++ = d2 * (q[l] >> 4) - m2;
                }
            }
            return;
        }
        case OR_Q8_K: {
            const blk_q8_K * b = (const blk_q8_K *) vb;
            for (int64_t i = 0; i < n / QK_K; i++)
                for (int j = 0; j < QK_K; j++) y[i * QK_K + j] = b[i].d * b[i].qs[j];
            return;
        }
    }
}

/* ------------------------------------------------------------------------------------------------
 * dots: exact integer sums per block, float epilogue per block (vec_dot_q8_0_q8_0 etc.)
 * ---------------------------------------------------------------------------------------------- */
static float dot_f32_8acc(const float * a, const float * b, int64_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

/* ggml's x86 summation order (g_ggml_lanes = 1), ggml 36da5713, the submodule the reference pins
 * (docs/benchmarks.md:36) and builds with GGML_LLAMAFILE=ON (:37):
 *  - q8_0 and q4_0 weights x q8_0 activations run through llamafile's tinyBLAS_Q0_AVX tiles
 *    (ggml-cpu/llamafile/sgemm.cpp) or, for shapes it declines, ggml_vec_dot_q8_0_q8_0 /
 *    ggml_vec_dot_q4_0_q8_0 (ggml-cpu/arch/x86/quants.c, AVX2 path). Both keep one __m256 of eight
 *    float lanes per output: the byte products of a 32-block are summed four consecutive bytes per
 *    int32 lane (_mm256_dpbusd_epi32, or maddubs + madd), converted to float, and each lane takes
 *    fma(dw * da, lane, acc) block by block; the eight lanes are then added by hsum_float_8. The
 *    reference measured the two paths bit-identical (docs/ggml-notes.md:246-251).
 *  - q4_K weights x q8_K activations run ggml_vec_dot_q4_K_q8_K (AVX2 path; llamafile has no
 *    k-quant tiles): per super-block, eight int32 lanes sum sc_j * (four consecutive products) over
 *    the eight sub-blocks (maddubs, then madd with the broadcast scale), and acc += (y.d * x.d) * lane
 *    per lane; the mins go to four float lanes, lane k = m_2k bsum_2k + m_2k+1 bsum_2k+1 (madd of the
 *    mins with the pairwise-added bsums), acc_m += (-y.d * x.dmin) * lane. The result is
 *    hsum_float_8(acc) plus the two-step horizontal sum of acc_m.
 * hsum_float_8(v) = ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)): the high 128 bits added to
 * the low, then movehl, then movehdup. */
static int g_ggml_lanes = 0;
void or_set_ggml_lanes(int on) { g_ggml_lanes = on; }
int or_get_ggml_lanes(void) { return g_ggml_lanes; }

static float hsum_lanes8(const float v[8]) { return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7])); }
static float hsum_lanes4(const float v[4]) { return (v[0] + v[2]) + (v[1] + v[3]); }

/* one output in ggml's x86 lane order: q = weight codes (int8, q4 values unsigned for q4_K), a =
 * activation codes, nb blocks (32) or super-blocks (256) */
static float dot_ggml_lanes(int wtype, const int8_t * q, const int8_t * a, int64_t nb, const float * dwr, const float * dmr,
                            const float * dar, const int32_t * scr, const int32_t * mr, const int32_t * bsr) {
    if (wtype == OR_Q4_K) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, accm[4] = {0, 0, 0, 0};
        for (int64_t b = 0; b < nb; b++) {
            int32_t sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < 8; j++) {
                const int8_t * qj = q + b * QK_K + 32 * j;
                const int8_t * aj = a + b * QK_K + 32 * j;
                for (int l = 0; l < 8; l++) {
                    int32_t p = 0;
                    for (int e = 4 * l; e < 4 * l + 4; e++) p += (int32_t) (uint8_t) qj[e] * (int32_t) aj[e];
                    sumi[l] += scr[b * 8 + j] * p;
                }
            }
            const float d = dar[b] * dwr[b];
            const float dmin = -dar[b] * dmr[b];
            for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float) sumi[l], acc[l]);
            for (int k = 0; k < 4; k++) {
                const int32_t prod = mr[b * 8 + 2 * k] * bsr[b * 8 + 2 * k] + mr[b * 8 + 2 * k + 1] * bsr[b * 8 + 2 * k + 1];
                accm[k] = fmaf(dmin, (float) prod, accm[k]);
            }
        }
        return hsum_lanes8(acc) + hsum_lanes4(accm);
    }
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = dwr[b] * dar[b];
        for (int l = 0; l < 8; l++) {
            int32_t si = 0;
            for (int e = 4 * l; e < 4 * l + 4; e++) si += (int32_t) q[b * 32 + e] * (int32_t) a[b * 32 + e];
            acc[l] = fmaf(d, (float) si, acc[l]);
        }
    }
    return hsum_lanes8(acc);
}

/* or_vec_dot in the lane order: the row's codes and scales expanded, then dot_ggml_lanes */
static float vec_dot_lanes(int wtype, int64_t n, const void * wrow, const void * arow) {
    const int kq = wtype == OR_Q4_K ? QK_K : 32;
    const int64_t nb = n / kq;
    int8_t * q = (int8_t *) malloc((size_t) n), * a = (int8_t *) malloc((size_t) n);
    float * dw = (float *) malloc(sizeof(float) * nb * 3);
    int32_t * ib = (int32_t *) malloc(sizeof(int32_t) * nb * 24);
    if (!q || !a || !dw || !ib) { free(q); free(a); free(dw); free(ib); return NAN; }
    float * dm = dw + nb, * da = dw + 2 * nb;
    int32_t * sc = ib, * mn = ib + nb * 8, * bs = ib + nb * 16;
    for (int64_t b = 0; b < nb; b++) {
        if (wtype == OR_Q4_K) {
            const blk_q4_K * X = (const blk_q4_K *) wrow + b; const blk_q8_K * Y = (const blk_q8_K *) arow + b;
            dw[b] = or_fp16_to_fp32(X->d); dm[b] = or_fp16_to_fp32(X->dmin); da[b] = Y->d;
            for (int j = 0; j < 8; j++) {
                uint8_t s6, m6;
                q4k_scale_min(j, X->scales, &s6, &m6);
                sc[b * 8 + j] = s6; mn[b * 8 + j] = m6;
                bs[b * 8 + j] = (int32_t) Y->bsums[2 * j] + (int32_t) Y->bsums[2 * j + 1];
                for (int l = 0; l < 32; l++) q[b * QK_K + 32 * j + l] = (int8_t) ((j & 1) ? (X->qs[32 * (j / 2) + l] >> 4) : (X->qs[32 * (j / 2) + l] & 0xF));
            }
            memcpy(a + b * QK_K, Y->qs, QK_K);
        } else {
            const blk_q8_0 * Y = (const blk_q8_0 *) arow + b;
            da[b] = or_fp16_to_fp32(Y->d);
            memcpy(a + b * 32, Y->qs, 32);
            if (wtype == OR_Q8_0) {
                const blk_q8_0 * X = (const blk_q8_0 *) wrow + b;
                dw[b] = or_fp16_to_fp32(X->d);
                memcpy(q + b * 32, X->qs, 32);
            } else {
                const blk_q4_0 * X = (const blk_q4_0 *) wrow + b;
                dw[b] = or_fp16_to_fp32(X->d);
                for (int j = 0; j < 16; j++) { q[b * 32 + j] = (int8_t) ((X->qs[j] & 0xF) - 8); q[b * 32 + j + 16] = (int8_t) ((X->qs[j] >> 4) - 8); }
            }
        }
    }
    const float r = dot_ggml_lanes(wtype, q, a, nb, dw, dm, da, sc, mn, bs);
    free(q); free(a); free(dw); free(ib);
    return r;
}

float or_vec_dot(int wtype, int64_t n, const void * wrow, const void * arow) {
    if (g_ggml_lanes && (wtype == OR_Q8_0 || wtype == OR_Q4_0 || wtype == OR_Q4_K)) return vec_dot_lanes(wtype, n, wrow, arow);
    switch (wtype) {
        case OR_F32: return dot_f32_8acc((const float *) wrow, (const float *) arow, n);
        case OR_F16: {
            /* both rows f16: widen and accumulate in f32 (ggml_vec_dot_f16) */
            const uint16_t * w = (const uint16_t *) wrow; const uint16_t * a = (const uint16_t *) arow;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int64_t i = 0;
            for (; i + 8 <= n; i += 8)
                for (int l = 0; l < 8; l++) acc[l] = fmaf(or_fp16_to_fp32(w[i + l]), or_fp16_to_fp32(a[i + l]), acc[l]);
            float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
            for (; i < n; i++) s = fmaf(or_fp16_to_fp32(w[i]), or_fp16_to_fp32(a[i]), s);
            return s;
        }
        case OR_Q8_0: {
            const blk_q8_0 * x = (const blk_q8_0 *) wrow; const blk_q8_0 * y = (const blk_q8_0 *) arow;
            float s = 0.0f;
            for (int64_t b = 0; b < n / QK8_0; b++) {
                int32_t si = 0;
                for (int j = 0; j < QK8_0; j++) si += (int32_t) x[b].qs[j] * (int32_t) y[b].qs[j];
                const float d = or_fp16_to_fp32(x[b].d) * or_fp16_to_fp32(y[b].d);
                s = fmaf((float) si, d, s);
            }
            return s;
        }
        case OR_Q4_0: {
            const blk_q4_0 * x = (const blk_q4_0 *) wrow; const blk_q8_0 * y = (const blk_q8_0 *) arow;
            float s = 0.0f;
            for (int64_t b = 0; b < n / QK4_0; b++) {
                int32_t si = 0;
                for (int j = 0; j < QK4_0 / 2; j++) {
                    si += ((x[b].qs[j] & 0xF) - 8) * (int32_t) y[b].qs[j];
                    si += ((x[b].qs[j] >> 4) - 8) * (int32_t) y[b].qs[j + QK4_0 / 2];
                }
                const float d = or_fp16_to_fp32(x[b].d) * or_fp16_to_fp32(y[b].d);
                s = fmaf((float) si, d, s);
            }
            return s;
        }
        case OR_Q4_K: {
            const blk_q4_K * x = (const blk_q4_K *) wrow; const blk_q8_K * y = (const blk_q8_K *) arow;
            float s = 0.0f, sm = 0.0f;
            for (int64_t b = 0; b < n / QK_K; b++) {
                int32_t isum = 0, msum = 0;
                const uint8_t * q4 = x[b].qs; const int8_t * q8 = y[b].qs;
                for (int j = 0; j < 8; j++) {
                    uint8_t sc, m;
                    q4k_scale_min(j, x[b].scales, &sc, &m);
                    const uint8_t * qq = q4 + 32 * (j / 2);
                    int32_t si = 0;
                    for (int l = 0; l < 32; l++) {
                        const int v = (j & 1) ? (qq[l] >> 4) : (qq[l] & 0xF);
                        si += v * (int32_t) q8[32 * j + l];
                    }
                    isum += (int32_t) sc * si;
                    msum += (int32_t) m * ((int32_t) y[b].bsums[2 * j] + (int32_t) y[b].bsums[2 * j + 1]);
                }
                s  = fmaf(or_fp16_to_fp32(x[b].d) * y[b].d, (float) isum, s);
                sm = fmaf(or_fp16_to_fp32(x[b].dmin) * y[b].d, (float) msum, sm);
            }
            return s - sm;
        }
    }
    return 0.0f;
}

/* ggml_compute_forward_mul_mat: src1 rows converted to the weight's vec_dot_type once, then one
 * vec_dot per output element; ggml_add of the bias afterwards (src/jepa.cpp:365-375).
 * The codes and scales of both operands are expanded once per row (int8 codes, f32 scales); the
 * arithmetic per output is exactly or_vec_dot's: exact int32 block sums, d = dw*da (an exact f32
 * product of two f16 values), acc = fmaf(sum, d, acc) block by block in K order. */
/* Summation order of the per-block float epilogue over K: 0 = block 0 first (ggml's generic C order),
 * 1 = last block first. Both are valid restatements of ggml's vec_dot (its SIMD builds differ in this
 * order); tests run both to measure how far two correct implementations drift apart through a deep
 * quantized encoder. */
static int g_reverse_blocks = 0;
void or_set_reverse_block_order(int on) { g_reverse_blocks = on; }
/* The blocks (q8_0 / q4_0) or super-blocks (q4_K) in k_split equal consecutive ranges, each summed in
 * its own chain from 0 (q4_K: main and mins chains, then their difference), the range results added
 * in order (a GEMM that gives each K range to its own worker). 1: one chain. */
static int g_k_split = 1;
void or_set_k_split(int s) { g_k_split = s < 1 ? 1 : s; }

int or_mul_mat(int wtype, const void * w, int64_t n_out, int64_t n_in,
               const float * x, int64_t n_rows, const float * bias, float * y, int n_threads) {
    const size_t wrow = or_row_size(wtype, n_in);
    if (wrow == 0 || (wtype != OR_F32 && wtype != OR_F16 && wtype != OR_Q8_0 && wtype != OR_Q4_0 && wtype != OR_Q4_K)) {
        fprintf(stderr, "oracle: mul_mat of type %d over rows of %lld not supported\n", wtype, (long long) n_in);
        return -1;
    }
    const uint8_t * W = (const uint8_t *) w;
    if (wtype == OR_F32 || wtype == OR_F16) {
        /* f16 weights: activations rounded to f16 (ggml's vec_dot_type for F16 is F16) */
        float * wf = (float *) malloc(sizeof(float) * n_out * n_in);
        float * xf = (float *) malloc(sizeof(float) * n_rows * n_in);
        if (!wf || !xf) { free(wf); free(xf); return -1; }
        for (int64_t o = 0; o < n_out; o++) or_dequantize(wtype, W + (size_t) o * wrow, wf + o * n_in, n_in);
        for (int64_t i = 0; i < n_rows * n_in; i++)
            xf[i] = wtype == OR_F16 ? or_fp16_to_fp32(or_fp32_to_fp16(x[i])) : x[i];
#pragma omp parallel for num_threads(n_threads) schedule(static) collapse(2)
        for (int64_t m = 0; m < n_rows; m++)
            for (int64_t o = 0; o < n_out; o++) {
                float v = dot_f32_8acc(wf + o * n_in, xf + m * n_in, n_in);
                if (bias) v = v + bias[o];
                y[m * n_out + o] = v;
            }
        free(wf); free(xf);
        return 0;
    }
    const int kq = wtype == OR_Q4_K ? QK_K : 32;
    const int64_t nb = n_in / kq;
    int8_t * qw = (int8_t *) malloc((size_t) n_out * n_in);
    int8_t * qa = (int8_t *) malloc((size_t) n_rows * n_in);
    float * dw = (float *) malloc(sizeof(float) * n_out * nb);
    float * dmw = (float *) malloc(sizeof(float) * n_out * nb);
    float * da = (float *) malloc(sizeof(float) * n_rows * nb);
    int32_t * scw = (int32_t *) malloc(sizeof(int32_t) * n_out * nb * 8);
    int32_t * mw = (int32_t *) malloc(sizeof(int32_t) * n_out * nb * 8);
    int32_t * bsa = (int32_t *) malloc(sizeof(int32_t) * n_rows * nb * 8);
    if (!qw || !qa || !dw || !dmw || !da || !scw || !mw || !bsa) {
        free(qw); free(qa); free(dw); free(dmw); free(da); free(scw); free(mw); free(bsa);
        return -1;
    }
    /* weights */
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t o = 0; o < n_out; o++) {
        const uint8_t * row = W + (size_t) o * wrow;
        for (int64_t b = 0; b < nb; b++) {
            int8_t * q = qw + o * n_in + b * kq;
            if (wtype == OR_Q8_0) {
                const blk_q8_0 * B = (const blk_q8_0 *) row + b;
                dw[o * nb + b] = or_fp16_to_fp32(B->d);
                for (int j = 0; j < 32; j++) q[j] = B->qs[j];
            } else if (wtype == OR_Q4_0) {
                const blk_q4_0 * B = (const blk_q4_0 *) row + b;
                dw[o * nb + b] = or_fp16_to_fp32(B->d);
                for (int j = 0; j < 16; j++) { q[j] = (int8_t) ((B->qs[j] & 0xF) - 8); q[j + 16] = (int8_t) ((B->qs[j] >> 4) - 8); }
            } else {
                const blk_q4_K * B = (const blk_q4_K *) row + b;
                dw[o * nb + b] = or_fp16_to_fp32(B->d);
                dmw[o * nb + b] = or_fp16_to_fp32(B->dmin);
                for (int j = 0; j < 8; j++) {
                    uint8_t sc, m;
                    q4k_scale_min(j, B->scales, &sc, &m);
                    scw[(o * nb + b) * 8 + j] = sc;
                    mw[(o * nb + b) * 8 + j] = m;
                    const uint8_t * qq = B->qs + 32 * (j / 2);
                    for (int l = 0; l < 32; l++) q[32 * j + l] = (int8_t) ((j & 1) ? (qq[l] >> 4) : (qq[l] & 0xF));
                }
            }
        }
    }
    /* activations: quantized per row exactly as ggml's from_float does */
#pragma omp parallel num_threads(n_threads)
    {
        blk_q8_K * tmp = (blk_q8_K *) malloc(sizeof(blk_q8_K) * (size_t) (n_in / QK_K + 1));
        blk_q8_0 * tmp0 = (blk_q8_0 *) malloc(sizeof(blk_q8_0) * (size_t) (n_in / 32 + 1));
#pragma omp for schedule(static)
        for (int64_t m = 0; m < n_rows; m++) {
            if (wtype == OR_Q4_K) {
                or_quantize_q8_K_act(x + m * n_in, tmp, n_in);
                for (int64_t b = 0; b < nb; b++) {
                    da[m * nb + b] = tmp[b].d;
                    memcpy(qa + m * n_in + b * QK_K, tmp[b].qs, QK_K);
                    for (int j = 0; j < 8; j++) bsa[(m * nb + b) * 8 + j] = (int32_t) tmp[b].bsums[2 * j] + (int32_t) tmp[b].bsums[2 * j + 1];
                }
            } else {
                or_quantize_q8_0_act(x + m * n_in, tmp0, n_in);
                for (int64_t b = 0; b < nb; b++) {
                    da[m * nb + b] = or_fp16_to_fp32(tmp0[b].d);
                    memcpy(qa + m * n_in + b * 32, tmp0[b].qs, 32);
                }
            }
        }
        free(tmp); free(tmp0);
    }
#pragma omp parallel for num_threads(n_threads) schedule(static) collapse(2)
    for (int64_t m = 0; m < n_rows; m++) {
        for (int64_t o = 0; o < n_out; o++) {
            const int8_t * a = qa + m * n_in;
            const int8_t * q = qw + o * n_in;
            float s = 0.0f, sm = 0.0f;
            if (g_ggml_lanes) {
                s = dot_ggml_lanes(wtype, q, a, nb, dw + o * nb, dmw + o * nb, da + m * nb, scw + o * nb * 8, mw + o * nb * 8,
                                   bsa + m * nb * 8);
            } else if (wtype == OR_Q4_K && g_k_split > 1 && nb % g_k_split == 0) {
                /* each K range gives its own main and mins chains and their difference; the range
                   results are added in order */
                const int64_t per = nb / g_k_split;
                for (int p = 0; p < g_k_split; p++) {
                    float sp = 0.0f, smp = 0.0f;
                    for (int64_t b = p * per; b < (p + 1) * per; b++) {
                        int32_t isum = 0, msum = 0;
                        for (int j = 0; j < 8; j++) {
                            int32_t si = 0;
                            for (int l = 0; l < 32; l++) si += (int32_t) q[b * QK_K + 32 * j + l] * (int32_t) a[b * QK_K + 32 * j + l];
                            isum += scw[(o * nb + b) * 8 + j] * si;
                            msum += mw[(o * nb + b) * 8 + j] * bsa[(m * nb + b) * 8 + j];
                        }
                        sp  = fmaf(dw[o * nb + b] * da[m * nb + b], (float) isum, sp);
                        smp = fmaf(dmw[o * nb + b] * da[m * nb + b], (float) msum, smp);
                    }
                    s = p == 0 ? sp - smp : s + (sp - smp);
                }
            } else if (wtype == OR_Q4_K) {
                for (int64_t bb = 0; bb < nb; bb++) {
                    const int64_t b = g_reverse_blocks ? nb - 1 - bb : bb;
                    int32_t isum = 0, msum = 0;
                    for (int j = 0; j < 8; j++) {
                        int32_t si = 0;
                        for (int l = 0; l < 32; l++) si += (int32_t) q[b * QK_K + 32 * j + l] * (int32_t) a[b * QK_K + 32 * j + l];
                        isum += scw[(o * nb + b) * 8 + j] * si;
                        msum += mw[(o * nb + b) * 8 + j] * bsa[(m * nb + b) * 8 + j];
                    }
                    s  = fmaf(dw[o * nb + b] * da[m * nb + b], (float) isum, s);
                    sm = fmaf(dmw[o * nb + b] * da[m * nb + b], (float) msum, sm);
                }
                s = s - sm;
            } else if (g_k_split > 1 && nb % g_k_split == 0) {
                const int64_t per = nb / g_k_split;
                for (int p = 0; p < g_k_split; p++) {
                    float sp = 0.0f;
                    for (int64_t b = p * per; b < (p + 1) * per; b++) {
                        int32_t si = 0;
                        for (int l = 0; l < 32; l++) si += (int32_t) q[b * 32 + l] * (int32_t) a[b * 32 + l];
                        sp = fmaf((float) si, dw[o * nb + b] * da[m * nb + b], sp);
                    }
                    s = p == 0 ? sp : s + sp;
                }
            } else {
                for (int64_t bb = 0; bb < nb; bb++) {
                    const int64_t b = g_reverse_blocks ? nb - 1 - bb : bb;
                    int32_t si = 0;
                    for (int l = 0; l < 32; l++) si += (int32_t) q[b * 32 + l] * (int32_t) a[b * 32 + l];
                    s = fmaf((float) si, dw[o * nb + b] * da[m * nb + b], s);
                }
            }
            if (bias) s = s + bias[o];
            y[m * n_out + o] = s;
        }
    }
    free(qw); free(qa); free(dw); free(dmw); free(da); free(scw); free(mw); free(bsa);
    return 0;
}

/* ggml_norm (two-pass: mean in double, centred variance in double, y = (x-mean) * 1/sqrt(var+eps))
 * then ggml_mul(w) and ggml_add(b) as separate roundings (src/jepa.cpp:356-361). */
void or_layer_norm(const float * x, int64_t n_rows, int64_t d, const float * w, const float * b, float eps, float * y) {
    for (int64_t r = 0; r < n_rows; r++) {
        const float * xr = x + r * d;
        float * yr = y + r * d;
        double sum = 0.0;
        for (int64_t i = 0; i < d; i++) sum += (double) xr[i];
        const float mean = (float) sum / (float) d;
        double sum2 = 0.0;
        for (int64_t i = 0; i < d; i++) { const float v = xr[i] - mean; yr[i] = v; sum2 += (double) (v * v); }
        const float variance = (float) (sum2 / (double) d);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < d; i++) {
            float v = yr[i] * scale;
            if (w) v = v * w[i];
            if (b) v = v + b[i];
            yr[i] = v;
        }
    }
}

static int g_round;   /* rounding switches, see or_set_rounding below */

/* the GPU epilogue's GELU (OR_ROUND_GELU): x Phi(x) with the normal tail h(t) = Phi(-t), t = |x|, as
 * 2^Q(min(t, 5.5)), Q of degree 8 in Horner fmas, Phi = 1 - h for x >= 0 and h below, with the same
 * coefficients and float operations (exp2f in place of the hardware exp2) */
static float gpu_gelu(float x) {
    const float t = fminf(fabsf(x), 5.5f);
    float q = -2.248140163e-06f;
    q = fmaf(q, t, 3.268636283e-05f);
    q = fmaf(q, t, -1.560558158e-04f);
    q = fmaf(q, t, -2.054840443e-04f);
    q = fmaf(q, t, 7.147170603e-03f);
    q = fmaf(q, t, -5.254988000e-02f);
    q = fmaf(q, t, -4.591920078e-01f);
    q = fmaf(q, t, -1.151106834e+00f);
    q = fmaf(q, t, -1.0f);
    const float h = exp2f(q);
    return x * (x >= 0.0f ? 1.0f - h : h);
}

/* ggml_vec_gelu_erf_f32 (docs/ggml-notes.md:291-292): 0.5*x*(1+erf(x/sqrt(2))) with libm erff */
float or_gelu_erf(float x) {
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    if (g_round & 8) return gpu_gelu(x);
    return 0.5f * x * (1.0f + erff(x * SQRT_2_INV));
}

/* the same over n values (the MLP activation, src/jepa.cpp:377-385) */
void or_gelu_erf_n(const float * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_gelu_erf(x[i]);
}

/* ------------------------------------------------------------------------------------------------
 * 3-D RoPE (src/rope3d.cpp:9-164, math spec src/rope3d.h:1-62)
 * ---------------------------------------------------------------------------------------------- */
static void rope_position(const or_rope_params * p, int64_t i, float * t, float * h, float * w) {
    const int64_t per_frame = (int64_t) p->grid_h * p->grid_w;
    *t = (float) (i / per_frame);
    *h = (float) ((i % per_frame) / p->grid_w);
    *w = (float) (i % p->grid_w);
    if (p->interpolate) {   /* rope3d.cpp:20-27: left-to-right float32, t never rescaled */
        if (p->grid_h > 1) *h = (*h * (float) (p->train_grid_h - 1)) / (float) (p->grid_h - 1);
        if (p->grid_w > 1) *w = (*w * (float) (p->train_grid_w - 1)) / (float) (p->grid_w - 1);
    }
}

void or_rope_tables(const or_rope_params * p, const int32_t * ids, int64_t n_rows, float * c, float * s, int signed_sin) {
    const int D = p->head_dim;
    const int d = 2 * ((D / 3) / 2);           /* rope3d.cpp:9 */
    const int half = d / 2;
    for (int64_t i = 0; i < n_rows * D; i++) { c[i] = 1.0f; s[i] = 0.0f; }
    if (d == 0) return;
    float omega[512];
    for (int k = 0; k < half; k++) omega[k] = 1.0f / powf(p->theta, (float) k / (float) half);   /* rope3d.cpp:45-53 */
    for (int64_t r = 0; r < n_rows; r++) {
        const int64_t id = ids ? ids[r] : r;
        const int64_t per_frame = (int64_t) p->grid_h * p->grid_w;
        const int64_t ti = id / per_frame, hi = (id % per_frame) / p->grid_w, wi = id % p->grid_w;
        float pos[3], tt, hh, ww;
        rope_position(p, ti * per_frame, &tt, &hh, &ww); pos[0] = tt;
        rope_position(p, hi * p->grid_w, &tt, &hh, &ww); pos[1] = hh;
        rope_position(p, wi, &tt, &hh, &ww); pos[2] = ww;
        for (int a = 0; a < 3; a++) {
            for (int j = 0; j < d; j++) {
                const int k = p->variant == 0 ? (j % half) : (j / 2);   /* tiled vs interleaved, rope3d.cpp:33-41 */
                const float ang = pos[a] * omega[k];
                c[r * D + a * d + j] = cosf(ang);
                s[r * D + a * d + j] = sinf(ang);
            }
        }
        if (signed_sin) for (int j = 0; j < D; j += 2) s[r * D + j] = -s[r * D + j];   /* rope3d.cpp:106-108 */
    }
}

/* out = x*C + swap(x)*S' with swap(x)[j] = x[j^1] (rope3d.cpp:136-164): two products then one add */
void or_rope_apply(float * x, int64_t n_tok, int n_head, int hd, const float * ct, const float * st) {
    float tmp[1024];
    for (int64_t t = 0; t < n_tok; t++) {
        for (int h = 0; h < n_head; h++) {
            float * v = x + (t * n_head + h) * hd;
            for (int j = 0; j < hd; j++) tmp[j] = v[j];
            for (int j = 0; j < hd; j++) {
                const float a = tmp[j] * ct[t * hd + j];
                const float b = tmp[j ^ 1] * st[t * hd + j];
                v[j] = a + b;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------
 * attention: ggml_flash_attn_ext on the CPU tiled path: Q f32, K/V f16 tiles widened to f32,
 * scores/softmax/accumulator f32 (docs/ggml-notes.md:48-58). Softmax written two-pass here.
 * ---------------------------------------------------------------------------------------------- */
void or_block_causal_mask(int gt, int gh, int gw, int n_prefix, float * out) {
    const int64_t tpf = (int64_t) gh * gw, np = n_prefix, N = np + (int64_t) gt * tpf;
    for (int64_t i = 0; i < N; i++)
        for (int64_t j = 0; j < N; j++) {
            int open;
            if (i < np) open = 1;                                   /* prefix rows read the whole clip */
            else open = j >= np && (j - np) / tpf <= (i - np) / tpf; /* own slot or earlier, no prefix */
            out[i * N + j] = open ? 0.0f : -INFINITY;
        }
}

/* Rounding switches: the oracle follows the reference's CPU arithmetic (tiled flash-attention path:
 * q, scores, softmax and accumulator in f32, K/V rounded to f16; libm erff in GELU) unless a bit of
 * g_round asks it to take one of the GPU kernels' roundings instead, so that the distance each one
 * adds can be measured on its own:
 *   OR_ROUND_Q16  (1): with f16 K/V, q is rounded to f16 before Q.K^T (the f16 matrix-core attention,
 *                      and ggml's own per-row CPU path and CUDA kernels)
 *   OR_ROUND_P16  (2): with f16 K/V, the softmax weights are rounded to f16 before P.V, and the f32
 *                      normalizer sums those rounded weights (as the GPU kernel's dot2 row sums do)
 *   OR_ROUND_EXP2 (4): weights as 2^(s*c - m*c) with c = scale*log2(e) in float, s the raw dot and m
 *                      the largest raw dot (the GPU kernel's exp2 form), instead of e^(s*scale - max)
 *   OR_ROUND_GELU (8): GELU as the GPU epilogue computes it (one polynomial for log2 of the normal tail
 *                      and one exp2) instead of libm erff */
static int g_round = 0;
void or_set_rounding(int bits) { g_round = bits; }
int or_get_rounding(void) { return g_round; }
void or_set_attn_f16(int on) { g_round = on ? (g_round | 3) : (g_round & ~3); }

void or_attention(const float * q, const float * k, const float * v, int64_t n_q, int64_t n_kv,
                  int n_head, int hd, float scale, int kv_f16, const float * mask, float * out, int n_threads) {
    const int64_t row = (int64_t) n_head * hd;
    for (int h = 0; h < n_head; h++) {
        float * kh = (float *) malloc(sizeof(float) * n_kv * hd);
        float * vh = (float *) malloc(sizeof(float) * n_kv * hd);
        for (int64_t j = 0; j < n_kv; j++)
            for (int d = 0; d < hd; d++) {
                float kv = k[j * row + h * hd + d], vv = v[j * row + h * hd + d];
                if (kv_f16) { kv = or_fp16_to_fp32(or_fp32_to_fp16(kv)); vv = or_fp16_to_fp32(or_fp32_to_fp16(vv)); }
                kh[j * hd + d] = kv; vh[j * hd + d] = vv;
            }
#pragma omp parallel num_threads(n_threads)
        {
            float * sc = (float *) malloc(sizeof(float) * n_kv);
            float acc[1024];
#pragma omp for schedule(static)
            for (int64_t i = 0; i < n_q; i++) {
                const float * qi = q + i * row + h * hd;
                float q16[1024];
                if ((g_round & 1) && kv_f16) {
                    for (int d = 0; d < hd; d++) q16[d] = or_fp16_to_fp32(or_fp32_to_fp16(qi[d]));
                    qi = q16;
                }
                const int exp2_form = (g_round & 4) != 0;
                const float c2 = scale * 1.4426950408889634f;
                float mx = -INFINITY;
                for (int64_t j = 0; j < n_kv; j++) {
                    const float dot = dot_f32_8acc(qi, kh + j * hd, hd);
                    sc[j] = exp2_form ? dot : dot * scale;
                    if (mask) sc[j] = sc[j] + mask[i * n_kv + j];
                    if (sc[j] > mx) mx = sc[j];
                }
                float sum = 0.0f;
                for (int d = 0; d < hd; d++) acc[d] = 0.0f;
                if (mx == -INFINITY) {   /* no visible key */
                    for (int d = 0; d < hd; d++) out[i * row + h * hd + d] = 0.0f;
                    continue;
                }
                const float mc = mx * c2;
                for (int64_t j = 0; j < n_kv; j++) {
                    const float p = exp2_form ? exp2f(fmaf(sc[j], c2, -mc)) : expf(sc[j] - mx);
                    const float pv = ((g_round & 2) && kv_f16) ? or_fp16_to_fp32(or_fp32_to_fp16(p)) : p;
                    sum += pv;
                    const float * vj = vh + j * hd;
                    for (int d = 0; d < hd; d++) acc[d] = fmaf(pv, vj[d], acc[d]);
                }
                const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
                for (int d = 0; d < hd; d++) out[i * row + h * hd + d] = acc[d] * inv;
            }
            free(sc);
        }
        free(kh); free(vh);
    }
}

/* ------------------------------------------------------------------------------------------------
 * minimal GGUF v2/v3 reader (its own code, independent of the product loader)
 * ---------------------------------------------------------------------------------------------- */
typedef struct { char name[128]; int type; int n_dims; int64_t ne[4]; uint64_t offset; } gg_tensor;
typedef struct { char key[96]; int vtype; int64_t ival; double fval; char sval[128]; float farr[4]; int nfarr; } gg_kv;
typedef struct {
    uint8_t * buf; size_t size; size_t data_off;
    gg_kv * kv; int n_kv;
    gg_tensor * t; int n_t;
} gg_file;

static int rd(const gg_file * f, size_t * p, void * dst, size_t n) {
    if (*p + n > f->size) return -1;
    memcpy(dst, f->buf + *p, n); *p += n; return 0;
}
static int rd_str(const gg_file * f, size_t * p, char * dst, size_t cap) {
    uint64_t n; if (rd(f, p, &n, 8)) return -1;
    if (*p + n > f->size) return -1;
    const size_t c = n < cap - 1 ? (size_t) n : cap - 1;
    memcpy(dst, f->buf + *p, c); dst[c] = 0; *p += n; return 0;
}
static size_t gg_scalar_size(int t) {
    switch (t) { case 0: case 1: case 7: return 1; case 2: case 3: return 2; case 4: case 5: case 6: return 4;
                 case 10: case 11: case 12: return 8; }
    return 0;
}
static int rd_scalar(const gg_file * f, size_t * p, int t, int64_t * iv, double * fv) {
    uint8_t b[8] = {0}; const size_t n = gg_scalar_size(t); *iv = 0; *fv = 0;
    if (!n || rd(f, p, b, n)) return -1;
    switch (t) {
        case 0: *iv = b[0]; break; case 1: *iv = (int8_t) b[0]; break; case 7: *iv = b[0] != 0; break;
        case 2: { uint16_t v; memcpy(&v, b, 2); *iv = v; break; } case 3: { int16_t v; memcpy(&v, b, 2); *iv = v; break; }
        case 4: { uint32_t v; memcpy(&v, b, 4); *iv = v; break; } case 5: { int32_t v; memcpy(&v, b, 4); *iv = v; break; }
        case 6: { float v; memcpy(&v, b, 4); *fv = v; *iv = (int64_t) v; return 0; }
        case 10: { uint64_t v; memcpy(&v, b, 8); *iv = (int64_t) v; break; } case 11: { int64_t v; memcpy(&v, b, 8); *iv = v; break; }
        case 12: { double v; memcpy(&v, b, 8); *fv = v; *iv = (int64_t) v; return 0; }
    }
    *fv = (double) *iv;
    return 0;
}

static void gg_close(gg_file * f) { free(f->buf); free(f->kv); free(f->t); memset(f, 0, sizeof(*f)); }

static int gg_open(const char * path, gg_file * f) {
    memset(f, 0, sizeof(*f));
    FILE * fp = fopen(path, "rb");
    if (!fp) { fprintf(stderr, "oracle: cannot open %s\n", path); return -1; }
    fseeko(fp, 0, SEEK_END); f->size = (size_t) ftello(fp); fseeko(fp, 0, SEEK_SET);
    f->buf = (uint8_t *) malloc(f->size);
    if (!f->buf || fread(f->buf, 1, f->size, fp) != f->size) { fclose(fp); gg_close(f); return -1; }
    fclose(fp);
    size_t p = 0; uint32_t magic, ver; uint64_t nt, nkv;
    if (rd(f, &p, &magic, 4) || memcmp(&magic, "GGUF", 4) || rd(f, &p, &ver, 4) || rd(f, &p, &nt, 8) || rd(f, &p, &nkv, 8)) { gg_close(f); return -1; }
    f->kv = (gg_kv *) calloc(nkv + 1, sizeof(gg_kv)); f->t = (gg_tensor *) calloc(nt + 1, sizeof(gg_tensor));
    f->n_kv = (int) nkv; f->n_t = (int) nt;
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        gg_kv * kv = &f->kv[i];
        uint32_t vt;
        if (rd_str(f, &p, kv->key, sizeof(kv->key)) || rd(f, &p, &vt, 4)) { gg_close(f); return -1; }
        kv->vtype = (int) vt;
        if (vt == 8) { if (rd_str(f, &p, kv->sval, sizeof(kv->sval))) { gg_close(f); return -1; } }
        else if (vt == 9) {
            uint32_t et; uint64_t n;
            if (rd(f, &p, &et, 4) || rd(f, &p, &n, 8)) { gg_close(f); return -1; }
            for (uint64_t j = 0; j < n; j++) {
                if (et == 8) { char tmp[8]; if (rd_str(f, &p, tmp, sizeof(tmp))) { gg_close(f); return -1; } }
                else { int64_t iv = 0; double fv = 0; if (rd_scalar(f, &p, (int) et, &iv, &fv)) { gg_close(f); return -1; }
                       if (j < 4) { kv->farr[j] = (float) fv; kv->nfarr = (int) (j + 1); } }
            }
        } else if (rd_scalar(f, &p, (int) vt, &kv->ival, &kv->fval)) { gg_close(f); return -1; }
        if (!strcmp(kv->key, "general.alignment")) alignment = (uint64_t) kv->ival;
    }
    for (uint64_t i = 0; i < nt; i++) {
        gg_tensor * t = &f->t[i];
        uint32_t nd, ty;
        if (rd_str(f, &p, t->name, sizeof(t->name)) || rd(f, &p, &nd, 4) || nd > 4) { gg_close(f); return -1; }
        t->n_dims = (int) nd;
        for (int d = 0; d < 4; d++) t->ne[d] = 1;
        for (uint32_t d = 0; d < nd; d++) { uint64_t v; if (rd(f, &p, &v, 8)) { gg_close(f); return -1; } t->ne[d] = (int64_t) v; }
        if (rd(f, &p, &ty, 4) || rd(f, &p, &t->offset, 8)) { gg_close(f); return -1; }
        t->type = (int) ty;
    }
    f->data_off = (p + alignment - 1) / alignment * alignment;
    return 0;
}

static const gg_kv * gg_find(const gg_file * f, const char * key) {
    for (int i = 0; i < f->n_kv; i++) if (!strcmp(f->kv[i].key, key)) return &f->kv[i];
    return NULL;
}
static int64_t gg_int(const gg_file * f, const char * key, int64_t def) { const gg_kv * k = gg_find(f, key); return k && k->vtype != 8 && k->vtype != 9 ? k->ival : def; }
static double gg_flt(const gg_file * f, const char * key, double def) { const gg_kv * k = gg_find(f, key); return k && k->vtype != 8 && k->vtype != 9 ? k->fval : def; }
static const char * gg_str(const gg_file * f, const char * key, const char * def) { const gg_kv * k = gg_find(f, key); return k && k->vtype == 8 ? k->sval : def; }

static const gg_tensor * gg_tensor_find(const gg_file * f, const char * name) {
    for (int i = 0; i < f->n_t; i++) if (!strcmp(f->t[i].name, name)) return &f->t[i];
    return NULL;
}
static const void * gg_data(const gg_file * f, const gg_tensor * t) { return f->buf + f->data_off + t->offset; }

/* a float vector tensor (f32 required by the reference loader, src/jepa-gguf.cpp:675-701) */
static const float * gg_vec(const gg_file * f, const char * name) {
    const gg_tensor * t = gg_tensor_find(f, name);
    if (!t) return NULL;
    if (t->type != OR_F32) { fprintf(stderr, "oracle: %s is not f32\n", name); return NULL; }
    return (const float *) gg_data(f, t);
}

/* ------------------------------------------------------------------------------------------------
 * encoder forward (src/jepa.cpp:444-471 block, 586-627 image graph, 846-895 video graph)
 * ---------------------------------------------------------------------------------------------- */
typedef struct { const gg_tensor * t; const void * data; } lin_w;

static int linear(const gg_file * f, const char * wname, const char * bname, const float * x, int64_t n_rows,
                  int64_t n_in, int64_t n_out, float * y, int n_threads) {
    const gg_tensor * t = gg_tensor_find(f, wname);
    if (!t || t->ne[0] != n_in || t->ne[1] != n_out) { fprintf(stderr, "oracle: bad/missing %s\n", wname); return -1; }
    const float * b = bname ? gg_vec(f, bname) : NULL;
    return or_mul_mat(t->type, gg_data(f, t), n_out, n_in, x, n_rows, b, y, n_threads);
}

static void patchify(const float * cthw, int C, int T, int H, int W, int P, int tub, float * rows) {
    /* src/jepa.cpp:476-504: token order t, h, w; inner order c, tt, py, px */
    const int GT = T / tub, GH = H / P, GW = W / P;
    const int64_t K = (int64_t) C * tub * P * P;
    for (int t = 0; t < GT; t++)
        for (int h = 0; h < GH; h++)
            for (int w = 0; w < GW; w++) {
                float * row = rows + ((int64_t) t * GH * GW + (int64_t) h * GW + w) * K;
                int64_t o = 0;
                for (int c = 0; c < C; c++)
                    for (int tt = 0; tt < tub; tt++) {
                        const int64_t plane = ((int64_t) c * T + (int64_t) t * tub + tt) * H * W;
                        for (int py = 0; py < P; py++) {
                            memcpy(row + o, cthw + plane + (int64_t) (h * P + py) * W + (int64_t) w * P, sizeof(float) * P);
                            o += P;
                        }
                    }
            }
}

/* One pre-LN block on x [R][D] in place (src/jepa.cpp:444-471), tensors "<pre>ln1.weight" etc.:
 * x += out(attn(rope(qkv(LN1 x)))) [* ls1]; x += down(gelu(up(LN2 x))) [* ls2]. rope_c null: no
 * rotation; mask (optional): additive [R][R]. The block's FFN width is read from its ffn_up tensor. */
static int block_fwd(const gg_file * f, const char * pre, float * x, int64_t R, int D, int H, const float * rope_c,
                     const float * rope_s, const float * mask, int kv_f16, float eps, int n_threads) {
    char n1[128], n2[128];
#define TN(buf, s) (snprintf(buf, sizeof(buf), "%s%s", pre, s), buf)
    const gg_tensor * up = gg_tensor_find(f, TN(n1, "ffn_up.weight"));
    if (!up) { fprintf(stderr, "oracle: missing %s\n", n1); return -1; }
    const int64_t F = up->ne[1];
    const int hd = D / H;
    int rc = -1;
    float * h = (float *) malloc(sizeof(float) * R * D);
    float * qkv = (float *) malloc(sizeof(float) * R * 3 * D);
    float * q = (float *) malloc(sizeof(float) * R * D), * kk = (float *) malloc(sizeof(float) * R * D), * vv = (float *) malloc(sizeof(float) * R * D);
    float * att = (float *) malloc(sizeof(float) * R * D);
    float * o = (float *) malloc(sizeof(float) * R * D);
    float * ff = (float *) malloc(sizeof(float) * R * F);
    or_layer_norm(x, R, D, gg_vec(f, TN(n1, "ln1.weight")), gg_vec(f, TN(n2, "ln1.bias")), eps, h);
    if (gg_tensor_find(f, TN(n1, "attn_qkv.weight"))) {
        if (linear(f, TN(n1, "attn_qkv.weight"), TN(n2, "attn_qkv.bias"), h, R, D, 3 * D, qkv, n_threads)) goto out;
        for (int64_t r = 0; r < R; r++) {
            memcpy(q + r * D, qkv + r * 3 * D, sizeof(float) * D);
            memcpy(kk + r * D, qkv + r * 3 * D + D, sizeof(float) * D);
            memcpy(vv + r * D, qkv + r * 3 * D + 2 * D, sizeof(float) * D);
        }
    } else {   /* separate q, k, v linears (src/jepa.cpp:408-414) */
        if (linear(f, TN(n1, "attn_q.weight"), TN(n2, "attn_q.bias"), h, R, D, D, q, n_threads) ||
            linear(f, TN(n1, "attn_k.weight"), TN(n2, "attn_k.bias"), h, R, D, D, kk, n_threads) ||
            linear(f, TN(n1, "attn_v.weight"), TN(n2, "attn_v.bias"), h, R, D, D, vv, n_threads)) goto out;
    }
    if (rope_c) {   /* q and k rotated before the 1/sqrt(d) scale (src/jepa.cpp:880-882) */
        or_rope_apply(q, R, H, hd, rope_c, rope_s);
        or_rope_apply(kk, R, H, hd, rope_c, rope_s);
    }
    or_attention(q, kk, vv, R, R, H, hd, 1.0f / sqrtf((float) hd), kv_f16, mask, att, n_threads);
    if (linear(f, TN(n1, "attn_out.weight"), TN(n2, "attn_out.bias"), att, R, D, D, o, n_threads)) goto out;
    {
        const float * ls1 = gg_vec(f, TN(n1, "ls1"));
        for (int64_t i = 0; i < R * D; i++) x[i] = x[i] + (ls1 ? o[i] * ls1[i % D] : o[i]);
    }
    or_layer_norm(x, R, D, gg_vec(f, TN(n1, "ln2.weight")), gg_vec(f, TN(n2, "ln2.bias")), eps, h);
    if (linear(f, TN(n1, "ffn_up.weight"), TN(n2, "ffn_up.bias"), h, R, D, F, ff, n_threads)) goto out;
#pragma omp parallel for num_threads(n_threads)
    for (int64_t i = 0; i < R * F; i++) ff[i] = or_gelu_erf(ff[i]);
    if (linear(f, TN(n1, "ffn_down.weight"), TN(n2, "ffn_down.bias"), ff, R, F, D, o, n_threads)) goto out;
    {
        const float * ls2 = gg_vec(f, TN(n1, "ls2"));
        for (int64_t i = 0; i < R * D; i++) x[i] = x[i] + (ls2 ? o[i] * ls2[i % D] : o[i]);
    }
#undef TN
    rc = 0;
out:
    free(h); free(qkv); free(q); free(kk); free(vv); free(att); free(o); free(ff);
    return rc;
}

/* Teacher forcing: when set, block l of item i starts from the residual stream the caller supplies
 * (teacher [n_items][n_layers + 1][R][D], entry l = the input of block l, e.g. a GPU trace) instead of
 * the oracle's own, so the trace's entry l + 1 is this oracle's block l applied to the caller's
 * input: the error of each block alone, without what the earlier blocks passed on. */
static const float * g_teacher = NULL;
static int64_t g_teacher_n = 0;
void or_set_teacher(const float * trace, int64_t n_floats) { g_teacher = trace; g_teacher_n = trace ? n_floats : 0; }
/* With a teacher, blocks before g_first_block are not run: their trace entries are the teacher's own
 * (entry l + 1 = teacher entry l + 1), so a deep model's last blocks can be checked alone. */
static int g_first_block = 0;
void or_set_first_block(int l0) { g_first_block = l0 < 0 ? 0 : l0; }

int64_t or_encode_file(const char * path, const float * in, int n_batch, int n_chans, int n_frames,
                       int height, int width, float * out, int64_t out_cap, float * trace, int64_t trace_cap,
                       int n_layers_limit, int n_threads) {
    gg_file f;
    if (gg_open(path, &f)) return -1;
    int64_t ret = -1;
    const char * fam = gg_str(&f, "jepa.family", "");
    const int video = !strcmp(fam, "vjepa2") || !strcmp(fam, "vjepa2_1") || !strcmp(fam, "levjepa");
    const int image = !strcmp(fam, "hfvit") || !strcmp(fam, "ijepa") || !strcmp(fam, "lewm");
    const int D = (int) gg_int(&f, "jepa.enc.embed_dim", 0), L = (int) gg_int(&f, "jepa.enc.n_layer", 0);
    const int H = (int) gg_int(&f, "jepa.enc.n_head", 0);
    const int P = (int) gg_int(&f, "jepa.enc.patch_size", 16), C = (int) gg_int(&f, "jepa.enc.in_chans", 3);
    const int cls = (int) gg_int(&f, "jepa.enc.cls_token", 0), n_reg = (int) gg_int(&f, "jepa.enc.n_registers", 0);
    const float eps = (float) gg_flt(&f, "jepa.enc.ln_eps", 1e-6);
    const int file_type = (int) gg_int(&f, "general.file_type", 0);
    const int hd = H > 0 ? D / H : 0;
    const int n_layers = n_layers_limit > 0 && n_layers_limit < L ? n_layers_limit : L;
    if ((!video && !image) || D <= 0 || H <= 0 || n_chans != C || n_reg < 0) {
        fprintf(stderr, "oracle: family '%s' / shape not covered by the oracle\n", fam);
        gg_close(&f); return -1;
    }
    const char * act = gg_str(&f, "jepa.enc.act", "gelu_erf");
    if (strcmp(act, "gelu_erf") != 0 && strcmp(act, "gelu") != 0) {
        fprintf(stderr, "oracle: only gelu_erf is restated\n"); gg_close(&f); return -1;
    }
    const int kv_f16 = file_type != 0;   /* JEPA_KV_AUTO on the CPU, src/jepa.cpp:531-535 */

    int tub = video ? (int) gg_int(&f, "jepa.enc.tubelet_size", 1) : 1;
    int image_path = 0;
    if (video && n_frames == 1 && gg_int(&f, "jepa.enc.image_patch_embed", 0) && gg_tensor_find(&f, "enc.patch_embed_img.weight")) {
        image_path = 1; tub = 1;   /* src/jepa.cpp:771-775 */
    }
    const int n_items = video ? n_batch : n_batch * n_frames;
    const int T = video ? n_frames : 1;
    if (height % P || width % P || T % tub) { fprintf(stderr, "oracle: shape not encodable\n"); gg_close(&f); return -1; }
    const int GT = T / tub, GH = height / P, GW = width / P;
    const int64_t Np = (int64_t) GT * GH * GW;
    /* prefix rows in front of the patch rows: the CLS row (hfvit; levjepa: the video family with one),
     * then the register rows (src/jepa.cpp:598-608 and 868-881 concatenate the registers, then CLS) */
    const int np = (cls ? 1 : 0) + n_reg;
    const int64_t R = Np + np;
    const int block_causal = !strcmp(gg_str(&f, "jepa.enc.attn_mode", "full"), "block_causal");
    if (block_causal && !video) { fprintf(stderr, "oracle: block_causal needs a video family\n"); gg_close(&f); return -1; }
    const int64_t K = (int64_t) C * tub * P * P;
    if (out_cap < (int64_t) n_items * R * D) { fprintf(stderr, "oracle: output too small\n"); gg_close(&f); return -1; }

    float * rope_c = NULL, * rope_s = NULL;
    if (video) {
        or_rope_params rp;
        rp.grid_t = GT; rp.grid_h = GH; rp.grid_w = GW; rp.head_dim = hd;
        rp.theta = (float) gg_flt(&f, "jepa.enc.rope_theta", 10000.0);
        rp.variant = !strcmp(gg_str(&f, "jepa.enc.rope_freq_layout", ""), "interleaved") ? 1 : 0;
        rp.interpolate = (int) gg_int(&f, "jepa.enc.rope_interpolate", 0);
        rp.train_grid_h = rp.train_grid_w = (int) gg_int(&f, "jepa.enc.rope_ref_grid", 0);
        /* the prefix rows carry no position: identity rows (cos 1, sin 0), src/jepa.cpp:960-966 */
        rope_c = (float *) malloc(sizeof(float) * R * hd); rope_s = (float *) malloc(sizeof(float) * R * hd);
        for (int64_t i = 0; i < (int64_t) np * hd; i++) { rope_c[i] = 1.0f; rope_s[i] = 0.0f; }
        or_rope_tables(&rp, NULL, Np, rope_c + (int64_t) np * hd, rope_s + (int64_t) np * hd, 1);
    }
    float * mask = NULL;
    if (block_causal) {
        mask = (float *) malloc(sizeof(float) * R * R);
        or_block_causal_mask(GT, GH, GW, np, mask);
    }

    float * rows = (float *) malloc(sizeof(float) * Np * K);
    float * x = (float *) malloc(sizeof(float) * R * D);
    float * chw = (float *) malloc(sizeof(float) * C * height * width * (video ? T : 1));
    const int64_t plane = (int64_t) height * width;

    for (int it = 0; it < n_items; it++) {
        /* gather the item (video: the whole clip; image: the (b, t) slice) and patchify */
        if (video) {
            memcpy(chw, in + (int64_t) it * C * T * plane, sizeof(float) * C * T * plane);
            patchify(chw, C, T, height, width, P, tub, rows);
        } else {
            const int b = it / n_frames, t = it % n_frames;
            for (int c = 0; c < C; c++) memcpy(chw + c * plane, in + (((int64_t) b * n_chans + c) * n_frames + t) * plane, sizeof(float) * plane);
            patchify(chw, C, 1, height, width, P, 1, rows);
        }
        float * xp = x + (R - Np) * D;   /* patch rows after the prefix */
        const char * pw = image_path ? "enc.patch_embed_img.weight" : "enc.patch_embed.weight";
        const char * pb = image_path ? "enc.patch_embed_img.bias" : "enc.patch_embed.bias";
        if (linear(&f, pw, pb, rows, Np, K, D, xp, n_threads)) goto done;
        if (video && gg_int(&f, "jepa.enc.modality_embed", 0)) {
            const float * mod = gg_vec(&f, image_path ? "enc.mod_embed_img" : "enc.mod_embed_video");
            if (!mod) goto done;
            for (int64_t r = 0; r < Np; r++) for (int d = 0; d < D; d++) xp[r * D + d] = xp[r * D + d] + mod[d];
        }
        if (cls) {   /* after the patch embedding, no position information (src/jepa.cpp:865-880) */
            const float * ct = gg_vec(&f, "enc.cls_token");
            if (!ct) goto done;
            memcpy(x, ct, sizeof(float) * D);
        }
        if (n_reg > 0) {   /* enc.reg_tokens [n_reg][D] after the CLS row (src/jepa.cpp:598-601, 868-874) */
            const gg_tensor * rt = gg_tensor_find(&f, "enc.reg_tokens");
            const float * rv = gg_vec(&f, "enc.reg_tokens");
            if (!rt || !rv || rt->ne[0] != D || rt->ne[1] != n_reg) { fprintf(stderr, "oracle: enc.reg_tokens missing or mis-shaped\n"); goto done; }
            memcpy(x + (int64_t) (cls ? 1 : 0) * D, rv, sizeof(float) * n_reg * D);
        }
        if (image) {
            const float * pos = gg_vec(&f, "enc.pos_embed");
            if (pos) {
                const gg_tensor * pt = gg_tensor_find(&f, "enc.pos_embed");
                if (pt->ne[1] != R) { fprintf(stderr, "oracle: pos_embed rows %lld != %lld\n", (long long) pt->ne[1], (long long) R); goto done; }
                for (int64_t r = 0; r < R; r++) for (int d = 0; d < D; d++) x[r * D + d] = x[r * D + d] + pos[r * D + d];
            }
        }
        if (trace) {
            const int64_t off = ((int64_t) it * (n_layers + 1)) * R * D;
            if (off + R * D > trace_cap) { fprintf(stderr, "oracle: trace too small\n"); goto done; }
            memcpy(trace + off, x, sizeof(float) * R * D);
        }
        for (int l = 0; l < n_layers; l++) {
            char pre[64];
            snprintf(pre, sizeof(pre), "enc.blk.%d.", l);
            if (g_teacher) {
                const int64_t off = (((int64_t) it * (n_layers + 1)) + l) * R * D;
                if (off + R * D > g_teacher_n) { fprintf(stderr, "oracle: teacher trace too small\n"); goto done; }
                memcpy(x, g_teacher + off, sizeof(float) * R * D);
                if (l < g_first_block) {
                    if (off + 2 * R * D > g_teacher_n) { fprintf(stderr, "oracle: teacher trace too small\n"); goto done; }
                    if (trace) memcpy(trace + (((int64_t) it * (n_layers + 1)) + l + 1) * R * D, g_teacher + off + R * D, sizeof(float) * R * D);
                    continue;
                }
            }
            if (block_fwd(&f, pre, x, R, D, H, video ? rope_c : NULL, rope_s, mask, kv_f16, eps, n_threads)) goto done;
            if (trace) memcpy(trace + (((int64_t) it * (n_layers + 1)) + l + 1) * R * D, x, sizeof(float) * R * D);
        }
        or_layer_norm(x, R, D, gg_vec(&f, "enc.norm.weight"), gg_vec(&f, "enc.norm.bias"), eps, out + (int64_t) it * R * D);
    }
    ret = R;
done:
    free(rows); free(x); free(chw);
    free(rope_c); free(rope_s); free(mask);
    gg_close(&f);
    return ret;
}

/* ------------------------------------------------------------------------------------------------
 * attentive-pool head (src/jepa.cpp:1026-1075): n_pool_layers self-attention blocks without RoPE on
 * the encoder rows, then one learned query cross-attends to LN_kv of them (no output projection);
 * y = q0 + attn; y += ffn_down(gelu(ffn_up(LN2 y))); logits = cls(y). The cross-attention K/V stay
 * f32 (kv_type F32 on the CPU, src/jepa.cpp:1053-1058); the blocks use the encoder's K/V rule.
 * ---------------------------------------------------------------------------------------------- */
int64_t or_head_file(const char * path, const float * x_in, int64_t N, float * pooled, float * logits, int64_t logits_cap,
                     int n_threads) {
    gg_file f;
    if (gg_open(path, &f)) return -1;
    int64_t ret = -1;
    const int D = (int) gg_int(&f, "jepa.enc.embed_dim", 0), H = (int) gg_int(&f, "jepa.enc.n_head", 0);
    const int n_pool = (int) gg_int(&f, "jepa.head.n_pool_layers", 0);
    const float eps = (float) gg_flt(&f, "jepa.enc.ln_eps", 1e-6);
    const int kv_f16 = gg_int(&f, "general.file_type", 0) != 0;
    const int hd = H > 0 ? D / H : 0;
    float * x = NULL, * kv = NULL, * k = NULL, * v = NULL, * q = NULL, * y = NULL, * h = NULL, * ff = NULL, * o = NULL;
    if (strcmp(gg_str(&f, "jepa.head.kind", "none"), "attentive_pool") != 0 || D <= 0 || H <= 0 || N <= 0) {
        fprintf(stderr, "oracle: no attentive-pool head\n"); goto done;
    }
    const gg_tensor * up = gg_tensor_find(&f, "head.xattn.ffn_up.weight");
    const gg_tensor * cls = gg_tensor_find(&f, "head.cls.weight");
    const float * q0 = gg_vec(&f, "head.query");
    if (!up || !cls || !q0) { fprintf(stderr, "oracle: head tensors missing\n"); goto done; }
    const int64_t F = up->ne[1], C = cls->ne[1];
    if (C > logits_cap) { fprintf(stderr, "oracle: logits buffer too small\n"); goto done; }
    x = (float *) malloc(sizeof(float) * N * D); kv = (float *) malloc(sizeof(float) * N * D);
    k = (float *) malloc(sizeof(float) * N * D); v = (float *) malloc(sizeof(float) * N * D);
    q = (float *) malloc(sizeof(float) * D); y = (float *) malloc(sizeof(float) * D); h = (float *) malloc(sizeof(float) * D);
    o = (float *) malloc(sizeof(float) * D); ff = (float *) malloc(sizeof(float) * F);
    memcpy(x, x_in, sizeof(float) * N * D);
    for (int l = 0; l < n_pool; l++) {
        char pre[64];
        snprintf(pre, sizeof(pre), "head.blk.%d.", l);
        if (block_fwd(&f, pre, x, N, D, H, NULL, NULL, NULL, kv_f16, eps, n_threads)) goto done;
    }
    or_layer_norm(x, N, D, gg_vec(&f, "head.xattn.ln_kv.weight"), gg_vec(&f, "head.xattn.ln_kv.bias"), eps, kv);
    if (linear(&f, "head.xattn.q.weight", "head.xattn.q.bias", q0, 1, D, D, q, n_threads) ||
        linear(&f, "head.xattn.k.weight", "head.xattn.k.bias", kv, N, D, D, k, n_threads) ||
        linear(&f, "head.xattn.v.weight", "head.xattn.v.bias", kv, N, D, D, v, n_threads)) goto done;
    or_attention(q, k, v, 1, N, H, hd, 1.0f / sqrtf((float) hd), 0, NULL, o, n_threads);
    for (int d = 0; d < D; d++) y[d] = o[d] + q0[d];   /* residual on the raw query */
    or_layer_norm(y, 1, D, gg_vec(&f, "head.xattn.ln2.weight"), gg_vec(&f, "head.xattn.ln2.bias"), eps, h);
    if (linear(&f, "head.xattn.ffn_up.weight", "head.xattn.ffn_up.bias", h, 1, D, F, ff, n_threads)) goto done;
    for (int64_t i = 0; i < F; i++) ff[i] = or_gelu_erf(ff[i]);
    if (linear(&f, "head.xattn.ffn_down.weight", "head.xattn.ffn_down.bias", ff, 1, F, D, o, n_threads)) goto done;
    for (int d = 0; d < D; d++) y[d] = y[d] + o[d];
    if (pooled) memcpy(pooled, y, sizeof(float) * D);
    if (logits && linear(&f, "head.cls.weight", "head.cls.bias", y, 1, D, C, logits, n_threads)) goto done;
    ret = C;
done:
    free(x); free(kv); free(k); free(v); free(q); free(y); free(h); free(o); free(ff);
    gg_close(&f);
    return ret;
}

/* ------------------------------------------------------------------------------------------------
 * masked predictor (src/predictor.cpp:23-285): context rows (gathered at the context ids) through
 * pred.embed (or the 2-layer MLP pred.embed.0 / .2), mask token row mask_index % n_mask for every
 * target, + the modality vector (2.1), 3-D RoPE from the token ids on the predictor grid, the pred.blk
 * blocks, pred.norm, and pred.proj of the target rows. LayerNorm epsilon: the encoder's.
 * modality: 1 video, 2 image (resolved by the caller).
 * ---------------------------------------------------------------------------------------------- */
int64_t or_predict_file(const char * path, const float * enc, int64_t n_tok, const int32_t * ctx_ids, int n_ctx,
                        const int32_t * tgt_ids, int n_tgt, int mask_index, int modality, float * out, int64_t out_cap,
                        int n_threads) {
    gg_file f;
    if (gg_open(path, &f)) return -1;
    int64_t ret = -1;
    const int De = (int) gg_int(&f, "jepa.enc.embed_dim", 0);
    const int Dp = (int) gg_int(&f, "jepa.pred.embed_dim", 0), L = (int) gg_int(&f, "jepa.pred.n_layer", 0);
    const int H = (int) gg_int(&f, "jepa.pred.n_head", 0);
    const int hd0 = (int) gg_int(&f, "jepa.pred.head_dim", 0), hd = hd0 > 0 ? hd0 : (H > 0 ? Dp / H : 0);
    const int out_dim = (int) gg_int(&f, "jepa.pred.out_dim", De);
    const float eps = (float) gg_flt(&f, "jepa.enc.ln_eps", 1e-6);
    const int kv_f16 = gg_int(&f, "general.file_type", 0) != 0;
    const int64_t N = (int64_t) n_ctx + n_tgt;
    float * x = NULL, * rc = NULL, * rs = NULL, * rows = NULL, * hid = NULL, * h = NULL;
    int32_t * ids = NULL;
    if (strcmp(gg_str(&f, "jepa.pred.kind", "none"), "masked") != 0 || Dp <= 0 || H <= 0 || hd * H != Dp || n_tgt <= 0 || n_ctx < 0) {
        fprintf(stderr, "oracle: no masked predictor / bad shape\n"); goto done;
    }
    if ((int64_t) n_tgt * out_dim > out_cap) { fprintf(stderr, "oracle: output too small\n"); goto done; }
    ids = (int32_t *) malloc(sizeof(int32_t) * N);
    int64_t max_id = 0;
    for (int i = 0; i < n_ctx; i++) { ids[i] = ctx_ids ? ctx_ids[i] : i; if (ids[i] < 0 || ids[i] >= n_tok) { fprintf(stderr, "oracle: bad context id\n"); goto done; } }
    for (int i = 0; i < n_tgt; i++) { ids[n_ctx + i] = tgt_ids ? tgt_ids[i] : i; if (ids[n_ctx + i] < 0) { fprintf(stderr, "oracle: bad target id\n"); goto done; } }
    for (int64_t i = 0; i < N; i++) if (ids[i] > max_id) max_id = ids[i];
    x = (float *) malloc(sizeof(float) * N * Dp);
    /* 1. context rows */
    if (n_ctx > 0) {
        rows = (float *) malloc(sizeof(float) * n_ctx * De);
        for (int i = 0; i < n_ctx; i++) memcpy(rows + (int64_t) i * De, enc + (int64_t) ids[i] * De, sizeof(float) * De);
        const gg_tensor * e0 = gg_tensor_find(&f, "pred.embed.0.weight");
        if (e0) {
            const int64_t nh = e0->ne[1];
            hid = (float *) malloc(sizeof(float) * n_ctx * nh);
            if (linear(&f, "pred.embed.0.weight", "pred.embed.0.bias", rows, n_ctx, De, nh, hid, n_threads)) goto done;
            for (int64_t i = 0; i < n_ctx * nh; i++) hid[i] = or_gelu_erf(hid[i]);
            if (linear(&f, "pred.embed.2.weight", "pred.embed.2.bias", hid, n_ctx, nh, Dp, x, n_threads)) goto done;
        } else if (linear(&f, "pred.embed.weight", "pred.embed.bias", rows, n_ctx, De, Dp, x, n_threads)) goto done;
    }
    /* 2. mask token rows */
    {
        const gg_tensor * mt = gg_tensor_find(&f, "pred.mask_tokens");
        if (!mt || mt->type != OR_F32 || mt->ne[0] != Dp) { fprintf(stderr, "oracle: pred.mask_tokens\n"); goto done; }
        const int64_t nm0 = gg_int(&f, "jepa.pred.n_mask_tokens", 0), n_mask = nm0 > 0 ? nm0 : mt->ne[1];
        int64_t idx = n_mask > 0 ? mask_index % n_mask : 0;
        if (idx < 0) idx += n_mask;
        const float * row = (const float *) gg_data(&f, mt) + idx * Dp;
        for (int i = 0; i < n_tgt; i++) memcpy(x + ((int64_t) n_ctx + i) * Dp, row, sizeof(float) * Dp);
    }
    /* 3. modality vector on every row */
    if (gg_int(&f, "jepa.pred.modality_embed", 0)) {
        const float * mod = gg_vec(&f, modality == 2 ? "pred.mod_embed_img" : "pred.mod_embed_video");
        if (!mod) { fprintf(stderr, "oracle: modality vector missing\n"); goto done; }
        for (int64_t r = 0; r < N; r++) for (int d = 0; d < Dp; d++) x[r * Dp + d] = x[r * Dp + d] + mod[d];
    }
    /* 4. RoPE tables from the ids (src/predictor.cpp:23-49) */
    {
        or_rope_params rp;
        const int gs = (int) gg_int(&f, "jepa.pred.grid_size", 0);
        const int grid = gs > 0 ? gs : (int) (gg_int(&f, "jepa.enc.img_size", 224) / gg_int(&f, "jepa.enc.patch_size", 16));
        rp.grid_h = rp.grid_w = grid;
        rp.grid_t = (int) (max_id / ((int64_t) grid * grid)) + 1;
        rp.head_dim = hd;
        rp.theta = (float) gg_flt(&f, "jepa.enc.rope_theta", 10000.0);
        rp.interpolate = (int) gg_int(&f, "jepa.pred.rope_interpolate", 0);
        rp.train_grid_h = rp.train_grid_w = (int) gg_int(&f, "jepa.pred.rope_ref_grid", 0);
        const char * lay = gg_str(&f, "jepa.pred.rope_freq_layout", "");
        rp.variant = lay[0] ? !strcmp(lay, "interleaved") : !strcmp(gg_str(&f, "jepa.family", ""), "vjepa2_1");
        rc = (float *) malloc(sizeof(float) * N * hd);
        rs = (float *) malloc(sizeof(float) * N * hd);
        or_rope_tables(&rp, ids, N, rc, rs, 1);
    }
    for (int l = 0; l < L; l++) {
        char pre[64];
        snprintf(pre, sizeof(pre), "pred.blk.%d.", l);
        if (block_fwd(&f, pre, x, N, Dp, H, rc, rs, NULL, kv_f16, eps, n_threads)) goto done;
    }
    h = (float *) malloc(sizeof(float) * n_tgt * Dp);
    or_layer_norm(x + (int64_t) n_ctx * Dp, n_tgt, Dp, gg_vec(&f, "pred.norm.weight"), gg_vec(&f, "pred.norm.bias"), eps, h);
    if (linear(&f, "pred.proj.weight", "pred.proj.bias", h, n_tgt, Dp, out_dim, out, n_threads)) goto done;
    ret = out_dim;
done:
    free(x); free(rc); free(rs); free(rows); free(hid); free(h); free(ids);
    gg_close(&f);
    return ret;
}
