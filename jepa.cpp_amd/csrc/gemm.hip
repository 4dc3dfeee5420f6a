// gemm.hip - block-quantized and f16 GEMMs for gfx950 (MFMA), with fused epilogues.
//
// Computes Y[m][n] = sum_k X[m][k] * W[n][k] for the encoder's linear layers (the ggml_mul_mat of
// reference src/jepa.cpp:365-375) with ggml's CPU numerics:
//   q8_0 / q4_0 weights x q8_0 activations:  sum_b dw[n,b] * da[m,b] * S_b[m,n]   (S_b exact integer)
//   q4_K weights x q8_K activations:         sum_sb (dw*da) * sum_j sc_j S_j  -  (dmin*da) * sum_j m_j bsum_j
//   f16 weights x f16-rounded activations:   f32 accumulation of exact f16 products
//
// MFMA mapping (v_mfma_f32_32x32x16_f16, wave64). The integer codes of both operands are held as
// f16 values, which are exact (|q| <= 945), so every MFMA product and every partial sum of a 32-deep
// block is an exact integer in f32. Per 32-deep block and 32x32 output tile a wave issues:
//   2 MFMAs  S  = A_blk . B_blk                       (the exact block sum S_b, already f32)
//   1 MFMA   sc = dw (x) da                            (outer product of the two f16 scale vectors:
//                                                       one non-zero K slot, so sc = dw*da exactly)
//   16 VALU  acc = fma(S, sc, acc)                     (one rounding per block, like ggml's AVX2 fmadd)
// so the per-block scale epilogue costs one VALU op per output element instead of three
// (convert + scale product + fma), and the kernel is MFMA-bound rather than VALU-bound.
//
// Tiling: 256 threads = 4 waves in a 2x2 arrangement; block tile 128 (n) x 128 (m); each wave owns
// 64 x 64 = 2 x 2 MFMA tiles with W rows on the MFMA "A" side, so a lane's 16 accumulators are
// 4 groups of 4 consecutive output features of ONE token: RoPE pairs, 32-feature quantization
// blocks and float4 stores all stay inside a lane (or a lane and its xor-32 partner).
// K advances 64 per LDS stage (two 32-blocks); global loads of stage k+1 are issued before the
// MFMAs of stage k. LDS rows are padded to 144 B so the 16-byte operand reads of 8 consecutive
// rows hit disjoint banks.
#include "kernels.h"
#include "model.h"

#include <hip/hip_fp16.h>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

namespace {

constexpr int BN = 128, BM = 128, KC = 64;

struct kargs {
    const _Float16 * A; const uint16_t * Ad; const uint16_t * Admin; const _Float16 * Amin;
    const _Float16 * B; const void * Bd; const _Float16 * Bsum;
    const float * bias;
    int64_t M, N, K;
    gemm_epi ep;
};

__device__ __forceinline__ float h2f(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2hbits(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

__device__ __forceinline__ float gelu_erf(float x) {
    // 0.5*x*(1 + erf(x/sqrt(2))) - ggml_vec_gelu_erf_f32 (reference docs/ggml-notes.md:291-292)
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, erff(__fmul_rn(x, SQRT_2_INV))));
}

__device__ __forceinline__ int perm16(int64_t tok) {
    // position of token `tok` inside its 16-token group of V^T (see attention.hip)
    const int key = (int) (tok & 15);
    const int gg = (key >> 2) & 1, s = (key & 3) + 4 * (key >> 3);
    return (int) (tok & ~(int64_t) 15) + 8 * gg + s;
}

// Epilogue of 4 consecutive features n..n+3 of row m (values t[] = raw accumulators).
template <int EPI>
__device__ __forceinline__ void epi4(const kargs & a, int64_t m, int64_t n, float t[4]) {
    const gemm_epi & ep = a.ep;
    if (a.bias) {
        const float4 b = *(const float4 *) (a.bias + n);
        t[0] = __fadd_rn(t[0], b.x); t[1] = __fadd_rn(t[1], b.y); t[2] = __fadd_rn(t[2], b.z); t[3] = __fadd_rn(t[3], b.w);
    }
    if constexpr (EPI == EPI_F32) {
        if (ep.addvec) {
            const float4 v = *(const float4 *) (ep.addvec + n);
            t[0] = __fadd_rn(t[0], v.x); t[1] = __fadd_rn(t[1], v.y); t[2] = __fadd_rn(t[2], v.z); t[3] = __fadd_rn(t[3], v.w);
        }
        const int64_t item = m / ep.rin, r = m - item * ep.rin;
        const int64_t row = item * ep.rout + ep.pre + r;
        if (ep.addrows) {
            const float4 v = *(const float4 *) (ep.addrows + (ep.pre + r) * ep.ldy + n);
            t[0] = __fadd_rn(t[0], v.x); t[1] = __fadd_rn(t[1], v.y); t[2] = __fadd_rn(t[2], v.z); t[3] = __fadd_rn(t[3], v.w);
        }
        *(float4 *) (ep.y + row * ep.ldy + n) = make_float4(t[0], t[1], t[2], t[3]);
    } else if constexpr (EPI == EPI_RESID) {
        if (ep.ls) {
            const float4 v = *(const float4 *) (ep.ls + n);
            t[0] = __fmul_rn(t[0], v.x); t[1] = __fmul_rn(t[1], v.y); t[2] = __fmul_rn(t[2], v.z); t[3] = __fmul_rn(t[3], v.w);
        }
        float4 * px = (float4 *) (ep.y + m * ep.ldy + n);
        float4 x = *px;
        x.x = __fadd_rn(x.x, t[0]); x.y = __fadd_rn(x.y, t[1]); x.z = __fadd_rn(x.z, t[2]); x.w = __fadd_rn(x.w, t[3]);
        *px = x;
    } else if constexpr (EPI == EPI_GELU_F32) {
        *(float4 *) (ep.y + m * ep.ldy + n) = make_float4(gelu_erf(t[0]), gelu_erf(t[1]), gelu_erf(t[2]), gelu_erf(t[3]));
    } else if constexpr (EPI == EPI_GELU_F16) {
        _Float16 * o = (_Float16 *) ep.oh + m * ep.ldy + n;
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 v = {(_Float16) gelu_erf(t[0]), (_Float16) gelu_erf(t[1]), (_Float16) gelu_erf(t[2]), (_Float16) gelu_erf(t[3])};
        *(h4 *) o = v;
    } else if constexpr (EPI == EPI_QKV) {
        const int D = ep.D, hd = ep.hd;
        const int which = (int) (n / D);
        const int nn = (int) (n - (int64_t) which * D);
        const int h = nn / hd, d0 = nn - h * hd;
        const int64_t item = m / ep.R, tok = m - item * ep.R;
        const int64_t head = item * ep.n_head + h;
        if (which < 2) {
            float o[4];
            if (ep.rope_c) {
                // out = x*C + swap(x)*S' (reference src/rope3d.cpp:136-164): two products, one add
                const float4 c = *(const float4 *) (ep.rope_c + tok * hd + d0);
                const float4 s = *(const float4 *) (ep.rope_s + tok * hd + d0);
                o[0] = __fadd_rn(__fmul_rn(t[0], c.x), __fmul_rn(t[1], s.x));
                o[1] = __fadd_rn(__fmul_rn(t[1], c.y), __fmul_rn(t[0], s.y));
                o[2] = __fadd_rn(__fmul_rn(t[2], c.z), __fmul_rn(t[3], s.z));
                o[3] = __fadd_rn(__fmul_rn(t[3], c.w), __fmul_rn(t[2], s.w));
            } else {
                o[0] = t[0]; o[1] = t[1]; o[2] = t[2]; o[3] = t[3];
            }
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            h4 v = {(_Float16) o[0], (_Float16) o[1], (_Float16) o[2], (_Float16) o[3]};
            _Float16 * dst = (_Float16 *) (which == 0 ? ep.q : ep.k) + (head * ep.R_pad + tok) * hd + d0;
            *(h4 *) dst = v;
        } else {
            _Float16 * vt = (_Float16 *) ep.vt + head * hd * ep.R_pad;
            const int p = perm16(tok);
            for (int e = 0; e < 4; e++) vt[(int64_t) (d0 + e) * ep.R_pad + p] = (_Float16) t[e];
        }
    }
}

// LDS tile of 128 rows x 64 f16 (128 B per row, 8 chunks of 16 B). Chunk c of row r is stored at
// position c ^ (r & 7): the 16-byte operand reads of 8 consecutive rows then hit 8 different bank
// groups, and a wave's direct HBM->LDS load (64 lanes x 16 B) fills 8 whole rows contiguously.
__device__ __forceinline__ int swz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }

typedef __attribute__((address_space(3))) void lds_void;

// Stage rows [R0, R0 + 8) of a 128 x 64 f16 tile straight from HBM into LDS: lane L loads row
// R0 + L/8, logical chunk (L%8) ^ (row & 7), and the hardware writes it at lds_row0 + 16 * L.
__device__ __forceinline__ void lds_load_rows(const _Float16 * src, int64_t ld, int64_t row0_global, int64_t row_max,
                                              int64_t k0, _Float16 * lds_tile, int R0, int lane) {
    const int r = R0 + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    int64_t gr = row0_global + r;
    if (gr > row_max) gr = row_max;        // rows past the end load a valid row; their results are dropped
    __builtin_amdgcn_global_load_lds((const void *) (src + gr * ld + k0 + 8 * c), (lds_void *) (lds_tile + R0 * 64), 16, 0, 0);
}

template <int WF, int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm_mfma(kargs a) {
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BN * KC];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][BM * KC];
    __shared__ uint16_t sAd[2][BN * 2];
    __shared__ uint16_t sBd[2][BM * 2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int l32 = lane & 31, g = lane >> 5;
    const int64_t n0 = (int64_t) blockIdx.x * BN, m0 = (int64_t) blockIdx.y * BM;
    const int64_t K = a.K, M = a.M;

    f16v acc[2][2];
    [[maybe_unused]] f16v ssb[2][2];
    const f16v zero = {0};
    for (int i = 0; i < 2; i++) for (int j = 0; j < 2; j++) { acc[i][j] = zero; if constexpr (WF == W_Q4K) ssb[i][j] = zero; }

    // one stage = 2 x 16 wave-loads of 1 KB (A and B tiles), 8 per wave
    auto issue_tiles = [&](int64_t k0, int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int R0 = (wave * 4 + i) * 8;
            lds_load_rows(a.A, K, n0, a.N - 1, k0, sA[buf], R0, lane);
            lds_load_rows(a.B, K, m0, M - 1, k0, sB[buf], R0, lane);
        }
    };
    uint16_t rad = 0, rbd = 0;
    auto load_scales = [&](int64_t k0) {
        if constexpr (WF == W_Q32) {
            const int row = tid >> 1, blk = tid & 1;
            rad = a.Ad[(n0 + row) * (K / 32) + k0 / 32 + blk];
            const int64_t mr = m0 + row;
            rbd = mr < M ? ((const uint16_t *) a.Bd)[mr * (K / 32) + k0 / 32 + blk] : (uint16_t) 0;
        }
    };
    auto store_scales = [&](int buf) {
        if constexpr (WF == W_Q32) { sAd[buf][tid] = rad; sBd[buf][tid] = rbd; }
    };

    const int64_t nst = K / KC;
    issue_tiles(0, 0);
    load_scales(0);
    store_scales(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int64_t st = 0; st < nst; st++) {
        const int cur = (int) (st & 1);
        const int64_t k0 = st * KC;
        if (st + 1 < nst) { issue_tiles(k0 + KC, cur ^ 1); load_scales(k0 + KC); }
        const _Float16 * A_ = sA[cur];
        const _Float16 * B_ = sB[cur];
#pragma unroll 1
        for (int blk = 0; blk < 2; blk++) {
            h8 bv[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int row = 64 * wm + 32 * j + l32;
#pragma unroll
                for (int hh = 0; hh < 2; hh++) bv[j][hh] = *(const h8 *) &B_[swz(row, blk * 4 + hh * 2 + g)];
            }
            [[maybe_unused]] h8 sb[2];
            if constexpr (WF == W_Q32) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    // da in K-slot 0 of lane group 0 only; group 1 contributes zeros
                    const uint32_t d = g == 0 ? (uint32_t) sBd[cur][(64 * wm + 32 * j + l32) * 2 + blk] : 0u;
                    sb[j] = __builtin_bit_cast(h8, make_uint4(d, 0u, 0u, 0u));
                }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (i == 1) __builtin_amdgcn_sched_barrier(0);
                const int row = 64 * wn + 32 * i + l32;
                const h8 a0 = *(const h8 *) &A_[swz(row, blk * 4 + g)];
                const h8 a1 = *(const h8 *) &A_[swz(row, blk * 4 + 2 + g)];
                if constexpr (WF == W_F16) {
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        acc[i][j] = MFMA16(a0, bv[j][0], acc[i][j]);
                        acc[i][j] = MFMA16(a1, bv[j][1], acc[i][j]);
                    }
                } else if constexpr (WF == W_Q32) {
                    // dw in K-slot 0 (both lane groups hold row n's scale; group 1 meets zeros in B)
                    const h8 sa = __builtin_bit_cast(h8, make_uint4((uint32_t) sAd[cur][row * 2 + blk], 0u, 0u, 0u));
                    f16v S0 = MFMA16(a0, bv[0][0], zero);
                    f16v S1 = MFMA16(a0, bv[1][0], zero);
                    const f16v c0 = MFMA16(sa, sb[0], zero);
                    const f16v c1 = MFMA16(sa, sb[1], zero);
                    S0 = MFMA16(a1, bv[0][1], S0);
                    S1 = MFMA16(a1, bv[1][1], S1);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[i][0][r] = fmaf(S0[r], c0[r], acc[i][0][r]);
                        acc[i][1][r] = fmaf(S1[r], c1[r], acc[i][1][r]);
                    }
                } else {   // W_Q4K: integer sums over the 256-deep super-block
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        ssb[i][j] = MFMA16(a0, bv[j][0], ssb[i][j]);
                        ssb[i][j] = MFMA16(a1, bv[j][1], ssb[i][j]);
                    }
                }
            }
        }
        if constexpr (WF == W_Q4K) {
            if (((k0 + KC) & 255) == 0) {
                const int64_t sbi = k0 >> 8, nsb = K >> 8;
                h8 bs[2];
                float da[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int64_t m = m0 + 64 * wm + 32 * j + l32;
                    const bool ok = m < M;
                    const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                    bs[j] = ok ? *(const h8 *) (a.Bsum + m * (K / 16) + sbi * 16 + g * 8) : z;
                    da[j] = ok ? ((const float *) a.Bd)[m * nsb + sbi] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int64_t nr = n0 + 64 * wn + 32 * i + l32;
                    const h8 am = *(const h8 *) (a.Amin + (nr * nsb + sbi) * 16 + g * 8);
                    float dw[16], dm[16];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int64_t n = n0 + 64 * wn + 32 * i + 8 * q + 4 * g;
                        const ushort4 v = *(const ushort4 *) (a.Ad + sbi * a.N + n);
                        const ushort4 u = *(const ushort4 *) (a.Admin + sbi * a.N + n);
                        dw[4 * q + 0] = h2f(v.x); dw[4 * q + 1] = h2f(v.y); dw[4 * q + 2] = h2f(v.z); dw[4 * q + 3] = h2f(v.w);
                        dm[4 * q + 0] = h2f(u.x); dm[4 * q + 1] = h2f(u.y); dm[4 * q + 2] = h2f(u.z); dm[4 * q + 3] = h2f(u.w);
                    }
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const f16v ms = MFMA16(am, bs[j], zero);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const float d1 = __fmul_rn(dw[r], da[j]), d2 = __fmul_rn(dm[r], da[j]);
                            acc[i][j][r] = fmaf(d1, ssb[i][j][r], acc[i][j][r]);
                            acc[i][j][r] = fmaf(-d2, ms[r], acc[i][j][r]);
                        }
                        ssb[i][j] = zero;
                    }
                }
            }
        }
        if (st + 1 < nst) store_scales(cur ^ 1);
        __builtin_amdgcn_s_waitcnt(0);                // this wave's HBM->LDS copies have landed
        __syncthreads();                              // ... and everyone else's
    }

    // epilogue: lane holds token m and features n0 + 64wn + 32i + 8q + 4g + e
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int64_t m = m0 + 64 * wm + 32 * j + l32;
            const int64_t nb = n0 + 64 * wn + 32 * i;
            if constexpr (EPI == EPI_GELU_Q8_0) {
                // q8_0 activation of the next linear, x86 rule: d = amax/127 (f16), q = rne(x*127/amax)
                float v[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int64_t n = nb + 8 * q + 4 * g;
                    const float4 b = a.bias ? *(const float4 *) (a.bias + n) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    v[4 * q + 0] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 0], b.x));
                    v[4 * q + 1] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 1], b.y));
                    v[4 * q + 2] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 2], b.z));
                    v[4 * q + 3] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 3], b.w));
                }
                float am = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(v[r]));
                am = fmaxf(am, __shfl_xor(am, 32));
                const float d = am / 127.0f;
                const float id = am != 0.0f ? 127.0f / am : 0.0f;
                if (m < M) {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int64_t n = nb + 8 * q + 4 * g;
                        h4 o;
#pragma unroll
                        for (int e = 0; e < 4; e++) o[e] = (_Float16) fminf(fmaxf(rintf(v[4 * q + e] * id), -128.0f), 127.0f);
                        *(h4 *) ((_Float16 *) a.ep.oq + m * a.N + n) = o;
                    }
                    if (g == 0) ((uint16_t *) a.ep.od)[m * (a.N / 32) + nb / 32] = f2hbits(d);
                }
            } else {
                if (m >= M) continue;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int64_t n = nb + 8 * q + 4 * g;
                    float t[4] = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    epi4<EPI>(a, m, n, t);
                }
            }
        }
    }
}

// f32 weights x f32 activations (hfvit patch embedding and f32 files): VALU FMA, 64x64 tiles,
// each thread 4 tokens x 4 consecutive features, K staged 16 at a time through LDS.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_f32(kargs a) {
    __shared__ float sW[16][64 + 4];
    __shared__ float sX[16][64 + 4];
    const int tid = threadIdx.x;
    const int tn = tid & 15, tm = tid >> 4;
    const int64_t n0 = (int64_t) blockIdx.x * 64, m0 = (int64_t) blockIdx.y * 64;
    const float * W = (const float *) a.A;
    const float * X = (const float *) a.B;
    float acc[4][4] = {{0}};
    for (int64_t k0 = 0; k0 < a.K; k0 += 16) {
        for (int c = tid; c < 64 * 16; c += 256) {
            const int r = c >> 4, kk = c & 15;
            const int64_t n = n0 + r, m = m0 + r, k = k0 + kk;
            sW[kk][r] = (n < a.N && k < a.K) ? W[n * a.K + k] : 0.0f;
            sX[kk][r] = (m < a.M && k < a.K) ? X[m * a.K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            float w[4], x[4];
#pragma unroll
            for (int e = 0; e < 4; e++) { w[e] = sW[kk][4 * tn + e]; x[e] = sX[kk][4 * tm + e]; }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][e] = fmaf(x[i], w[e], acc[i][e]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + 4 * tm + i, n = n0 + 4 * tn;
        if (m < a.M && n < a.N) epi4<EPI>(a, m, n, acc[i]);
    }
}

// f32 fused-qkv rows -> Q, K (RoPE'd) and V^T through the same epilogue the QKV GEMM runs
__global__ void k_qkv_split(kargs a, const float * __restrict__ qkv) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t groups = a.N / 4;
    if (id >= a.M * groups) return;
    const int64_t m = id / groups, n = (id % groups) * 4;
    const float4 v = *(const float4 *) (qkv + m * a.N + n);
    float t[4] = {v.x, v.y, v.z, v.w};
    epi4<EPI_QKV>(a, m, n, t);
}

template <int WF>
void dispatch_mfma(const kargs & a, hipStream_t s) {
    dim3 grid((unsigned) (a.N / BN), (unsigned) ((a.M + BM - 1) / BM));
    switch (a.ep.kind) {
        case EPI_F32:       k_gemm_mfma<WF, EPI_F32><<<grid, 256, 0, s>>>(a); break;
        case EPI_RESID:     k_gemm_mfma<WF, EPI_RESID><<<grid, 256, 0, s>>>(a); break;
        case EPI_GELU_F32:  k_gemm_mfma<WF, EPI_GELU_F32><<<grid, 256, 0, s>>>(a); break;
        case EPI_GELU_F16:  k_gemm_mfma<WF, EPI_GELU_F16><<<grid, 256, 0, s>>>(a); break;
        case EPI_GELU_Q8_0: k_gemm_mfma<WF, EPI_GELU_Q8_0><<<grid, 256, 0, s>>>(a); break;
        case EPI_QKV:       k_gemm_mfma<WF, EPI_QKV><<<grid, 256, 0, s>>>(a); break;
    }
}

}  // namespace

void launch_gemm(const dev_linear & W, const act_view & X, int64_t M, const gemm_epi & ep, hipStream_t s) {
    kargs a{};
    a.A = (const _Float16 *) W.w;
    a.Ad = (const uint16_t *) W.wd;
    a.Admin = (const uint16_t *) W.wdmin;
    a.Amin = (const _Float16 *) W.wmin;
    a.B = (const _Float16 *) X.q;
    a.Bd = X.d;
    a.Bsum = (const _Float16 *) X.bsum;
    a.bias = W.bias;
    a.M = M; a.N = W.n_out; a.K = W.n_in;
    a.ep = ep;
    if (M <= 0) return;
    if (W.fmt == W_F32) {
        dim3 grid((unsigned) ((a.N + 63) / 64), (unsigned) ((M + 63) / 64));
        switch (ep.kind) {
            case EPI_F32:      k_gemm_f32<EPI_F32><<<grid, 256, 0, s>>>(a); break;
            case EPI_RESID:    k_gemm_f32<EPI_RESID><<<grid, 256, 0, s>>>(a); break;
            case EPI_GELU_F32: k_gemm_f32<EPI_GELU_F32><<<grid, 256, 0, s>>>(a); break;
            case EPI_QKV:      k_gemm_f32<EPI_QKV><<<grid, 256, 0, s>>>(a); break;
            default: jepa_log("jepa: internal error: epilogue %d has no f32 GEMM\n", ep.kind); break;
        }
        return;
    }
    switch (W.fmt) {
        case W_F16: dispatch_mfma<W_F16>(a, s); break;
        case W_Q32: dispatch_mfma<W_Q32>(a, s); break;
        case W_Q4K: dispatch_mfma<W_Q4K>(a, s); break;
    }
}

void launch_qkv_split(const float * qkv, int64_t M, int64_t N, const gemm_epi & ep, hipStream_t s) {
    kargs a{};
    a.M = M; a.N = N; a.K = 0;
    a.ep = ep;
    const int64_t total = M * (N / 4);
    if (total > 0) k_qkv_split<<<(unsigned) ((total + 255) / 256), 256, 0, s>>>(a, qkv);
}
