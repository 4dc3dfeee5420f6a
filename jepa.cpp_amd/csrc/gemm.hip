// gemm.hip - block-quantized and f16 GEMMs for gfx950 (MFMA), with fused epilogues.
//
// Computes Y[m][n] = sum_k X[m][k] * W[n][k] for the encoder's linear layers (the ggml_mul_mat of
// reference src/jepa.cpp:365-375) with ggml's CPU numerics:
//   q8_0 / q4_0 weights x q8_0 activations:  sum_b dw[n,b] * da[m,b] * S_b[m,n]   (S_b exact integer)
//   q4_K weights x q8_K activations:         sum_sb (dw*da) * sum_j sc_j S_j  -  (dmin*da) * sum_j m_j bsum_j
//   f16 weights x f16-rounded activations:   f32 accumulation of exact f16 products
//
// q8_0 (int8 codes in HBM and LDS) and q4_0 (4-bit codes in HBM and LDS, each unpacked in registers to
// the int8 16 (q - 8)), per 32-deep block b and 32x32 output tile:
//   v_mfma_i32_32x32x32_i8   S  = A_b . B_b (with at most two MFMA tiles per wave started from the bits
//                               of 1.5 * 2^23, so that the int32 result read as a float is 12582912 + S;
//                               q4_0: 1.5 * 2^19 + 16 S, read as the float 786432 + S)
//   v_mfma_f32_32x32x8_f16   c  = dw_b (x) da_b (an outer product of the two f16 scale vectors; one
//                               non-zero K slot, so every c = dw * da is exact)
//   32 VALU                  acc = fma(float(S), c, acc): one rounding per block
// q4_K (4-bit codes in HBM and LDS, unpacked in registers), per 256-deep super-block: int8 MFMAs sum
// (sh q) . a and (sl q) . a over its eight sub-blocks (sc = 8 sh + sl), one float epilogue per super-block.
// f16 weights run f16 MFMAs (v_mfma_f32_32x32x16_f16) over 64-column stages.
//
// Workgroups are eight waves (two per SIMD); a wave owns TI x TJ tiles of 32 x 32 with the weight
// rows on the MFMA "A" side, so a lane's 16 accumulators are 4 groups of 4 consecutive output features
// of one token (RoPE pairs, 32-feature quantization blocks and float4 stores stay inside a lane or a
// lane and its xor-32 partner). Operand stages of 128 bytes per row are copied HBM -> LDS by buffer
// loads with an LDS destination into an XOR-swizzled layout, several stages in flight.
#include "kernels.h"
#include "model.h"
#include "lds_dma.h"
#include "lanes.h"
#include "quant_dev.h"

#include <hip/hip_fp16.h>

#include <atomic>
#include <type_traits>

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef unsigned int u4v __attribute__((ext_vector_type(4)));

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)
#define MFMA8(a, b, c) __builtin_amdgcn_mfma_f32_32x32x8f16((a), (b), (c), 0, 0, 0)
#define MFMA_I8(a, b, c) __builtin_amdgcn_mfma_i32_32x32x32_i8((a), (b), (c), 0, 0, 0)

namespace {

struct kargs {
    const _Float16 * A;      // [N][K] weight codes (or f16 / f32 weights)
    const uint16_t * Ad;     // W_Q32, W_Q40: f16 d [N][K/32]; W_Q4K: u32 (d | dmin << 16) [K/256][N]
    const _Float16 * Amin;   // W_Q4K: [N][K/256][16] sub-block mins, each twice
    const uint8_t * Asc;     // W_Q4K: [N][K/256][8] 6-bit sub-block scales
    const _Float16 * B;      // [M][K] activation codes (or f16 / f32 activations)
    const void * Bd;         // A_Q8_0: f16 d [M][K/32]; A_Q8_K: f32 d [M][K/256]
    const _Float16 * Bsum;   // A_Q8_K: f16 bsums [M][K/16]
    const float * bias;
    int64_t M, N, K;
    int tn, tm;              // workgroup tiles along N and M
    int xa, xb;              // tiles per XCD block along N and M (0: plain order)
    int split;               // K halves computed by separate workgroups (1 or 2; q8_0 / q4_0 / q4_K)
    float * part;            // split: raw accumulators of every workgroup [split][tiles][BN*BM]
    int * cnt;               // split: arrivals per tile (0 between launches)
    gemm_epi ep;
};

__device__ __forceinline__ float h2f(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2hbits(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

// GELU(x) = 0.5 x (1 + erf(x / sqrt 2)) = x Phi(x) (ggml_vec_gelu_erf_f32, reference
// docs/ggml-notes.md:291-292), Phi the standard normal CDF, from its tail h(t) = Phi(-t), t = |x|:
//   Phi(x) = 1 - h(t) for x >= 0, h(t) for x < 0,   h(t) = 2^Q(min(t, 5.5)), Q of degree 8 with Q(0) = -1
// One polynomial and one hardware exp2 per value, no branch: 14 VALU ops where erf's two-piece form
// (both pieces evaluated, one selected) took 25. Coefficients from fit_gelu.py (fitted with weight h,
// so the absolute error of Phi is minimised; Q(0) = -1 gives Phi(0) = 1/2 exactly): the float32
// evaluation stays within 1.5 units of 2^-24 of Phi (2.5 with exp2 two units off), about the accuracy
// of the libm erff form. At t = 5.5, h = 1.9e-8 < 2^-25, so 1 - h is 1.0f and GELU(x) = x beyond.
__device__ __forceinline__ float gelu_erf(float x) {
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
    const float h = __builtin_amdgcn_exp2f(q);
    return __fmul_rn(x, x >= 0.0f ? __fsub_rn(1.0f, h) : h);
}

// The residual epilogue with the row's current values x already loaded: x + (t + bias) * ls
// (bias b and layer scale v already loaded: zero / unused when absent)
__device__ __forceinline__ void resid4(const kargs & a, int64_t m, int64_t n, float t[4], float4 x, float4 b, float4 v) {
    const gemm_epi & ep = a.ep;
    if (a.bias) {
        t[0] = __fadd_rn(t[0], b.x); t[1] = __fadd_rn(t[1], b.y); t[2] = __fadd_rn(t[2], b.z); t[3] = __fadd_rn(t[3], b.w);
    }
    if (ep.ls) {
        t[0] = __fmul_rn(t[0], v.x); t[1] = __fmul_rn(t[1], v.y); t[2] = __fmul_rn(t[2], v.z); t[3] = __fmul_rn(t[3], v.w);
    }
    x.x = __fadd_rn(x.x, t[0]); x.y = __fadd_rn(x.y, t[1]); x.z = __fadd_rn(x.z, t[2]); x.w = __fadd_rn(x.w, t[3]);
    *(float4 *) (ep.y + m * ep.ldy + n) = x;
}

// The f32-output epilogue with its operands already loaded: bias b, modality vector v, position row r
__device__ __forceinline__ void f32out4(const kargs & a, int64_t m, int64_t n, float t[4], float4 b, float4 v, float4 r) {
    const gemm_epi & ep = a.ep;
    if (a.bias) { t[0] = __fadd_rn(t[0], b.x); t[1] = __fadd_rn(t[1], b.y); t[2] = __fadd_rn(t[2], b.z); t[3] = __fadd_rn(t[3], b.w); }
    if (ep.addvec) { t[0] = __fadd_rn(t[0], v.x); t[1] = __fadd_rn(t[1], v.y); t[2] = __fadd_rn(t[2], v.z); t[3] = __fadd_rn(t[3], v.w); }
    if (ep.addrows) { t[0] = __fadd_rn(t[0], r.x); t[1] = __fadd_rn(t[1], r.y); t[2] = __fadd_rn(t[2], r.z); t[3] = __fadd_rn(t[3], r.w); }
    const int64_t item = m / ep.rin, rr = m - item * ep.rin;
    const int64_t row = item * ep.rout + ep.pre + rr;
    *(float4 *) (ep.y + row * ep.ldy + n) = make_float4(t[0], t[1], t[2], t[3]);
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
        const int D = ep.D, hd = ep.hd, hds = ep.hds ? ep.hds : hd;
        const int64_t ng = n + ep.col0;        // column of the [q | k | v] layout (the bias above is this launch's)
        const int which = (int) (ng / D);
        const int nn = (int) (ng - (int64_t) which * D);
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
            _Float16 * dst = (_Float16 *) (which == 0 ? ep.q : ep.k) + (head * ep.R_pad + tok) * hds + d0;
            *(h4 *) dst = v;
        } else {
            _Float16 * vt = (_Float16 *) ep.vt + head * hds * ep.R_pad;
            const int p = perm16(tok);
            for (int e = 0; e < 4; e++) vt[(int64_t) (d0 + e) * ep.R_pad + p] = (_Float16) t[e];
        }
    }
}

// Stage barrier: wait until at most N_ of this wave's HBM->LDS copies are outstanding and its LDS reads
// have returned (s_waitcnt vmcnt(N_) lgkmcnt(0); gfx9 encoding: vmcnt in bits [3:0] and [15:14],
// expcnt [6:4], lgkmcnt [11:8]), then a bare s_barrier. __syncthreads() would add a workgroup fence,
// which waits for every copy in flight and so drains the pipeline at each stage.
template <int N_>
__device__ __forceinline__ void stage_barrier() {
    static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit field");
    __builtin_amdgcn_s_waitcnt((N_ & 15) | ((N_ >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
}

// Workgroup tile geometry. WN x WM waves (8: two per SIMD, so one wave's MFMAs fill the other's
// barrier, LDS-latency and VALU phases, and eight waves keep enough HBM->LDS copies in flight: a wave
// sustains only ~10 GB/s of loads), each owning TI x TJ MFMA tiles of 32 x 32. The workgroup tile is
// BN = 32 WN TI weight rows by BM = 32 WM TJ tokens. One LDS stage holds 128 B of every one of the
// BN + BM rows, 16-byte chunks swizzled by lds_slot(): KC = 128 K-columns of int8
// codes (q8_0 / q4_0, plus the four f16 block scales of every row) or 64 K-columns of f16 values
// (f16 weights, q4_K codes). q4_K keeps its super-block data (d/dmin, mins, activation d, bsums) in a
// separate double buffer.
template <int WF, int WN, int WM, int TI, int TJ>
struct tiling {
    static constexpr int NW = WN * WM, NT = 64 * NW;
    static constexpr int BN = 32 * WN * TI, BM = 32 * WM * TJ;
    // LDS rows of 128 B per stage: the weight rows (q4_K: two rows of 64 B of 4-bit codes share one),
    // then the activation rows
    static constexpr int AROWS = WF == W_Q4K || WF == W_Q40 ? BN / 2 : BN;
    static constexpr int ROWS = AROWS + BM;
    static constexpr int ESZ = WF == W_F16 ? 2 : 1;          // bytes per activation code
    static constexpr int KC = 128 / ESZ;                      // K-columns per stage
    static constexpr int TILE = ROWS * 128;
    static constexpr int STAGE = TILE;
    // q4_K super-block data (one set per 256 K = two stages): per weight row (d | dmin << 16), the eight
    // 6-bit sub-block scales as bytes and the 16 f16 mins; per token the q8_K d and the 16 f16 bsums.
    // Three buffers: the set of super-block sb + 1 is copied while stage 2 sb + 3 - NST is computed,
    // and every wave is then past the epilogue of sb - 2 (end of stage 2 sb - 3) when NST <= 4.
    static constexpr int X_DW = 0, X_SC = BN * 4, X_MIN = X_SC + BN * 8, X_DA = X_MIN + BN * 32, X_BS = X_DA + BM * 4;
    static constexpr int XSB = WF == W_Q4K ? X_BS + BM * 32 : 0;
    static constexpr int NXSB = WF == W_Q4K ? 3 : 0;
    // At most four stages in LDS (three in flight beyond the one computed): the 128x64 tile with six
    // (its LDS fits them) issued a 120 KB burst of copies per workgroup at the start and ran slower
    // (ViT-L out-proj 0.39 -> 0.36 ms and fc2 0.89 -> 0.86 ms per clip with four, ViT-S/16 0.554 ->
    // 0.529 ms per image; five and three measured in between)
    static constexpr int NST_MAX = 4;
    static constexpr int NST_FIT = (160 * 1024 - NXSB * XSB) / STAGE;
    static constexpr int NST = NST_FIT < NST_MAX ? NST_FIT : NST_MAX;
    static constexpr int LDS = NST * STAGE + NXSB * XSB;
    static constexpr int LOADS = ROWS / 8 / NW;    // 1 KB tile loads per wave per stage
    static constexpr int PARTS = LOADS;            // copies per wave per stage (q4_K adds its own)
    static constexpr int SLD = WF == W_Q32 || WF == W_Q40 ? TI + TJ : 0;   // q8_0 / q4_0 scale loads per wave per stage
    static_assert(NST >= 2, "LDS too small for two stages");
    static_assert(AROWS % (8 * NW) == 0 && BN % 64 == 0 && BM % 64 == 0 && ROWS % (8 * NW) == 0, "load split");
    static_assert((NST - 2) * PARTS < 64, "vmcnt range");
};

// 16-byte chunk c of LDS row r sits in slot c ^ ((r >> 1) & 7). Rows are 128 B, so even and odd rows
// start in opposite halves of the 64 banks; keying the slot on r >> 1 gives the 16 rows a ds_read_b128
// serves together (one chunk each) 16 different 4-bank groups.
__device__ __forceinline__ int lds_slot(int r, int c) { return c ^ ((r >> 1) & 7); }

template <class V>
__device__ __forceinline__ V lds_chunk(const unsigned char * base, int r, int c) {
    return *(const V *) (base + r * 128 + (lds_slot(r, c) << 4));
}

// LDS reads in inline asm, for data whose copy is known to have landed (by the stage barriers): the
// compiler cannot tell their addresses from the HBM->LDS copies in flight and would wait for all of
// those (vmcnt(0)) before an ordinary read. The caller waits for the results with lds_wait() and
// passes each through lds_take() before its first use.
__device__ __forceinline__ uint32_t lds_addr(const void * p) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) void *) p;
}
template <class V>
__device__ __forceinline__ V lds_read_asm(const void * p) {
    V r;
    if constexpr (sizeof(V) == 16) asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
    else if constexpr (sizeof(V) == 8) asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
    else asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
    return r;
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <class V>
__device__ __forceinline__ void lds_take(V & v) { asm volatile("" : "+v"(v)); }

// Y[m][n] over the workgroup tile (n0, m0). K advances one stage (KC) per iteration; NST - 1 stages
// are in flight as direct HBM->LDS copies (buffer_load_dwordx4 ... lds: each lane moves 16 B, a wave
// 8 rows), so a stage's loads have NST - 1 compute phases to land. One barrier per stage.
// The fields the prologue needs come first as scalar arguments, which the dispatch preloads into SGPRs
// (-amdgpu-kernarg-preload-count: a struct argument is not preloaded), so that the first copies do
// not wait on a load of the argument block; the rest of kargs follows in memory (launch: GEMM_ARGS).
// EPI_QKV_RE: the QKV epilogue in the form that copies its RoPE rows during the last two K stages
// (chosen by the launcher, below; its kernels run with EPI = EPI_QKV and RE set).
constexpr int EPI_QKV_RE = EPI_GELU_Q8_K + 1;

template <int WF, int EPI_, int WN, int WM, int TI, int TJ>
__global__ __launch_bounds__(64 * WN * WM, 1) void k_gemm_mfma(const void * pA, const void * pB, const void * pAd, const void * pBd,
                                                               int pM, int pN, int pK, int ptn, int ptm, int psplit, kargs a_rest) {
    constexpr bool RE = EPI_ == EPI_QKV_RE;
    constexpr int EPI = RE ? EPI_QKV : EPI_;
    kargs a = a_rest;
    a.A = (const _Float16 *) pA; a.B = (const _Float16 *) pB; a.Ad = (const uint16_t *) pAd; a.Bd = pBd;
    a.M = pM; a.N = pN; a.K = pK; a.tn = ptn; a.tm = ptm; a.split = psplit;
    using T = tiling<WF, WN, WM, TI, TJ>;
    constexpr int BN = T::BN, NST = T::NST, NW = T::NW, KC = T::KC, ESZ = T::ESZ;
    __shared__ __attribute__((aligned(16))) unsigned char smem[T::LDS];

    // wave index made uniform (readfirstlane) so the per-wave copy selection stays scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, wm = wave / WN;
    const int l32 = lane & 31, g = lane >> 5;

    // Workgroups are dealt to the 8 XCDs round-robin (workgroup w runs on XCD w % 8). Each XCD gets one
    // block of xa x xb tiles, chosen on the host so that the weight and activation rows the XCD's L2
    // has to fetch (xa BN + xb BM rows per K-column) are fewest.
    // split-K (residual and plain epilogues only; elsewhere it folds away): workgroups
    // [s * tiles, (s + 1) * tiles) compute K part s of every tile
    constexpr bool SPLITTABLE = (EPI == EPI_RESID || EPI == EPI_F32);
    const int split = SPLITTABLE ? a.split : 1;
    const int ntile = a.tn * a.tm;
    const int sp = split > 1 ? (int) blockIdx.x / ntile : 0;
    const int bid = (int) blockIdx.x - sp * ntile;
    int64_t tni, tmi;
    if (a.xa > 0) {
        const int x = bid & 7, slot = bid >> 3;
        const int nbn = a.tn / a.xa;
        tni = (int64_t) (x % nbn) * a.xa + slot / a.xb;
        tmi = (int64_t) (x / nbn) * a.xb + slot % a.xb;
    } else {
        tni = bid / a.tm;
        tmi = bid - tni * a.tm;
    }
    const int64_t n0 = tni * BN, m0 = tmi * T::BM;
    const int64_t K = a.K, M = a.M, KB = K >> 5;
    // stages of this workgroup (q8_0 / q4_0: the last stage may hold 64 columns; a split has whole
    // stages per half) and the K-stage its addresses start at
    const int64_t nst = split > 1 ? K / KC / split : (K + KC - 1) / KC;
    const int64_t kst0 = (int64_t) sp * nst;
    const int64_t rowbytes = K * ESZ;                                  // activation row
    const int64_t rowbytesA = WF == W_Q4K || WF == W_Q40 ? K / 2 : rowbytes;   // weight row (4-bit codes)

    // buffer resources rebased at the tile's first weight row and first token, so that every copy's
    // offset stays below 4 GiB
    const brsrc rA = make_brsrc((const unsigned char *) a.A + n0 * rowbytesA, (a.N - n0) * rowbytesA);
    const brsrc rB = make_brsrc((const unsigned char *) a.B + m0 * rowbytes, (M - m0) * rowbytes);
    [[maybe_unused]] brsrc rAd, rBd, rAmin, rBs, rAsc;
    [[maybe_unused]] const int64_t nsb = K >> 8;
    if constexpr (WF == W_Q32 || WF == W_Q40) {
        rAd = make_brsrc(a.Ad + n0 * KB, (a.N - n0) * KB * 2);
        rBd = make_brsrc((const uint16_t *) a.Bd + m0 * KB, (M - m0) * KB * 2);
    }
    if constexpr (WF == W_Q4K) {
        rAd = make_brsrc((const uint32_t *) a.Ad + n0, (nsb * a.N - n0) * 4);
        rAmin = make_brsrc(a.Amin + n0 * nsb * 16, (a.N - n0) * nsb * 32);
        rAsc = make_brsrc(a.Asc + n0 * nsb * 8, (a.N - n0) * nsb * 8);
        rBd = make_brsrc((const float *) a.Bd + m0 * nsb, (M - m0) * nsb * 4);
        rBs = make_brsrc(a.Bsum + m0 * (K >> 4), (M - m0) * (K >> 4) * 2);
    }
    // token row of this tile for tile-relative row r (rows past M repeat row M - 1; results dropped)
    auto tok_row = [&](int r) -> uint32_t { return (uint32_t) (m0 + r < M ? r : M - 1 - m0); };

    // Copy i (0 <= i < LOADS) of stage st: this wave's 1 KB of 8 tile rows (128 B each). Lane L fills
    // slot L % 8 of row r, i.e. chunk lds_slot(r, L % 8); the rows one wave copies are equal modulo 16
    // (8 NW is a multiple of 16), so the chunk is the same for all of them. In a final half stage
    // (64 bytes left in the row) chunks 4..7 repeat 0..3 and are never read.
    static_assert((8 * NW) % 16 == 0, "copy rows of a wave must agree modulo 16");
    auto issue_tile = [&](int64_t st, int64_t sa, int i) {
        unsigned char * base = smem + (int) (st % NST) * T::STAGE;
        const int64_t k0 = (sa + kst0) * KC;
        const int c = lds_slot(8 * wave + (lane >> 3), lane & 7);
        const uint32_t soff = (uint32_t) (k0 * ESZ);
        const uint32_t cb = 16 * ((k0 * ESZ + 128 > rowbytes) ? (c & 3) : c);
        const int L = NW * i + wave;
        const int r = 8 * L + (lane >> 3);
        if (i < T::AROWS / (8 * NW)) {
            if constexpr (WF == W_Q4K || WF == W_Q40) {   // LDS row r: weight rows 2r (chunks 0-3) and 2r + 1 (chunks 4-7), 64 B each
                const int cw = lds_slot(r, lane & 7);
                dma_to_lds<16>(rA, (uint32_t) (2 * r + (cw >> 2)) * (uint32_t) rowbytesA + 16 * (cw & 3), (uint32_t) (k0 / 2), base + 1024 * L);
            } else
                dma_to_lds<16>(rA, (uint32_t) r * (uint32_t) rowbytes + cb, soff, base + 1024 * L);
        } else {
            dma_to_lds<16>(rB, tok_row(r - T::AROWS) * (uint32_t) rowbytes + cb, soff, base + 1024 * L);
        }
    };
    // q8_0 / q4_0 stages issue their PARTS copies one per compute step of the stage NST - 1 earlier
    // (spread, so that no wave stalls behind a burst of copies). Stages past the end copy the last
    // stage's data again into the buffer of the stage just finished, which no one reads any more:
    // the copies stay unconditional (a branch around them would split the software pipeline). In the
    // RE kernels they all go to the buffer of stage nst (that of stage nst - 4, long finished, or one
    // no stage uses), so that the buffers of stages nst - 3 and nst - 2 are free for the RoPE rows.
    [[maybe_unused]] auto issue_part = [&](int64_t st, int p) {
        const int64_t sa = st < nst ? st : nst - 1;
        issue_tile(RE ? (st < nst ? st : nst) : st, sa, p);
    };
    // RE (QKV epilogue with early RoPE rows, chosen on the host for q8_0 / q4_0 weights, heads of 64, K
    // a whole number of at least three stages and tiles with four stage buffers): the main loop copies
    // the cos and sin rows of the tile's tokens before its last two stages, cos rows into the buffer of
    // stage nst - 3, sin rows into that of stage nst - 2 (both read for the last time before the
    // barrier of the stage after them), so that they land during those stages instead of after them.
    // The layout is the epilogue's: copy L holds rows 4 L .. 4 L + 3, 16-byte chunk c of row r in
    // slot c ^ (r mod 16). Tiles of V columns take no RoPE: their copies go through empty resources
    // and read nothing (no branch splits the pipeline).
    constexpr int RCH = T::BM * 64 * 4 / 1024;   // 1 KB copies per table
    [[maybe_unused]] brsrc rRc, rRs;
    if constexpr (RE) {
        static_assert(EPI == EPI_QKV && (WF == W_Q32 || WF == W_Q40) && RCH % NW == 0 && T::BM * 64 * 4 <= T::STAGE &&
                      NST >= 4, "early RoPE rows need four stage buffers of at least BM rows of 64 floats");
        const int64_t tb = n0 + a.ep.col0 < 2 * (int64_t) a.ep.D ? (int64_t) a.ep.R * 64 * 4 : 0;
        rRc = make_brsrc(a.ep.rope_c, tb);
        rRs = make_brsrc(a.ep.rope_s, tb);
    }
    [[maybe_unused]] auto issue_rope_rows = [&](const brsrc & r, int64_t st) {
        unsigned char * dst = smem + (int) (st % NST) * T::STAGE;
        const int r_l = lane >> 4, sl = lane & 15;
#pragma unroll
        for (int c = 0; c < RCH / NW; c++) {
            const int L = NW * c + wave, row = 4 * L + r_l;
            const int64_t m = m0 + row, mm = m < M ? m : M - 1;
            dma_to_lds<16>(r, (uint32_t) ((mm % a.ep.R) * 256 + ((sl ^ (row & 15)) << 4)), 0, dst + 1024 * L);
        }
    };
    // q4_K super-block data of this workgroup's super-block st / 2 (data of K super-block (st + kst0) / 2),
    // copied with stage st when st is even, into buffer (st / 2) % 3; nothing past the last stage
    auto issue_xsb = [&](int64_t st) {
        if constexpr (WF == W_Q4K) {
            if ((st & 1) == 0 && st < nst) {
                const uint32_t sb = (uint32_t) ((st + kst0) >> 1);
                unsigned char * xb = smem + NST * T::STAGE + (int) ((st >> 1) % 3) * T::XSB;
                constexpr int N1 = BN / 64, N5 = BN / 32, N2 = BN / 32, N3 = T::BM / 64, N4 = T::BM / 32;
                for (int L = wave; L < N1 + N5 + N2 + N3 + N4; L += NW) {
                    if (L < N1) {
                        dma_to_lds<4>(rAd, (uint32_t) (sb * a.N + 64 * L + lane) * 4, 0, xb + T::X_DW + 256 * L);
                    } else if (L < N1 + N5) {   // sub-block scales: two lanes per row, one dword each
                        const int L5 = L - N1;
                        const uint32_t n = 32 * L5 + (lane >> 1);
                        dma_to_lds<4>(rAsc, (n * (uint32_t) nsb + sb) * 8 + 4 * (lane & 1), 0, xb + T::X_SC + 256 * L5);
                    } else if (L < N1 + N5 + N2) {
                        const int L2 = L - N1 - N5;
                        const uint32_t n = 32 * L2 + (lane >> 1);
                        dma_to_lds<16>(rAmin, ((n * (uint32_t) nsb + sb) * 16 + 8 * (lane & 1)) * 2, 0, xb + T::X_MIN + 1024 * L2);
                    } else if (L < N1 + N5 + N2 + N3) {
                        const int L3 = L - N1 - N5 - N2;
                        const uint32_t m = tok_row(64 * L3 + lane);
                        dma_to_lds<4>(rBd, (m * (uint32_t) nsb + sb) * 4, 0, xb + T::X_DA + 256 * L3);
                    } else {
                        const int L4 = L - N1 - N5 - N2 - N3;
                        const uint32_t m = tok_row(32 * L4 + (lane >> 1));
                        dma_to_lds<16>(rBs, (m * (uint32_t) (K >> 4) + sb * 16 + 8 * (lane & 1)) * 2, 0, xb + T::X_BS + 1024 * L4);
                    }
                }
            }
        }
    };
    // all copies of stage st (the prologue of the q4_K fallback loop)
    auto issue = [&](int64_t st) {
        issue_xsb(st);
#pragma unroll
        for (int i = 0; i < T::LOADS; i++) issue_tile(st, st, i);
    };

    f16v acc[TI][TJ];
    [[maybe_unused]] f16v accm[TI][TJ];   // q4_K: mins accumulator
    const f16v zero = {};
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            acc[i][j] = zero;
            if constexpr (WF == W_Q4K) accm[i][j] = zero;
        }

    // ---- q8_0 / q4_0 ----
    // A stage holds 4 blocks of 32 K-columns. Steps u = (block, tile), tiles i-major, U = 4 TI TJ per
    // stage: one int8 MFMA gives the exact block sum S, one f16 MFMA (32x32x8) of the scale operands
    // gives the exact f32 dw[n] * da[m], and acc = fma(float(S), dw*da, acc).
    // Scale operands, read once per stage: the weight row's four f16 block scales, as they lie in LDS,
    // fill K-slots 0-3 (both lane groups); the token's scale of block blk alone fills K-slot blk of lane
    // group 0 (group 1 is zero), so the product picks dw_blk * da_blk.
    // The 32 VALU ops per step (magic-offset subtraction or conversion, then the fma) bound this path:
    // at four cycles each they take four times the int8 MFMA's 32 cycles, and the matrix unit runs
    // alongside them (VALU work during 60-70 % of its busy cycles, by counters). Everything else is
    // meant to hide behind them:
    //  - software pipeline: operand chunks are read two steps ahead, the MFMAs of step u+1 are issued
    //    before the VALU work of step u, across stage boundaries;
    //  - the barrier that publishes stage st+1 sits two steps before the end of stage st, after the
    //    wave's last LDS read of stage st, so the first reads of stage st+1 overlap the last steps;
    //  - each step issues one of the HBM->LDS copies of stage st + NST - 1 (spread, not a burst).
    // Scale operands: a lane needs 8 bytes per stage, the four f16 block scales of its weight row and
    // of its token row. They are not staged through LDS: bounds-checked buffer loads bring them into
    // registers two stages ahead (the compiler cannot prove an LDS read unrelated to a pending LDS copy
    // and waits for the youngest copy before it; a scale read at each stage's publication drained the
    // whole copy pipeline). In a final half stage the loads read past the stage's two blocks into the
    // next row, or as zero past the buffer; those words are never used.
    const uint32_t msk_lo = g == 0 ? 0x0000ffffu : 0u, msk_hi = g == 0 ? 0xffff0000u : 0u;
    typedef unsigned int u2v __attribute__((ext_vector_type(2)));
    [[maybe_unused]] auto load_scales = [&](int64_t st, u2v (&ra)[TI], u2v (&rb)[TJ]) {
        const int64_t sa = st < nst ? st : nst - 1;
        const uint32_t kb0 = (uint32_t) (((sa + kst0) * KC) >> 5);
#pragma unroll
        for (int i = 0; i < TI; i++)
            ra[i] = __builtin_amdgcn_raw_buffer_load_b64(rAd, ((uint32_t) (32 * (wn * TI + i) + l32) * (uint32_t) KB + kb0) * 2, 0, 0);
#pragma unroll
        for (int j = 0; j < TJ; j++)
            rb[j] = __builtin_amdgcn_raw_buffer_load_b64(rBd, (tok_row(32 * (wm * TJ + j) + l32) * (uint32_t) KB + kb0) * 2, 0, 0);
    };
    // the weight row's four block scales fill K-slots 0-3 (both lane groups); the token's scale of
    // block blk alone fills K-slot blk of lane group 0 (group 1 is zero)
    auto q32_scales = [&](const u2v (&ra)[TI], const u2v (&rb)[TJ], h4 (&sa)[TI], h4 (&sb)[4][TJ]) {
#pragma unroll
        for (int i = 0; i < TI; i++) sa[i] = __builtin_bit_cast(h4, ra[i]);
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const uint2 w = make_uint2(rb[j].x, rb[j].y);
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const uint32_t msk = (blk & 1) ? msk_hi : msk_lo;
                const uint2 o = blk < 2 ? make_uint2(w.x & msk, 0u) : make_uint2(0u, w.y & msk);
                sb[blk][j] = __builtin_bit_cast(h4, o);
            }
        }
    };
    // Residual epilogue (int8 and 4-bit weights): the rows it adds to are loaded during the last K
    // stage, so that their latency hides under that stage's MFMAs instead of following them (rows
    // past M read row M - 1; their results are dropped). Not for 4-tile waves: no registers left.
    constexpr bool RPF = EPI == EPI_RESID && (WF == W_Q32 || WF == W_Q40 || WF == W_Q4K) && TI * TJ < 4;
    [[maybe_unused]] float4 xres[RPF ? TI : 1][RPF ? TJ : 1][4];
    [[maybe_unused]] auto prefetch_resid = [&]() {
        if constexpr (RPF) {
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int64_t m = m0 + 32 * (wm * TJ + j) + l32, mm = m < M ? m : M - 1;
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        xres[i][j][q] = *(const float4 *) (a.ep.y + mm * a.ep.ldy + n0 + 32 * (wn * TI + i) + 8 * q + 4 * g);
            }
        }
    };
    [[maybe_unused]] auto q32_main = [&](int64_t nfull) {
      if constexpr (WF == W_Q32 || WF == W_Q40) {
        constexpr int TT = TI * TJ, U = 4 * TT;
        static_assert(NST >= 3, "the in-stage barrier needs a stage in flight beyond the next one");
        // copies of this wave still allowed in flight at the barrier that publishes stage st+1 (held
        // in stage st at step U-2): the NST-3 stages after st+1, plus those of stage st+NST-1 that
        // steps 0..U-2 of stage st have issued
        // per stage every wave issues the PARTS copies of one stage, spread over the steps of a body
        // (step u issues copies [u PARTS / U, (u+1) PARTS / U))
        constexpr int P1 = T::PARTS;
        // copies issued after the last copy of stage st+1 when stage st publishes it (step U-2, after
        // that step's copies): the NST-3 stages after it, and this body's copies so far
        // Every body first issues its SLD scale loads (two stages ahead), then its copies. At the
        // publication of stage st+1, the loads issued after stage st+1's last copy are at least the
        // NST-3 bodies' copies in between, this body's scale loads and its copies up to step U-2
        // (exactly that for st = 1; later bodies add older scale loads, which only tightens the wait).
        constexpr int NBAR = (NST - 3) * P1 + T::SLD + (U - 1) * P1 / U;
        // q4_0 (W_Q40): 4-bit codes in HBM and LDS, read as one 16-byte chunk per two blocks (the q4_K
        // layout) and unpacked at the step's first MFMA into A[0]
        constexpr bool P4 = WF == W_Q40;
        i4v A[P4 ? 1 : 4][TI], B[4][TJ];
        [[maybe_unused]] u4v AR[2][TI];
        h4 SA[TI], SB[4][TJ];
        u2v RS0A[TI], RS0B[TJ], RS1A[TI], RS1B[TJ];   // raw scales: stage st+2 (being loaded), st+1
        i16v S[2];
        f16v C[2];
        // Tiles of at most two MFMA tiles per wave start the int8 MFMA from 0x4B400000, the bits of
        // 1.5 * 2^23: the int32 result M + S, read as a float, is exactly 12582912 + S for |S| < 2^22
        // (|S| <= 32 * 128 * 128 here), so one f32 subtraction gives float(S) exactly (measured ~7 %
        // faster than v_cvt_f32_i32). Larger wave tiles cannot spare the 16 VGPRs the constant takes
        // as an MFMA operand and convert with v_cvt_f32_i32.
        // q4_0 codes are 16 (q - 8) (the signed nibble in the high half of a byte), so the MFMA sums
        // 16 S; it starts from the bits of 1.5 * 2^19, where a float's unit in the last place is 1/16:
        // read as a float, M + 16 S is exactly 786432 + S (|S| <= 32 * 8 * 127). Without the constant
        // the accumulators take float(16 S) (exact: |16 S| < 2^24) and hold 16 times the sums, scaled
        // back once after the last stage: a power-of-two factor commutes with every rounding of the
        // fma chain (values far from the f32 subnormal range), so the result is the same bits.
        constexpr bool MAGIC = TI * TJ <= (P4 ? 3 : 2);   // (4-bit operands leave room for three)
        i16v magic;
#pragma unroll
        for (int r = 0; r < 16; r++) magic[r] = MAGIC ? (P4 ? 0x49400000 : 0x4B400000) : 0;
        float neg_magic;   // in a VGPR: a VALU op with an SGPR operand issues at half rate here
        if constexpr (P4) asm("v_mov_b32 %0, 0xc9400000" : "=v"(neg_magic));
        else asm("v_mov_b32 %0, 0xcb400000" : "=v"(neg_magic));
        auto ld_step = [&](const unsigned char * base, int u) {
            const int blk = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            if constexpr (P4) {
                if (j == 0 && (blk & 1) == 0) {
                    const int n = 32 * (wn * TI + i) + l32, r = n >> 1;
                    AR[blk >> 1][i] = *(const u4v *) (base + r * 128 + (lds_slot(r, ((n & 1) << 2) + 2 * (blk >> 1) + g) << 4));
                }
            } else {
                if (j == 0) A[blk][i] = lds_chunk<i4v>(base, 32 * (wn * TI + i) + l32, 2 * blk + g);
            }
            if (i == 0) B[blk][j] = lds_chunk<i4v>(base, T::AROWS + 32 * (wm * TJ + j) + l32, 2 * blk + g);
        };
        auto mma = [&](int u, const h4 (&sa)[TI], const h4 (&sb)[4][TJ]) {
            const int blk = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            if constexpr (P4) {
                if (j == 0) {
                    // byte b of each code dword holds codes b (low nibble) and b + 4 (high nibble)
                    const u4v ar = AR[blk >> 1][i];
                    const uint32_t p0 = (blk & 1) ? ar.z : ar.x, p1 = (blk & 1) ? ar.w : ar.y;
                    A[0][i] = i4v{(int) ((p0 << 4) & 0xF0F0F0F0u), (int) (p0 & 0xF0F0F0F0u), (int) ((p1 << 4) & 0xF0F0F0F0u),
                                  (int) (p1 & 0xF0F0F0F0u)};
                }
                if constexpr (MAGIC) S[u & 1] = MFMA_I8(A[0][i], B[blk][j], magic);
                else S[u & 1] = MFMA_I8(A[0][i], B[blk][j], i16v{});
            } else {
                if constexpr (MAGIC) S[u & 1] = MFMA_I8(A[blk][i], B[blk][j], magic);
                else S[u & 1] = MFMA_I8(A[blk][i], B[blk][j], i16v{});
            }
            C[u & 1] = MFMA8(sa[i], sb[blk][j], zero);
        };
        auto valu = [&](int u) {
            const int t = u % TT, i = t / TJ, j = t % TJ;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float sf = MAGIC ? __fadd_rn(__int_as_float(S[u & 1][r]), neg_magic) : (float) S[u & 1][r];
                acc[i][j][r] = fmaf(sf, C[u & 1][r], acc[i][j][r]);
            }
        };
        // prologue: only stage 0 is copied before the first barrier (the waves would otherwise stall
        // behind NST-1 stages of copies before any compute); stages 1..NST-1 follow spread over the
        // steps of stage 0. Copies are unconditional, so that every barrier count is exact: stages
        // past the end copy the last stage again into buffers no stage uses.
        load_scales(0, RS0A, RS0B);
        load_scales(1, RS1A, RS1B);
#pragma unroll
        for (int p = 0; p < T::PARTS; p++) issue_part(0, p);
        stage_barrier<0>();
        q32_scales(RS0A, RS0B, SA, SB);
        ld_step(smem, 0);
        ld_step(smem, 1);
        mma(0, SA, SB);
        __builtin_amdgcn_sched_barrier(0);
        // one full stage; CROSS: publish stage st+1 and start its pipeline in the last two steps;
        // FIRST (stage 0): issue the copies of stages 1..NST-1 instead of those of stage NST-1 alone
        auto body = [&](int64_t st, auto cross_c, auto first_c, auto extra_c) {
            constexpr bool CROSS = decltype(cross_c)::value, FIRST = decltype(first_c)::value;
            constexpr int Q = FIRST ? (NST - 1) * P1 : P1;          // copies this stage issues
            // copies younger than the last one of stage st+1 at its publication (step U-2); extra_c
            // counts those issued just before this body (the RoPE rows of the RE kernels)
            constexpr int NB = (FIRST ? (U - 1) * Q / U - P1 : NBAR) + decltype(extra_c)::value;
            static_assert(NB >= 0 && NB < 64, "barrier count");
            const unsigned char * base = smem + (int) (st % NST) * T::STAGE;
            const unsigned char * nbase = smem + (int) ((st + 1) % NST) * T::STAGE;
            h4 SAn[TI], SBn[4][TJ];
            if constexpr (CROSS) load_scales(st + 2, RS0A, RS0B);
#pragma unroll
            for (int u = 0; u < U; u++) {
#pragma unroll
                for (int k = u * Q / U; k < (u + 1) * Q / U; k++) {
                    if constexpr (FIRST) issue_part(1 + k / P1, k % P1);
                    else issue_part(st + NST - 1, k);
                }
                if (u + 2 < U) ld_step(base, u + 2);
                if constexpr (CROSS) {
                    if (u == U - 2) {
                        stage_barrier<NB>();
                        q32_scales(RS1A, RS1B, SAn, SBn);
                        ld_step(nbase, 0);
                    }
                    if (u == U - 1) ld_step(nbase, 1);
                }
                if (u + 1 < U) mma(u + 1, SA, SB);
                else if constexpr (CROSS) mma(0, SAn, SBn);
                valu(u);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (CROSS) {
#pragma unroll
                for (int i = 0; i < TI; i++) { SA[i] = SAn[i]; RS1A[i] = RS0A[i]; }
#pragma unroll
                for (int j = 0; j < TJ; j++) RS1B[j] = RS0B[j];
#pragma unroll
                for (int blk = 0; blk < 4; blk++)
#pragma unroll
                    for (int j = 0; j < TJ; j++) SB[blk][j] = SBn[blk][j];
            }
        };
        // stage 0 always publishes stage 1 (with a single full stage that is a copy of stage 0 into an
        // unused buffer, read and discarded)
        using X0 = std::integral_constant<int, 0>;
        if (nfull > 0) body(0, std::true_type{}, std::true_type{}, X0{});
        if constexpr (RE) {   // nfull == nst >= 3
            for (int64_t st = 1; st + 2 < nfull; st++) body(st, std::true_type{}, std::false_type{}, X0{});
            issue_rope_rows(rRc, nfull - 3);
            body(nfull - 2, std::true_type{}, std::false_type{}, std::integral_constant<int, RCH / NW>{});
            issue_rope_rows(rRs, nfull - 2);
            body(nfull - 1, std::false_type{}, std::false_type{}, X0{});
        } else {
            for (int64_t st = 1; st + 1 < nfull; st++) body(st, std::true_type{}, std::false_type{}, X0{});
            prefetch_resid();
            if (nfull > 1) body(nfull - 1, std::false_type{}, std::false_type{}, X0{});
        }
        // final half stage (K % 128 == 64): blocks 0 and 1 of stage nfull, after all copies landed
        if (nfull < nst) {
            stage_barrier<0>();
            const unsigned char * base = smem + (int) (nfull % NST) * T::STAGE;
            // its scales: loaded into RS1 by the body that published the last full stage, or, with
            // no full stage at all, by the prologue
            q32_scales(RS1A, RS1B, SA, SB);
#pragma unroll
            for (int u = 0; u < 2 * TT; u++) {
                ld_step(base, u);
                mma(u, SA, SB);
                valu(u);
            }
        }
        // the copies issued during the last stages must land before the workgroup's LDS is released
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
        if constexpr (P4 && !MAGIC) {
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = __fmul_rn(acc[i][j][r], 0.0625f);
        }
      }
    };

    // ---- q4_K ----
    // Weights stay 4-bit in HBM and LDS. A stage is 128 K-columns: 64 B of codes per weight row (two rows
    // share an LDS row) and 128 int8 q8_K codes per token; a super-block (256 K) is two stages. Steps
    // u = (sub-block jl of the stage, tile), tiles i-major, U = 4 TI TJ. Per sub-block the lane's 16
    // codes are unpacked from 8 bytes (and / shift) and multiplied, four bytes per v_pk_mul_lo_u16, by the
    // row's 6-bit scale split as sc = 8 sh + sl (sh, sl <= 7, so every byte product is <= 105 and no
    // carry crosses a byte): two int8 MFMAs then accumulate H += (sh q) . a and L += (sl q) . a over the
    // whole super-block in int32, the first sub-block starting from zero. At the end of the
    // super-block isum = 8 H + L is ggml's sum_j sc_j S_j exactly, and the epilogue (ggml's x86
    // vec_dot_q4_K_q8_K) does acc += (dw*da) isum, accm += (dmin*da) sum_j m_j bsum_j with the mins sum
    // from one f16 MFMA (exact); the result is acc - accm.
    // The pipeline is the q8_0 one: operand reads two steps ahead, copies spread over the steps of the
    // stage NST - 1 earlier, stage st+1 published two steps before the end of stage st. The super-block
    // data (not the same copy count on every wave) is left out of the barrier counts, which only makes
    // the waits longer; it is issued before the tile copies of the super-block's first stage, so it has
    // landed when that stage is published.
    [[maybe_unused]] auto q4k_main = [&]() {
      if constexpr (WF == W_Q4K) {
        constexpr int TT = TI * TJ, U = 4 * TT;
        static_assert(NST >= 3 && NST <= 4, "three to four stages: one in flight beyond the next, and the super-block buffers' reuse");
        constexpr int P1 = T::PARTS;
        constexpr int NBAR = (NST - 3) * P1 + (U - 1) * P1 / U;
        typedef unsigned int u2v __attribute__((ext_vector_type(2)));
        typedef unsigned short us2 __attribute__((ext_vector_type(2)));
        // operand registers by sub-block: with two or more MFMA tiles per wave, the reads two steps ahead
        // reach at most the next sub-block, so two sets suffice
        constexpr int NR = TT >= 2 ? 2 : 4, NP = TI == 1 ? 2 : 1;
        u4v AR[2][TI];            // raw 4-bit codes of sub-blocks jl, jl + 1 (jl even; 8 bytes each per lane)
        i4v B[NR][TJ];            // int8 activation codes of sub-block jl
        i4v AH[NP][TI], AL[NP][TI];   // sh * q and sl * q as int8
        u2v SCR[TI];              // the lane's weight row's eight sub-block scales (bytes)
        i16v HI[TI][TJ], LO[TI][TJ];
        auto xsb_of = [&](int64_t st) -> const unsigned char * { return smem + NST * T::STAGE + (int) ((st >> 1) % 3) * T::XSB; };
        // the row's sub-block scales of the super-block of stage st (read at the end of the stage
        // before; waited for at the start of stage st)
        auto ld_sc = [&](int64_t st) {
            const unsigned char * xb = xsb_of(st);
#pragma unroll
            for (int i = 0; i < TI; i++) SCR[i] = lds_read_asm<u2v>(xb + T::X_SC + 8 * (32 * (wn * TI + i) + l32));
        };
        auto take_sc = [&]() {
            lds_wait();
#pragma unroll
            for (int i = 0; i < TI; i++) lds_take(SCR[i]);
        };
        auto ld_step = [&](const unsigned char * base, int u) {
            const int jl = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            if (j == 0 && (jl & 1) == 0) {
                // a stage row's 64 B: [g0: jl 0, 1] [g1: jl 0, 1] [g0: jl 2, 3] [g1: jl 2, 3], 8 B each
                const int n = 32 * (wn * TI + i) + l32, r = n >> 1;
                // the 16 lanes of one ds_read_b128 pass (8 LDS rows, both halves of the 64 banks, chunks
                // c ^ ((r >> 1) & 7) with c in {c0, c0 + 4}) hit 16 different 4-bank groups
                AR[(jl >> 1) & 1][i] = *(const u4v *) (base + r * 128 + (lds_slot(r, ((n & 1) << 2) + 2 * (jl >> 1) + g) << 4));
            }
            if (i == 0) B[jl % NR][j] = lds_chunk<i4v>(base, T::AROWS + 32 * (wm * TJ + j) + l32, 2 * jl + g);
        };
        auto pk_mul = [](uint32_t c, uint32_t f) -> int {
            const us2 v = __builtin_bit_cast(us2, c) * (us2) {(unsigned short) f, (unsigned short) f};
            return __builtin_bit_cast(int, v);
        };
        auto mma = [&](int u, auto half_c) {
            constexpr int HALF = decltype(half_c)::value;
            const int jl = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            const int pb = jl % NP, rb = jl % NR;
            if (j == 0) {
                const uint32_t w = SCR[i][HALF];
                const uint32_t sh = (w >> (8 * jl + 3)) & 7u, sl = (w >> (8 * jl)) & 7u;
                const u4v ar = AR[(jl >> 1) & 1][i];
                const uint32_t p0 = (jl & 1) ? ar.z : ar.x, p1 = (jl & 1) ? ar.w : ar.y;
                const uint32_t c[4] = {p0 & 0x0F0F0F0Fu, (p0 >> 4) & 0x0F0F0F0Fu, p1 & 0x0F0F0F0Fu, (p1 >> 4) & 0x0F0F0F0Fu};
#pragma unroll
                for (int k = 0; k < 4; k++) { AH[pb][i][k] = pk_mul(c[k], sh); AL[pb][i][k] = pk_mul(c[k], sl); }
            }
            if (HALF == 0 && jl == 0) {
                HI[i][j] = MFMA_I8(AH[pb][i], B[rb][j], i16v{});
                LO[i][j] = MFMA_I8(AL[pb][i], B[rb][j], i16v{});
            } else {
                HI[i][j] = MFMA_I8(AH[pb][i], B[rb][j], HI[i][j]);
                LO[i][j] = MFMA_I8(AL[pb][i], B[rb][j], LO[i][j]);
            }
        };
        auto sb_epilogue = [&](int64_t st) {
            const unsigned char * xb = xsb_of(st);
            u4v bsr[TJ];
            uint32_t dar[TJ];
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int rm = 32 * (wm * TJ + j) + l32;
                bsr[j] = lds_read_asm<u4v>(xb + T::X_BS + rm * 32 + 16 * g);
                dar[j] = lds_read_asm<uint32_t>(xb + T::X_DA + 4 * rm);
            }
#pragma unroll
            for (int i = 0; i < TI; i++) {
                const int rn = 32 * (wn * TI + i);
                u4v amr = lds_read_asm<u4v>(xb + T::X_MIN + (rn + l32) * 32 + 16 * g);
                u4v dwr[4];   // rows 8q + 4g + e of the MFMA tile: (d, dmin) of four consecutive rows
#pragma unroll
                for (int q = 0; q < 4; q++) dwr[q] = lds_read_asm<u4v>(xb + T::X_DW + 4 * (rn + 8 * q + 4 * g));
                lds_wait();
                lds_take(amr);
#pragma unroll
                for (int q = 0; q < 4; q++) lds_take(dwr[q]);
                if (i == 0) {
#pragma unroll
                    for (int j = 0; j < TJ; j++) { lds_take(bsr[j]); lds_take(dar[j]); }
                }
                const h8 am = __builtin_bit_cast(h8, amr);
                f16v ms[TJ];
#pragma unroll
                for (int j = 0; j < TJ; j++) ms[j] = MFMA16(am, __builtin_bit_cast(h8, bsr[j]), zero);
                float da[TJ];
#pragma unroll
                for (int j = 0; j < TJ; j++) da[j] = __uint_as_float(dar[j]);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u4v v = dwr[q];
                    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float dw = h2f((uint16_t) (vv[e] & 0xffffu)), dm = h2f((uint16_t) (vv[e] >> 16));
                        const int r = 4 * q + e;
#pragma unroll
                        for (int j = 0; j < TJ; j++) {
                            const int isum = (HI[i][j][r] << 3) + LO[i][j][r];
                            const float d1 = __fmul_rn(dw, da[j]), d2 = __fmul_rn(dm, da[j]);
                            acc[i][j][r] = fmaf(d1, (float) isum, acc[i][j][r]);
                            accm[i][j][r] = fmaf(d2, ms[j][r], accm[i][j][r]);
                        }
                    }
                }
            }
        };
        issue_xsb(0);
#pragma unroll
        for (int p = 0; p < P1; p++) issue_part(0, p);
        stage_barrier<0>();
        ld_sc(0);
        ld_step(smem, 0);
        ld_step(smem, 1);
        __builtin_amdgcn_sched_barrier(0);
        auto body = [&](int64_t st, auto cross_c, auto first_c, auto half_c) {
            constexpr bool CROSS = decltype(cross_c)::value, FIRST = decltype(first_c)::value;
            constexpr int HALF = decltype(half_c)::value;
            constexpr int Q = FIRST ? (NST - 1) * P1 : P1;
            constexpr int NB = FIRST ? (U - 1) * Q / U - P1 : NBAR;
            static_assert(NB >= 0 && NB < 64, "barrier count");
            const unsigned char * base = smem + (int) (st % NST) * T::STAGE;
            const unsigned char * nbase = smem + (int) ((st + 1) % NST) * T::STAGE;
            if constexpr (FIRST) {
                // super-block data of the stages 1..NST-1 this body copies, before their tile copies
#pragma unroll
                for (int s2 = 2; s2 < NST; s2 += 2) issue_xsb(s2);
            }
            if constexpr (HALF == 0) take_sc();
#pragma unroll
            for (int u = 0; u < U; u++) {
                if constexpr (!FIRST) {
                    if (u == 0) issue_xsb(st + NST - 1);
                }
#pragma unroll
                for (int k = u * Q / U; k < (u + 1) * Q / U; k++) {
                    if constexpr (FIRST) issue_part(1 + k / P1, k % P1);
                    else issue_part(st + NST - 1, k);
                }
                mma(u, half_c);
                if (u + 2 < U) ld_step(base, u + 2);
                if constexpr (CROSS) {
                    if (u == U - 2) {
                        stage_barrier<NB>();
                        ld_step(nbase, 0);
                    }
                    if (u == U - 1) {
                        if constexpr (HALF == 1) ld_sc(st + 1);   // after this stage's last use of SCR
                        ld_step(nbase, 1);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (HALF == 1) sb_epilogue(st);
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        using H0 = std::integral_constant<int, 0>;
        using H1 = std::integral_constant<int, 1>;
        // nst is even (K % 256 == 0; a split has whole super-blocks per half)
        body(0, T_{}, T_{}, H0{});
        for (int64_t st = 1; st + 2 < nst; st += 2) {
            body(st, T_{}, F_{}, H1{});
            body(st + 1, T_{}, F_{}, H0{});
        }
        prefetch_resid();
        body(nst - 1, F_{}, F_{}, H1{});
        // the copies issued during the last stages must land before the workgroup's LDS is released
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
      }
    };

    // ---- f16 ----
    // A stage holds 64 K-columns (two 32-deep halves); steps u = (half, tile), tiles i-major, two f16
    // MFMAs (32x32x16) per step, U = 2 TI TJ per stage. The same pipeline as q8_0 / q4_0: operand
    // chunks two steps ahead, copies spread over the steps of the stage NST - 1 earlier (stage 0's
    // alone before the first barrier), stage st+1 published two steps before the end of stage st.
    constexpr bool PIPE16 = WF == W_F16;
    [[maybe_unused]] auto f16_main = [&]() {
      if constexpr (PIPE16) {
        constexpr int TT = TI * TJ, U = 2 * TT;
        static_assert(NST >= 3, "the in-stage barrier needs a stage in flight beyond the next one");
        constexpr int P1 = T::PARTS;
        constexpr int NBAR = (NST - 3) * P1 + (U - 1) * P1 / U;
        h8 A0[2][TI], A1[2][TI], B0[2][TJ], B1[2][TJ];
        auto ld_step = [&](const unsigned char * base, int u) {
            const int blk = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            if (j == 0) {
                const int r = 32 * (wn * TI + i) + l32;
                A0[blk][i] = lds_chunk<h8>(base, r, 4 * blk + g);
                A1[blk][i] = lds_chunk<h8>(base, r, 4 * blk + 2 + g);
            }
            if (i == 0) {
                const int r = BN + 32 * (wm * TJ + j) + l32;
                B0[blk][j] = lds_chunk<h8>(base, r, 4 * blk + g);
                B1[blk][j] = lds_chunk<h8>(base, r, 4 * blk + 2 + g);
            }
        };
        auto mma = [&](int u) {
            const int blk = u / TT, t = u % TT, i = t / TJ, j = t % TJ;
            acc[i][j] = MFMA16(A0[blk][i], B0[blk][j], acc[i][j]);
            acc[i][j] = MFMA16(A1[blk][i], B1[blk][j], acc[i][j]);
        };
#pragma unroll
        for (int p = 0; p < P1; p++) issue_part(0, p);
        stage_barrier<0>();
        ld_step(smem, 0);
        if (U > 1) ld_step(smem, 1);
        __builtin_amdgcn_sched_barrier(0);
        auto body = [&](int64_t st, auto cross_c, auto first_c) {
            constexpr bool CROSS = decltype(cross_c)::value, FIRST = decltype(first_c)::value;
            constexpr int Q = FIRST ? (NST - 1) * P1 : P1;
            constexpr int NB = FIRST ? (U - 1) * Q / U - P1 : NBAR;
            static_assert(NB >= 0 && NB < 64, "barrier count");
            const unsigned char * base = smem + (int) (st % NST) * T::STAGE;
            const unsigned char * nbase = smem + (int) ((st + 1) % NST) * T::STAGE;
#pragma unroll
            for (int u = 0; u < U; u++) {
#pragma unroll
                for (int k = u * Q / U; k < (u + 1) * Q / U; k++) {
                    if constexpr (FIRST) issue_part(1 + k / P1, k % P1);
                    else issue_part(st + NST - 1, k);
                }
                // the MFMAs of this step come first: with one tile per wave the next stage's first
                // operands go to the registers this step reads
                mma(u);
                if (u + 2 < U) ld_step(base, u + 2);
                if constexpr (CROSS) {
                    if (u == U - 2) {
                        stage_barrier<NB>();
                        ld_step(nbase, 0);
                    }
                    if (u == U - 1) ld_step(nbase, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (nst > 0) body(0, std::true_type{}, std::true_type{});
        for (int64_t st = 1; st + 1 < nst; st++) body(st, std::true_type{}, std::false_type{});
        if (nst > 1) body(nst - 1, std::false_type{}, std::false_type{});
        // the copies issued during the last stages must land before the workgroup's LDS is released
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
      }
    };

    // q8_0 / q4_0 with K % 128 == 64 end in a half stage, peeled off the loop so that the loop body
    // has one path (the accumulators then stay in place across iterations)
    const int64_t nfull = WF == W_Q32 || WF == W_Q40 ? (split > 1 ? nst : K / KC) : nst;
    if constexpr (WF == W_Q32 || WF == W_Q40) {
        q32_main(nfull);
    } else if constexpr (WF == W_Q4K) {
        q4k_main();
    } else if constexpr (PIPE16) {
        f16_main();
    } else {
    // f16 weights whose tile leaves room for fewer than three stages: one barrier per stage
    for (int s = 0; s < NST - 1; s++)
        if (s < nst) issue(s);

    // stage st has landed once at most the loads of the NST - 2 younger stages are outstanding (all
    // waves' copies of stage st visible; every wave done reading stage st-1's buffer)
    auto stage_begin = [&](int64_t st) -> const unsigned char * {
        if (st + NST - 2 < nst) stage_barrier<(NST - 2) * T::PARTS>();
        else stage_barrier<0>();
        if (st + NST - 1 < nst) issue(st + NST - 1);
        return smem + (int) (st % NST) * T::STAGE;
    };
    for (int64_t st = 0; st < nfull; st++) {
        const unsigned char * base = stage_begin(st);
#pragma unroll
        for (int blk = 0; blk < 2; blk++) {
            h8 a0[TI], a1[TI], b0[TJ], b1[TJ];
#pragma unroll
            for (int i = 0; i < TI; i++) {
                const int r = 32 * (wn * TI + i) + l32;
                a0[i] = lds_chunk<h8>(base, r, 4 * blk + g);
                a1[i] = lds_chunk<h8>(base, r, 4 * blk + 2 + g);
            }
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int r = BN + 32 * (wm * TJ + j) + l32;
                b0[j] = lds_chunk<h8>(base, r, 4 * blk + g);
                b1[j] = lds_chunk<h8>(base, r, 4 * blk + 2 + g);
            }
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++) {
                    acc[i][j] = MFMA16(a0[i], b0[j], acc[i][j]);
                    acc[i][j] = MFMA16(a1[i], b1[j], acc[i][j]);
                }
        }
    }
    }

    if constexpr (WF == W_Q4K) {
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = __fsub_rn(acc[i][j][r], accm[i][j][r]);
    }

    if constexpr (SPLITTABLE) {
        if (split > 1) {
            // Publish this part's accumulators; of the `split` workgroups of a tile, the last to arrive
            // adds all parts in split order, p0 + p1 + ... + p(split-1) (its own from registers), and runs
            // the epilogue; the others leave. The result does not depend on the arrival order, and
            // nothing waits on another workgroup.
            // The partials bypass the XCD-private L2s (cache policy sc1, what agent-scope atomic loads
            // and stores use), so no L2 write-back or invalidation is needed: once this wave's stores
            // have completed (vmcnt(0)) they are visible to every XCD, and the arrival counter is an
            // agent-coherent atomic.
            constexpr int TT = TI * TJ, SC1 = 16, SMAX = WF == W_F16 ? 4 : 2;   // parts: f16 up to 4, else halves
            const int64_t tile_floats = (int64_t) BN * T::BM;
            const brsrc rall = make_brsrc(a.part, (int64_t) split * ntile * tile_floats * 4);
            auto part_off = [&](int k, int t, int q) {   // byte offset of this lane's 4 floats of part k
                return (uint32_t) ((((int64_t) k * ntile + bid) * tile_floats) * 4 + ((t * 4 + q) * T::NT + tid) * 16);
            };
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f16v & v = acc[t / TJ][t % TJ];
                    const u4v b = {__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                                   __float_as_uint(v[4 * q + 3])};
                    __builtin_amdgcn_raw_buffer_store_b128(b, rall, part_off(sp, t, q), 0, SC1);
                }
            __builtin_amdgcn_s_waitcnt(0x0f70);    // vmcnt(0): this wave's partial has been written
            __syncthreads();
            int * flag = (int *) smem;              // the stage buffers are free (all copies landed)
            if (tid == 0) flag[0] = atomicAdd(a.cnt + bid, 1);
            __syncthreads();
            if (flag[0] != split - 1) return;       // not the last part to arrive
            if (tid == 0) __hip_atomic_store(a.cnt + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // ready for the next launch
            // v[4q..4q+3] = p0 + p1 + ... in split order, with part k's values in o[k] (sp's own: v)
            auto add_parts = [&](f16v & v, int q, const auto & o) {
                const float4 mine = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
                float4 sum = mine;
#pragma unroll
                for (int k = 0; k < SMAX; k++) {
                    if (k >= split) break;
                    const float4 x = k == sp ? mine : make_float4(__uint_as_float(o[k].x), __uint_as_float(o[k].y),
                                                                  __uint_as_float(o[k].z), __uint_as_float(o[k].w));
                    if (k == 0) sum = x;
                    else {
                        sum.x = __fadd_rn(sum.x, x.x); sum.y = __fadd_rn(sum.y, x.y);
                        sum.z = __fadd_rn(sum.z, x.z); sum.w = __fadd_rn(sum.w, x.w);
                    }
                }
                v[4 * q] = sum.x; v[4 * q + 1] = sum.y; v[4 * q + 2] = sum.z; v[4 * q + 3] = sum.w;
            };
#pragma unroll
            for (int t = 0; t < TT; t++) {
                f16v & v = acc[t / TJ][t % TJ];
                if constexpr (WF == W_F16) {
                    // the other parts' values of the whole 32x32 tile in flight at once (one memory
                    // round trip per tile; the f16 tiles that split, one MFMA tile per wave, have the
                    // registers)
                    u4v o[4][SMAX];
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int k = 0; k < SMAX; k++)
                            if (k < split && k != sp) o[q][k] = __builtin_amdgcn_raw_buffer_load_b128(rall, part_off(k, t, q), 0, SC1);
#pragma unroll
                    for (int q = 0; q < 4; q++) add_parts(v, q, o[q]);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        u4v o[SMAX];
#pragma unroll
                        for (int k = 0; k < SMAX; k++)
                            if (k < split && k != sp) o[k] = __builtin_amdgcn_raw_buffer_load_b128(rall, part_off(k, t, q), 0, SC1);
                        add_parts(v, q, o);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);   // one tile's loads in flight at a time (registers)
            }
        }
    }

    // The bias values of the wave's features and, in the QKV epilogue, the RoPE table rows of the
    // workgroup's tokens are fetched for all tiles before the first output store: a load issued after
    // a store cannot be moved ahead of it, so loads made inside the tile loops each waited one memory
    // round trip. The RoPE rows (head widths 32 and 64) are copied HBM->LDS into the stage buffers,
    // which the main loop no longer needs, by buffer copies of whole rows (the rows of consecutive
    // tokens are contiguous), and read per lane from LDS; gathering them per lane from the tables (a
    // 16-byte piece of 32 different rows per load) cost ~4 us of the ViT-L QKV GEMM's 31. 16-byte
    // chunk c of row r sits in slot c ^ (r mod chunks per row), so the 32 tokens of one LDS read fall
    // on different banks. Rows past M copy row M - 1 (their results are dropped). RE kernels have
    // copied them during the main loop's last two stages (ViT-L 16f q8_0 QKV 0.686 -> 0.672 ms per
    // clip; without any RoPE rows it would take 0.609).
    [[maybe_unused]] const unsigned char * lrc = nullptr;
    [[maybe_unused]] const unsigned char * lrs = nullptr;
    [[maybe_unused]] bool rope_late = false;
    if constexpr (EPI == EPI_QKV) {
        const int hd = a.ep.hd;
        if constexpr (RE) {
            // copied by the main loop before its last two stages; every wave has waited for its own
            // copies (vmcnt(0) at the loop's end), the barrier makes all of them visible
            if (n0 + a.ep.col0 < 2 * (int64_t) a.ep.D) {
                __syncthreads();
                lrc = smem + (int) ((nst - 3) % NST) * T::STAGE;
                lrs = smem + (int) ((nst - 2) % NST) * T::STAGE;
            }
        } else if (a.ep.rope_c && (hd == 32 || hd == 64) && n0 + a.ep.col0 < 2 * (int64_t) a.ep.D && 2 * T::BM * hd * 4 <= T::LDS) {
            rope_late = true;
            __builtin_amdgcn_s_waitcnt(0);      // no HBM->LDS copy of this wave still in flight
            __syncthreads();                    // every wave is past its last read of the stage buffers
            unsigned char * wc = smem;
            unsigned char * ws = smem + T::BM * hd * 4;
            const int cpr = hd / 4;                             // 16-byte chunks per row
            const int rpi = 64 / cpr;                           // rows per 1 KB copy
            const int64_t rows_tab = (int64_t) a.ep.R;          // table rows
            const brsrc tc = make_brsrc(a.ep.rope_c, rows_tab * hd * 4);
            const brsrc tsn = make_brsrc(a.ep.rope_s, rows_tab * hd * 4);
            const int r_l = lane / cpr, slot = lane - r_l * cpr;
            for (int k = wave; k < T::BM / rpi; k += NW) {      // 1 KB copies, dealt to the waves
                const int r = k * rpi + r_l;
                const int64_t m = m0 + r, mm = m < M ? m : M - 1;
                const uint32_t off = (uint32_t) ((mm % rows_tab) * hd * 4 + ((slot ^ (r & (cpr - 1))) << 4));
                dma_to_lds<16>(tc, off, 0, wc + k * 1024);
                dma_to_lds<16>(tsn, off, 0, ws + k * 1024);
            }
            lrc = wc; lrs = ws;
        }
    }
    constexpr bool BPRE = true;
    [[maybe_unused]] float4 bpre[BPRE ? TI : 1][4];
    if constexpr (BPRE) {
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                bpre[i][q] = a.bias ? *(const float4 *) (a.bias + n0 + 32 * (wn * TI + i) + 8 * q + 4 * g)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if constexpr (EPI == EPI_QKV) {
        if (rope_late) {
            __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0): this wave's row copies (and bias loads) have landed
            __syncthreads();
        }
    }

    if constexpr (EPI == EPI_GELU_Q8_K) {
        // q8_K activation of the next linear (quantize_row_q8_K_ref): per token and 256 features,
        // max = the first value of largest |x|, iscale = -127/max, q = min(127, rne(iscale*x)),
        // d = 1/iscale, bsums of 16. A workgroup row of WN waves covers one 256-block: each wave
        // reduces its 64 features (lane pair l, l^32), then the WN partial results of every token
        // meet in LDS. A wave's first element of its own largest magnitude is the block's first one
        // of that magnitude whenever the wave holds the block maximum, so one exchange of
        // (max, key = 2*index + sign) per wave suffices.
        static_assert(BN == 256, "one q8_K block per workgroup row of waves");
        float * xmax = (float *) smem;                                        // [TJ][WM*32][WN]
        uint32_t * xkey = (uint32_t *) (smem + TJ * WM * 32 * WN * 4);
        // no HBM->LDS copy of this wave is still in flight (the pipelines' tail copies land in stage
        // buffers), and every wave is past its last read of the stage buffers
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const int64_t m = m0 + 32 * (wm * TJ + j) + l32;
            float v[TI][16];
            float am = 0.0f;
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 b = bpre[i][q];
                    const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v[i][4 * q + e] = gelu_erf(__fadd_rn(acc[i][j][4 * q + e], bb[e]));
                        am = fmaxf(am, fabsf(v[i][4 * q + e]));
                    }
                }
            am = halves_max(am);
            uint32_t key = 0xffffffffu;
#pragma unroll
            for (int i = TI - 1; i >= 0; i--)
#pragma unroll
                for (int r = 15; r >= 0; r--)
                    if (fabsf(v[i][r]) == am)
                        key = 2u * (uint32_t) (32 * (wn * TI + i) + 8 * (r >> 2) + 4 * g + (r & 3)) + (__float_as_uint(v[i][r]) >> 31);
            key = halves_min_u32(key);
            const int slot = ((j * WM + wm) * 32 + l32) * WN;
            if (g == 0) { xmax[slot + wn] = am; xkey[slot + wn] = key; }
            __syncthreads();
            float bmax = xmax[slot];
            uint32_t bkey = xkey[slot];
#pragma unroll
            for (int w = 1; w < WN; w++) {
                const float a2 = xmax[slot + w];
                const uint32_t k2 = xkey[slot + w];
                if (a2 > bmax) { bmax = a2; bkey = k2; }
                else if (a2 == bmax) bkey = min(bkey, k2);
            }
            const float mx = (bkey & 1u) ? -bmax : bmax;
            const float iscale = bmax != 0.0f ? -127.0f / mx : 0.0f;
            float bs[TI][2];
#pragma unroll
            for (int i = 0; i < TI; i++) {
                bs[i][0] = bs[i][1] = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    v[i][r] = fminf(rintf(iscale * v[i][r]), 127.0f);
                    bs[i][r >> 3] += v[i][r];
                }
                bs[i][0] = halves_sum(bs[i][0]);   // features 16h..16h+15 of the tile: q = 2h, 2h+1 of both lane groups
                bs[i][1] = halves_sum(bs[i][1]);
            }
            if (m < M) {
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const int64_t nb = n0 + 32 * (wn * TI + i);
                    int8_t * o = (int8_t *) a.ep.oh + m * a.N + nb + 4 * g;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        uint32_t w = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) w |= ((uint32_t) (int) v[i][4 * q + e] & 0xffu) << (8 * e);
                        *(uint32_t *) (o + 8 * q) = w;   // int8 codes
                    }
                    if (g == 0) {
                        _Float16 * ob = (_Float16 *) a.ep.ob + m * (a.N / 16) + nb / 16;
                        ob[0] = (_Float16) bs[i][0];
                        ob[1] = (_Float16) bs[i][1];
                    }
                }
                if (wn == 0 && g == 0) ((float *) a.ep.od)[m * (a.N / 256) + n0 / 256] = bmax != 0.0f ? 1.0f / iscale : 0.0f;
            }
        }
        return;
    }

    // epilogue: lane holds token m and features nb + 8q + 4g + e of each tile
#pragma unroll
    for (int i = 0; i < TI; i++) {
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const int64_t m = m0 + 32 * (wm * TJ + j) + l32;
            const int64_t nb = n0 + 32 * (wn * TI + i);
            if constexpr (EPI == EPI_GELU_Q8_0) {
                // q8_0 activation of the next linear, x86 rule: d = amax/127 (f16), q = rne(x*127/amax)
                float v[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 b = bpre[i][q];
                    v[4 * q + 0] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 0], b.x));
                    v[4 * q + 1] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 1], b.y));
                    v[4 * q + 2] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 2], b.z));
                    v[4 * q + 3] = gelu_erf(__fadd_rn(acc[i][j][4 * q + 3], b.w));
                }
                float am = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(v[r]));
                am = halves_max(am);
                const float d = am / 127.0f;
                const float id = am != 0.0f ? 127.0f / am : 0.0f;
                if (m < M) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int64_t n = nb + 8 * q + 4 * g;
                        uint32_t o = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            o |= q8_byte(v[4 * q + e], id) << (8 * e);
                        }
                        *(uint32_t *) ((int8_t *) a.ep.oq + m * a.N + n) = o;   // int8 codes
                    }
                    if (g == 0) ((uint16_t *) a.ep.od)[m * (a.N / 32) + nb / 32] = f2hbits(d);
                }
            } else if constexpr (EPI == EPI_QKV) {
                if (a.ep.hd & 31) {
                    // head widths that are not a multiple of 32 (80 = I-JEPA ViT-H): a tile's 32 features
                    // can span two heads, so head and offset are found per group of four features
                    if (m >= M) continue;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float t[4] = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                        epi4<EPI_QKV>(a, m, nb + 8 * q + 4 * g, t);
                    }
                    continue;
                }
                // the tile's 32 features lie in one head of one of Q, K, V (D and hd are multiples of 32):
                // head and offset are wave-uniform, the token is one 32-bit division per lane
                const gemm_epi & ep = a.ep;
                const int hd = ep.hd, hds = ep.hds ? ep.hds : hd;
                const int nbi = __builtin_amdgcn_readfirstlane((int) (nb + ep.col0));
                const int which = nbi / ep.D, nn = nbi - which * ep.D;
                const int h = nn / hd, dbase = nn - h * hd + 4 * g;
                if (m >= M) continue;
                const uint32_t mu = (uint32_t) m, Ru = (uint32_t) ep.R;
                const uint32_t item = mu / Ru, tok = mu - item * Ru;
                const int64_t head = (int64_t) item * ep.n_head + h;
                float t[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 b = bpre[i][q];
                    const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) t[4 * q + e] = a.bias ? __fadd_rn(acc[i][j][4 * q + e], bb[e]) : acc[i][j][4 * q + e];
                }
                if (which < 2) {
                    _Float16 * dst = (_Float16 *) (which == 0 ? ep.q : ep.k) + (head * ep.R_pad + tok) * hds + dbase;
                    float4 c4[4], s4[4];
                    if (ep.rope_c) {
                        const int lr = 32 * (wm * TJ + j) + l32;      // the token's row of the workgroup
                        const int cpr = hd / 4;
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            if (lrc) {
                                const int off = lr * hd * 4 + ((((dbase + 8 * q) >> 2) ^ (lr & (cpr - 1))) << 4);
                                c4[q] = *(const float4 *) (lrc + off);
                                s4[q] = *(const float4 *) (lrs + off);
                            } else {
                                c4[q] = *(const float4 *) (ep.rope_c + (int64_t) tok * hd + dbase + 8 * q);
                                s4[q] = *(const float4 *) (ep.rope_s + (int64_t) tok * hd + dbase + 8 * q);
                            }
                        }
                    }
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float o[4] = {t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]};
                        if (ep.rope_c) {
                            // out = x*C + swap(x)*S' (reference src/rope3d.cpp:136-164): two products, one add
                            const float4 c = c4[q], sn = s4[q];
                            o[0] = __fadd_rn(__fmul_rn(t[4 * q + 0], c.x), __fmul_rn(t[4 * q + 1], sn.x));
                            o[1] = __fadd_rn(__fmul_rn(t[4 * q + 1], c.y), __fmul_rn(t[4 * q + 0], sn.y));
                            o[2] = __fadd_rn(__fmul_rn(t[4 * q + 2], c.z), __fmul_rn(t[4 * q + 3], sn.z));
                            o[3] = __fadd_rn(__fmul_rn(t[4 * q + 3], c.w), __fmul_rn(t[4 * q + 2], sn.w));
                        }
                        h4 v = {(_Float16) o[0], (_Float16) o[1], (_Float16) o[2], (_Float16) o[3]};
                        *(h4 *) (dst + 8 * q) = v;
                    }
                } else {
                    _Float16 * vt = (_Float16 *) ep.vt + (head * hds + dbase) * ep.R_pad + perm16(tok);
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int e = 0; e < 4; e++) vt[(int64_t) (8 * q + e) * ep.R_pad] = (_Float16) t[4 * q + e];
                }
            } else {
                if (m >= M) continue;
                // every load of the tile's four groups (residual rows, layer scale, modality vector,
                // position rows) before its first store
                const gemm_epi & ep = a.ep;
                const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                float4 o1[4], o2[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int64_t n = nb + 8 * q + 4 * g;
                    o1[q] = z4; o2[q] = z4;
                    if constexpr (EPI == EPI_RESID) {
                        if constexpr (!RPF) o1[q] = *(const float4 *) (ep.y + m * ep.ldy + n);
                        if (ep.ls) o2[q] = *(const float4 *) (ep.ls + n);
                    } else if constexpr (EPI == EPI_F32) {
                        if (ep.addvec) o1[q] = *(const float4 *) (ep.addvec + n);
                        if (ep.addrows) {
                            const int64_t item = m / ep.rin, rr = m - item * ep.rin;
                            o2[q] = *(const float4 *) (ep.addrows + (ep.pre + rr) * ep.ldy + n);
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int64_t n = nb + 8 * q + 4 * g;
                    float t[4] = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    if constexpr (EPI == EPI_RESID) {
                        if constexpr (RPF) resid4(a, m, n, t, xres[i][j][q], bpre[i][q], o2[q]);
                        else resid4(a, m, n, t, o1[q], bpre[i][q], o2[q]);
                    } else if constexpr (EPI == EPI_F32) {
                        f32out4(a, m, n, t, bpre[i][q], o1[q], o2[q]);
                    } else {
                        // GELU to f32 / f16: the bias is the only operand
                        const float4 b = bpre[i][q];
                        if (a.bias) { t[0] = __fadd_rn(t[0], b.x); t[1] = __fadd_rn(t[1], b.y); t[2] = __fadd_rn(t[2], b.z); t[3] = __fadd_rn(t[3], b.w); }
                        kargs nb_a = a;
                        nb_a.bias = nullptr;
                        epi4<EPI>(nb_a, m, n, t);
                    }
                }
            }
        }
    }
}

// f32 weights x f32 activations (hfvit patch embedding and f32 files): VALU FMA on tiles of 16 tokens x
// 32 features, so that even a one-image patch embedding (196 x 384 outputs) runs on 156 workgroups.
// A workgroup stages up to F32_KC columns of its 16 activation rows and 32 weight rows in LDS at once,
// row-major as loaded (16-byte stores; rows padded by 4 floats so that the rows one read touches fall
// on different banks), then each of its sixteen waves (four per SIMD, to hide the LDS and FMA
// latencies) sums one slice of those columns, four columns at a time: a lane holds 2 tokens x 4
// consecutive features, six 16-byte LDS reads per 32 FMAs. The partial sums meet in LDS and are added
// in wave order; a K longer than F32_KC runs several such
// chunks, each chunk's total added to the running sum.
constexpr int F32_KC = 768, F32_LD = F32_KC + 4;
constexpr int F32_NW = 16;                              // waves per workgroup, one K slice each
template <int EPI>
__global__ __launch_bounds__(64 * F32_NW) void k_gemm_f32(kargs a) {
    __shared__ __attribute__((aligned(16))) float sX[16][F32_LD];
    __shared__ __attribute__((aligned(16))) float sW[32][F32_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t) blockIdx.x * 32, m0 = (int64_t) blockIdx.y * 16;
    const float * W = (const float *) a.A;
    const float * X = (const float *) a.B;
    const int tg = lane >> 3, fg = lane & 7;            // tokens 2 tg, 2 tg + 1; features 4 fg .. 4 fg + 3
    const bool al = (a.K & 3) == 0 && (((uintptr_t) X | (uintptr_t) W) & 15) == 0;   // rows 16-byte aligned
    float tot[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    float * red = &sW[0][0];                            // [F32_NW - 1][64][8] partials of waves 1.. (reuses sW)
    // one 4-column piece of row r of a (rows past `rows`, columns past kc read as 0)
    auto piece = [&](const float * base, int64_t row, int64_t rows, int64_t k0, int kk, int kc) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (row < rows) {
            const float * src = base + row * a.K + k0 + kk;
            if (kk + 4 <= kc && al) v = *(const float4 *) src;
            else { v.x = src[0]; if (kk + 1 < kc) v.y = src[1]; if (kk + 2 < kc) v.z = src[2]; if (kk + 3 < kc) v.w = src[3]; }
        }
        return v;
    };
    for (int64_t k0 = 0; k0 < a.K; k0 += F32_KC) {
        const int kc = (int) (a.K - k0 < F32_KC ? a.K - k0 : F32_KC);
        const int kc4 = (kc + 3) & ~3;                  // columns staged: kc rounded up to 4 (zeros past kc)
        __syncthreads();                                // the previous chunk's reads (and reduction) are done
        // every load is issued before the LDS stores (a store between two loads would hold the second
        // back: the compiler cannot tell the rows from LDS); 9 pieces per thread, one round trip
        constexpr int PT = 16 * (F32_KC / 4) / (64 * F32_NW);   // pieces per thread per 16 rows
        float4 v[3][PT];
#pragma unroll
        for (int b = 0; b < 3; b++)                     // rows 0-15 of X, then 0-15 and 16-31 of W
#pragma unroll
            for (int i = 0; i < PT; i++) {
                const int c = tid + 64 * F32_NW * i, r = c / (F32_KC / 4), kk = 4 * (c % (F32_KC / 4));
                v[b][i] = kk < kc ? (b == 0 ? piece(X, m0 + r, a.M, k0, kk, kc) : piece(W, n0 + 16 * (b - 1) + r, a.N, k0, kk, kc))
                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
        for (int b = 0; b < 3; b++)
#pragma unroll
            for (int i = 0; i < PT; i++) {
                const int c = tid + 64 * F32_NW * i, r = c / (F32_KC / 4), kk = 4 * (c % (F32_KC / 4));
                if (kk < kc) *(float4 *) (b == 0 ? &sX[r][kk] : &sW[16 * (b - 1) + r][kk]) = v[b][i];
            }
        __syncthreads();
        const int q = ((kc4 / 4 + F32_NW - 1) / F32_NW) * 4;   // columns per wave, a multiple of 4
        const int kb = wave * q, ke = kb + q < kc4 ? kb + q : kc4;
        float acc[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
        for (int k = kb; k < ke; k += 4) {
            const float4 x0 = *(const float4 *) &sX[2 * tg][k], x1 = *(const float4 *) &sX[2 * tg + 1][k];
            float4 w[4];
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = *(const float4 *) &sW[4 * fg + e][k];
            const float xa[2][4] = {{x0.x, x0.y, x0.z, x0.w}, {x1.x, x1.y, x1.z, x1.w}};
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float wv = j == 0 ? w[e].x : j == 1 ? w[e].y : j == 2 ? w[e].z : w[e].w;
                    acc[0][e] = fmaf(xa[0][j], wv, acc[0][e]);
                    acc[1][e] = fmaf(xa[1][j], wv, acc[1][e]);
                }
        }
        __syncthreads();                                // every wave is past its reads of sW
        if (wave > 0) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) red[((wave - 1) * 64 + lane) * 8 + 4 * i + e] = acc[i][e];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = acc[i][e];
                    for (int w = 0; w < F32_NW - 1; w++) v = __fadd_rn(v, red[(w * 64 + lane) * 8 + 4 * i + e]);
                    tot[i][e] = k0 == 0 ? v : __fadd_rn(tot[i][e], v);
                }
        }
    }
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int64_t m = m0 + 2 * tg + i, n = n0 + 4 * fg;
            if (m < a.M && n < a.N) epi4<EPI>(a, m, n, tot[i]);
        }
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

struct tile_cfg { int wn, wm, ti, tj; };
// eight-wave workgroup tiles (BN x BM): 256x128, 192x128, 128x128 (two wave shapes), 64x128, 128x64,
// 256x64 (two wave shapes; the second, one weight tile and two token tiles per wave, only for the
// 256-feature q8_K epilogue)
constexpr tile_cfg k_tiles[] = {{4, 2, 2, 2}, {2, 4, 3, 1}, {2, 4, 2, 1}, {4, 2, 1, 2}, {2, 4, 1, 1}, {4, 2, 1, 1}, {4, 2, 2, 1},
                                {8, 1, 1, 2}, {4, 2, 3, 1}};
// relative efficiency of one workgroup tile (larger tiles re-read less from L2 and LDS)
constexpr double k_tile_eff[] = {1.0, 0.95, 0.85, 0.85, 0.65, 0.66, 0.8, 0.8, 0.9};

std::atomic<int> g_force_tile{-1};
std::atomic<int> g_force_split{-1};
constexpr int64_t SPLIT_MAX_N = 1024;

int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// 4-bit weights (q4_K, packed q4_0) run the tiles whose weight rows pair up into whole 1 KB copies (BN
// a multiple of 128); q4_K, whose four accumulator sets per MFMA tile must fit 256 VGPRs with two waves
// per SIMD, at most two MFMA tiles per wave. The 384x64 tile (for N = 3072: 256 tiles at M = 2048, the
// role the 192x128 tile has for int8 weights) fits three LDS stages only with 4-bit weights.
bool tile_ok(int wf, int c) {
    if (wf == W_Q4K) return c == 2 || c == 3 || c == 5 || c == 6 || c == 7;
    if (wf == W_Q40) return c != 1 && c != 4;
    return c != 8;
}

// The tile with the least estimated time: whole waves of workgroups over the CUs (one workgroup per
// CU) times the work of one tile, discounted by the tile's efficiency. Only tiles dividing N.
int pick_tile(int wf, int64_t N, int64_t M, int need_bn = 0, int split = 1) {
    const int f = g_force_tile.load();
    const int nt = (int) (sizeof(k_tiles) / sizeof(k_tiles[0]));
    const auto bn_of = [](int c) { return 32 * k_tiles[c].wn * k_tiles[c].ti; };
    if (f >= 0 && f < nt && N % bn_of(f) == 0 && (need_bn == 0 || bn_of(f) == need_bn) && tile_ok(wf, f) &&
        (f != 7 || need_bn == 256)) return f;
    const int cus = cu_count();
    double best = 1e300;
    int b = need_bn ? -1 : 5;
    for (int c = 0; c < nt; c++) {
        const int64_t bn = 32 * k_tiles[c].wn * k_tiles[c].ti, bm = 32 * k_tiles[c].wm * k_tiles[c].tj;
        if (N % bn || (need_bn && bn != need_bn) || (c == 7 && need_bn != 256)) continue;
        if (!tile_ok(wf, c)) continue;
        const int64_t t = (N / bn) * ((M + bm - 1) / bm) * split;
        const double waves = (double) ((t + cus - 1) / cus);
        // q4_K unpacks a wave's weight operand once for its TJ token tiles: tiles with two token tiles
        // per wave gain (ViT-L qkv, N 3072: 128x128 33.3 us against 36.7 us for three rounds of
        // 128x64), tiles with several weight tiles and one token tile lose
        double eff = k_tile_eff[c];
        if (wf == W_Q4K) eff *= k_tiles[c].tj >= 2 ? 1.1 : k_tiles[c].ti > 1 ? 0.8 : 1.0;
        const double cost = waves * (double) (bn * bm) / eff;
        if (cost < best) { best = cost; b = c; }
    }
    return b;
}

// k_gemm_mfma's arguments: the prologue's fields as scalars, then the whole kargs
#define GEMM_ARGS(a) (a).A, (a).B, (const void *) (a).Ad, (a).Bd, (int) (a).M, (int) (a).N, (int) (a).K, (a).tn, (a).tm, (a).split, (a)

// The QKV GEMM of q8_0 / q4_0 weights with heads of 64 runs the EPI_QKV_RE kernel (RoPE rows copied during the
// last two stages) wherever K is a whole number of at least three stages and the tile has four stage
// buffers of at least BM rows of 64 floats; elsewhere the rows are copied after the main loop.
template <int WF, int EPI, int WN, int WM, int TI, int TJ>
void launch_tile(const kargs & a, unsigned grid, hipStream_t s) {
    using T = tiling<WF, WN, WM, TI, TJ>;
    if constexpr (EPI == EPI_QKV && (WF == W_Q32 || WF == W_Q40) && (T::BM * 64 * 4 / 1024) % T::NW == 0 &&
                  T::BM * 64 * 4 <= T::STAGE && T::NST >= 4) {
        if (a.ep.rope_c && a.ep.rope_s && a.ep.hd == 64 && a.K % T::KC == 0 && a.K / T::KC >= 3) {
            k_gemm_mfma<WF, EPI_QKV_RE, WN, WM, TI, TJ><<<grid, T::NT, 0, s>>>(GEMM_ARGS(a));
            return;
        }
    }
    k_gemm_mfma<WF, EPI, WN, WM, TI, TJ><<<grid, T::NT, 0, s>>>(GEMM_ARGS(a));
}

template <int WF, int EPI>
void launch_tiles(int c, const kargs & a, hipStream_t s) {
    const unsigned grid = (unsigned) ((int64_t) a.tn * a.tm * (a.split > 1 ? a.split : 1));
    if constexpr (EPI == EPI_GELU_Q8_K) {   // 256-wide tiles only (pick_tile keeps to them)
        if (c == 6) launch_tile<WF, EPI, 4, 2, 2, 1>(a, grid, s);
        if (c == 7) launch_tile<WF, EPI, 8, 1, 1, 2>(a, grid, s);
        if constexpr (WF != W_Q4K)   // q4_K runs the 256x64 tile only
            if (c == 0) launch_tile<WF, EPI, 4, 2, 2, 2>(a, grid, s);
    } else if constexpr (WF == W_Q4K || WF == W_Q40) {
        switch (c) {
            case 0: if constexpr (WF == W_Q40) launch_tile<WF, EPI, 4, 2, 2, 2>(a, grid, s); break;
            case 8: if constexpr (WF == W_Q40) launch_tile<WF, EPI, 4, 2, 3, 1>(a, grid, s); break;
            case 2: launch_tile<WF, EPI, 2, 4, 2, 1>(a, grid, s); break;
            case 3: launch_tile<WF, EPI, 4, 2, 1, 2>(a, grid, s); break;
            case 5: launch_tile<WF, EPI, 4, 2, 1, 1>(a, grid, s); break;
            default: launch_tile<WF, EPI, 4, 2, 2, 1>(a, grid, s); break;
        }
    } else {
        switch (c) {
            case 0: launch_tile<WF, EPI, 4, 2, 2, 2>(a, grid, s); break;
            case 1: launch_tile<WF, EPI, 2, 4, 3, 1>(a, grid, s); break;
            case 2: launch_tile<WF, EPI, 2, 4, 2, 1>(a, grid, s); break;
            case 3: launch_tile<WF, EPI, 4, 2, 1, 2>(a, grid, s); break;
            case 4: launch_tile<WF, EPI, 2, 4, 1, 1>(a, grid, s); break;
            case 5: launch_tile<WF, EPI, 4, 2, 1, 1>(a, grid, s); break;
            default: launch_tile<WF, EPI, 4, 2, 2, 1>(a, grid, s); break;
        }
    }
}

// K parts of an f16-weight GEMM whose tiles leave most CUs idle (the residual GEMMs of a ViT-S/16 image:
// 197 tokens x 384 outputs are 12 tiles of 128x64, and fc2's K = 1536 is 24 stages per tile, copied at
// the ~80 GB/s one CU's copies sustain). Each of the S parts covers whole 64-column stages. Measured at
// 197 rows (us, S = 1 / 2 / 3 / 4): K 1536 12.4 / 10.6 / 9.7 / 9.4, K 3072 (N 768) 21.0 / 15.3 / 12.8 /
// 11.9, K 384 6.3 / 7.6 / 7.7 / -, K 768 (N 768) 8.4 / 8.8 / 8.6 / 8.8: the exchange (partial stores, the
// arrival atomic, the last part's loads) costs ~2 us, so only K >= 1024 (16 stages) splits, into the
// largest S of 4, 3, 2 that leaves each part 4 stages and each workgroup its own CU. The summation order
// then depends on the row count through the tile count (rounding-level differences between batch sizes,
// as f16 files have in the reference's batched image graph), so only the residual GEMMs of f16 blocks
// split by themselves, and only where the workspace allows it: the f16 patch embedding of a q8_0 /
// q4_K model keeps that model's items bit-identical across batch sizes, and so does every GEMM of a
// video workspace (the reference encodes each clip in a graph of its own, so n clips in one call must
// equal n one-clip calls exactly). The hook forces S for any splittable epilogue (1 = off).
int f16_split(int64_t K, int64_t tiles, int64_t tile_floats, const gemm_split_ws & sw, bool resid) {
    constexpr int KC16 = 64;
    if (K % KC16) return 1;
    const int64_t nst = K / KC16;
    const int cus = cu_count();
    const int f = g_force_split.load();
    if (f == 1 || (f < 1 && (!sw.f16_by_tiles || !resid || tiles * 2 > cus || nst < 16))) return 1;
    for (int S : {4, 3, 2}) {
        if (f >= 2 && S != f) continue;
        if (nst % S || nst / S < (f >= 2 ? 2 : 4) || tiles * S > cus || tiles * tile_floats * S > sw.part_floats ||
            tiles > sw.cnt_n) continue;
        return S;
    }
    return 1;
}

template <int WF>
void dispatch_mfma(kargs a, hipStream_t s, const gemm_split_ws * sw) {
    // split-K runs with the residual and plain epilogues (the N <= 1024 GEMMs of an encoder block)
    const bool can_split = sw && sw->part && sw->cnt && (a.ep.kind == EPI_RESID || a.ep.kind == EPI_F32);
    a.split = can_split && WF != W_F16 ? gemm_split_for(WF, a.N, a.K) : 1;
    a.part = nullptr; a.cnt = nullptr;
    const int c = pick_tile(WF, a.N, a.M, a.ep.kind == EPI_GELU_Q8_K ? 256 : 0, a.split);
    if (c < 0) {
        jepa_log("jepa: internal error: no 256-wide GEMM tile for the q8_K epilogue (N = %lld)\n", (long long) a.N);
        return;
    }
    const int bn = 32 * k_tiles[c].wn * k_tiles[c].ti, bm = 32 * k_tiles[c].wm * k_tiles[c].tj;
    a.tn = (int) (a.N / bn);
    a.tm = (int) ((a.M + bm - 1) / bm);
    if (WF == W_F16 && can_split) a.split = f16_split(a.K, (int64_t) a.tn * a.tm, (int64_t) bn * bm, *sw, a.ep.kind == EPI_RESID);
    if (a.split > 1) {
        const int64_t tiles = (int64_t) a.tn * a.tm;
        if (tiles * bn * bm * a.split > sw->part_floats || tiles > sw->cnt_n) {
            jepa_log("jepa: internal error: split-K scratch too small for %lld tiles\n", (long long) tiles);
            return;
        }
        a.part = sw->part; a.cnt = sw->cnt;
    }
    // XCD blocks: eight xa x xb blocks tiling the tn x tm grid, least rows per block
    a.xa = a.xb = 0;
    const int64_t ntile = (int64_t) a.tn * a.tm;
    if (ntile % 8 == 0) {
        const int64_t per = ntile / 8;
        int64_t best = -1;
        for (int xa = 1; xa <= a.tn; xa++) {
            if (a.tn % xa || per % xa || a.tm % (per / xa)) continue;
            const int64_t rows = (int64_t) xa * bn + (per / xa) * bm;
            if (best < 0 || rows < best) { best = rows; a.xa = xa; a.xb = (int) (per / xa); }
        }
    }
    switch (a.ep.kind) {
        case EPI_F32:       launch_tiles<WF, EPI_F32>(c, a, s); break;
        case EPI_RESID:     launch_tiles<WF, EPI_RESID>(c, a, s); break;
        case EPI_GELU_F32:  launch_tiles<WF, EPI_GELU_F32>(c, a, s); break;
        case EPI_GELU_F16:  launch_tiles<WF, EPI_GELU_F16>(c, a, s); break;
        case EPI_GELU_Q8_0: launch_tiles<WF, EPI_GELU_Q8_0>(c, a, s); break;
        case EPI_QKV:       launch_tiles<WF, EPI_QKV>(c, a, s); break;
        case EPI_GELU_Q8_K: launch_tiles<WF, EPI_GELU_Q8_K>(c, a, s); break;
    }
}

}  // namespace

int gemm_split_for(int wf, int64_t N, int64_t K) {
    // GEMMs with N <= 1024 cannot fill 256 CUs with tiles big enough to run well (2048 tokens x 1024
    // outputs is 64 tiles of 256x128); split-K gives each 128x128 tile two workgroups, one per K half
    // (each of whole 128-column stages; q4_K: each half starts at a super-block and spans whole
    // 4-stage super-blocks), at the cost of a partial-sum exchange (~2 us: the stores, the arrival
    // atomic, the partner's loads). By default it runs for q4_K from K = 2048 (ViT-L fc2: 41 -> 35 us);
    // the q8_0 / q4_0 fc2 runs as fast on the unsplit 128x64 tile (~39 us either way, with 20 MB less
    // HBM traffic), and neither pays at K = 1024 (out-proj: 12.8 -> 16.8 us). The hook forces either.
    if (!((wf == W_Q32 || wf == W_Q40) && K % 256 == 0) && !(wf == W_Q4K && K % 512 == 0)) return 1;
    const int f = g_force_split.load();
    if (f >= 1) return f >= 2 ? 2 : 1;
    return wf == W_Q4K && N <= SPLIT_MAX_N && K >= 2048 ? 2 : 1;
}

void gemm_split_ws_size(int64_t max_rows, int64_t * part_floats, int64_t * cnt_n) {
    // tiles x BN x BM <= (rows rounded up to 128) x N for every tile: two halves (int8 / 4-bit weights),
    // up to four parts for up to 1024 rows (f16 weights); tiles <= that / 64^2
    const int64_t rows = (max_rows + 127) / 128 * 128;
    *part_floats = (rows <= 1024 ? 4 : 2) * rows * SPLIT_MAX_N;
    *cnt_n = (rows / 64) * (SPLIT_MAX_N / 64) + 64;
}

void launch_gemm(const dev_linear & W, const act_view & X, int64_t M, const gemm_epi & ep, hipStream_t s, const gemm_split_ws * sw) {
    kargs a{};
    a.A = (const _Float16 *) W.w;
    a.Ad = (const uint16_t *) W.wd;
    a.Amin = (const _Float16 *) W.wmin;
    if (W.fmt == W_Q4K) a.Asc = (const uint8_t *) W.w + W.n_out * (W.n_in / 2);   // scales follow the codes
    a.B = (const _Float16 *) X.q;
    a.Bd = X.d;
    a.Bsum = (const _Float16 *) X.bsum;
    a.bias = W.bias;
    a.M = M; a.N = W.n_out; a.K = W.n_in;
    a.ep = ep;
    if (M <= 0) return;
    if (M > INT32_MAX || a.N > INT32_MAX || a.K > INT32_MAX) {   // k_gemm_mfma takes them as 32-bit scalars
        jepa_log("jepa: internal error: GEMM of %lld x %lld x %lld exceeds 32-bit sizes\n", (long long) M, (long long) a.N,
                 (long long) a.K);
        return;
    }
    if (a.ep.kind == EPI_F32 && a.ep.rin <= 0) { a.ep.rin = M; a.ep.rout = M; a.ep.pre = 0; }   // identity row map
    if (W.fmt == W_F32) {
        dim3 grid((unsigned) ((a.N + 31) / 32), (unsigned) ((M + 15) / 16));
        switch (ep.kind) {
            case EPI_F32:      k_gemm_f32<EPI_F32><<<grid, 64 * F32_NW, 0, s>>>(a); break;
            case EPI_RESID:    k_gemm_f32<EPI_RESID><<<grid, 64 * F32_NW, 0, s>>>(a); break;
            case EPI_GELU_F32: k_gemm_f32<EPI_GELU_F32><<<grid, 64 * F32_NW, 0, s>>>(a); break;
            case EPI_QKV:      k_gemm_f32<EPI_QKV><<<grid, 64 * F32_NW, 0, s>>>(a); break;
            default: jepa_log("jepa: internal error: epilogue %d has no f32 GEMM\n", ep.kind); break;
        }
        return;
    }
    switch (W.fmt) {
        case W_F16: dispatch_mfma<W_F16>(a, s, sw); break;
        case W_Q32: dispatch_mfma<W_Q32>(a, s, sw); break;
        case W_Q40: dispatch_mfma<W_Q40>(a, s, sw); break;
        case W_Q4K: dispatch_mfma<W_Q4K>(a, s, sw); break;
    }
}

int gemm_force_split(int split) {
    // int8 / 4-bit weights: 1 or 2 halves; f16 weights: 1 to 4 parts (f16_split)
    g_force_split.store(split < 1 ? -1 : split > 4 ? 4 : split);
    return 0;
}

int gemm_force_tile(int index) {
    if (index >= (int) (sizeof(k_tiles) / sizeof(k_tiles[0]))) return -1;
    g_force_tile.store(index < 0 ? -1 : index);
    return 0;
}

void launch_qkv_split(const float * qkv, int64_t M, int64_t N, const gemm_epi & ep, hipStream_t s) {
    kargs a{};
    a.M = M; a.N = N; a.K = 0;
    a.ep = ep;
    const int64_t total = M * (N / 4);
    if (total > 0) k_qkv_split<<<(unsigned) ((total + 255) / 256), 256, 0, s>>>(a, qkv);
}
