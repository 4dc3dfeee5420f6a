// misc.hip - bandwidth-bound kernels: LayerNorm + activation quantization, patchify, prefix rows,
// load-time weight repacking, and small test hooks.
#include "kernels.h"
#include "model.h"
#include "quant_dev.h"
#include "rownorm_dev.h"

#include <hip/hip_fp16.h>

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ float h2f(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }

// ------------------------------------------------------------------------------------------------
// Row kernel: one wave per row of D floats (LayerNorm and / or output conversion, rownorm_dev.h).
// ------------------------------------------------------------------------------------------------
using rowln::MAXOCT;

template <int OUT, bool NORM, int NOCT>
__global__ __launch_bounds__(256) void k_rownorm(const float * __restrict__ x, int64_t M, int64_t D,
                                                 const float * __restrict__ w, const float * __restrict__ b, float eps,
                                                 act_view out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    float v[NOCT][8];
    float gw[NOCT][8], gb[NOCT][8];   // affine parameters, loaded with x
    rowln::load_row<NOCT>(x + row * D, D, lane, v);
    if constexpr (NORM) rowln::load_affine<NOCT>(w, b, D, lane, gw, gb);
    rowln::finish_row<OUT, NORM, NOCT>(v, row, D, w != nullptr, b != nullptr, gw, gb, eps, out, lane);
}

// ------------------------------------------------------------------------------------------------
// patchify (reference src/jepa.cpp:476-504): token order t, h, w; inner order c, tt, py, px.
// One thread per 8 consecutive outputs of a patch row (P % 8 == 0): consecutive threads write
// consecutive 16- or 32-byte pieces of the output, and read 32 contiguous bytes of one image row.
// ------------------------------------------------------------------------------------------------
template <bool HALF>
__global__ void k_patchify(const float * __restrict__ in, void * __restrict__ rows, int64_t n_items, int C, int T, int H,
                           int W, int P, int tub, int video) {
    const int GT = video ? T / tub : 1, GH = H / P, GW = W / P;
    const int64_t Np = (int64_t) GT * GH * GW;
    const int64_t K = (int64_t) C * tub * P * P;
    const int per_row = P / 8;
    const int64_t total = n_items * Np * C * tub * P * per_row;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    int64_t r = id;
    const int px0 = 8 * (int) (r % per_row); r /= per_row;
    const int py = (int) (r % P); r /= P;
    const int tt = (int) (r % tub); r /= tub;
    const int c = (int) (r % C); r /= C;
    const int64_t tok = r % Np; const int64_t item = r / Np;
    const int t = (int) (tok / (GH * GW)), hh = (int) ((tok / GW) % GH), ww = (int) (tok % GW);
    int64_t b, f;
    if (video) { b = item; f = (int64_t) t * tub + tt; }
    else { b = item / T; f = item % T; }
    const float * src = in + (((b * C + c) * T + f) * H + (int64_t) hh * P + py) * W + (int64_t) ww * P + px0;
    const int64_t off = (item * Np + tok) * K + ((int64_t) (c * tub + tt) * P + py) * P + px0;
    // P % 8 == 0 (the launcher's choice) and W % P == 0 make src and the output 32-byte aligned
    const float4 lo = *(const float4 *) src, hi = *(const float4 *) (src + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    if (HALF) {
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (_Float16) v[e];
        *(h8 *) ((_Float16 *) rows + off) = o;
    } else {
        float * dst = (float *) rows + off;
        *(float4 *) dst = make_float4(v[0], v[1], v[2], v[3]);
        *(float4 *) (dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// patch sizes that are not a multiple of 8 (e.g. 14): one thread per patch row of P pixels
template <bool HALF>
__global__ void k_patchify_rows(const float * __restrict__ in, void * __restrict__ rows, int64_t n_items, int C, int T,
                                int H, int W, int P, int tub, int video) {
    const int GT = video ? T / tub : 1, GH = H / P, GW = W / P;
    const int64_t Np = (int64_t) GT * GH * GW;
    const int64_t K = (int64_t) C * tub * P * P;
    const int64_t total = n_items * Np * C * tub * P;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    int64_t r = id;
    const int py = (int) (r % P); r /= P;
    const int tt = (int) (r % tub); r /= tub;
    const int c = (int) (r % C); r /= C;
    const int64_t tok = r % Np; const int64_t item = r / Np;
    const int t = (int) (tok / (GH * GW)), hh = (int) ((tok / GW) % GH), ww = (int) (tok % GW);
    int64_t b, f;
    if (video) { b = item; f = (int64_t) t * tub + tt; }
    else { b = item / T; f = item % T; }
    const float * src = in + (((b * C + c) * T + f) * H + (int64_t) hh * P + py) * W + (int64_t) ww * P;
    const int64_t off = (item * Np + tok) * K + ((int64_t) (c * tub + tt) * P + py) * P;
    if (HALF) {
        _Float16 * dst = (_Float16 *) rows + off;
        for (int px = 0; px < P; px++) dst[px] = (_Float16) src[px];
    } else {
        float * dst = (float *) rows + off;
        for (int px = 0; px < P; px++) dst[px] = src[px];
    }
}

__global__ void k_cls_rows(float * x, const float * cls, const float * pos, int64_t n_items, int64_t R, int64_t D) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_items * D) return;
    const int64_t it = id / D, n = id % D;
    float v = cls[n];
    if (pos) v = __fadd_rn(v, pos[n]);
    x[it * R * D + n] = v;
}

// Prefix rows of every item, in front of its patch rows: the CLS row (when cls), then n_reg register
// rows, each plus its position row when pos is given (reference src/jepa.cpp:598-608: the registers
// and then the CLS row are concatenated in front, the position table is added to every row)
__global__ void k_prefix_rows(float * x, const float * cls, const float * reg, int n_reg, const float * pos, int64_t n_items,
                              int64_t R, int64_t D) {
    const int nc = cls ? 1 : 0, np = nc + n_reg;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_items * np * D) return;
    const int64_t it = id / (np * D), p = (id / D) % np, n = id % D;
    float v = p < nc ? cls[n] : reg[(p - nc) * D + n];
    if (pos) v = __fadd_rn(v, pos[p * D + n]);
    x[(it * R + p) * D + n] = v;
}

// ------------------------------------------------------------------------------------------------
// weight expansion at load (ggml blocks -> GEMM operand arrays)
// ------------------------------------------------------------------------------------------------
// q8_0 weights, and q4_0 rows not a multiple of 128 -> int8 codes [n_out][n_in] (q, or q - 8) + f16 d
// [n_out][n_in/32]
__global__ void k_repack_q8_0(const uint8_t * __restrict__ raw, int64_t n_out, int64_t n_in, int8_t * w, uint16_t * wd) {
    const int64_t nb = n_in / 32;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_out * nb) return;
    const uint8_t * blk = raw + id * 34;
    wd[id] = (uint16_t) (blk[0] | (blk[1] << 8));
    const int64_t n = id / nb, bi = id % nb;
    int8_t * dst = w + n * n_in + bi * 32;
    for (int j = 0; j < 32; j++) dst[j] = (int8_t) blk[2 + j];
}

__global__ void k_repack_q4_0(const uint8_t * __restrict__ raw, int64_t n_out, int64_t n_in, int8_t * w, uint16_t * wd) {
    const int64_t nb = n_in / 32;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_out * nb) return;
    const uint8_t * blk = raw + id * 18;
    wd[id] = (uint16_t) (blk[0] | (blk[1] << 8));
    const int64_t n = id / nb, bi = id % nb;
    int8_t * dst = w + n * n_in + bi * 32;
    for (int j = 0; j < 16; j++) {
        dst[j]      = (int8_t) ((blk[2 + j] & 0xF) - 8);
        dst[j + 16] = (int8_t) ((blk[2 + j] >> 4) - 8);
    }
}

// q4_0 rows that are a multiple of 128 stay 4-bit: codes [n_out][n_in/2] + f16 d [n_out][n_in/32]. Each
// code is q - 8 as a 4-bit two's complement (q ^ 8), so that a nibble moved to the high half of a byte
// is the int8 16 (q - 8). A block of 32 is two halves g of 16 values, each 8 bytes: two dwords whose
// byte b holds values b (low nibble) and b + 4 (high nibble) of its first and of its second eight
// values, so that (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0 are four consecutive codes each. The four
// blocks of each 128 values (64 B) lie as [g0: blocks 0, 1] [g1: blocks 0, 1] [g0: blocks 2, 3] [g1:
// blocks 2, 3], one 16-byte read per lane and two blocks. ggml's q4_0 block (the reference's ggml
// quantizer) is d, then 16 bytes whose low nibbles are values 0..15 and high nibbles values 16..31.
__global__ void k_repack_q4_0_packed(const uint8_t * __restrict__ raw, int64_t n_out, int64_t n_in, uint32_t * w, uint16_t * wd) {
    const int64_t nb = n_in / 32;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_out * nb) return;
    const uint8_t * blk = raw + id * 18;
    wd[id] = (uint16_t) (blk[0] | (blk[1] << 8));
    const int64_t n = id / nb, bi = id % nb;
    uint8_t v[32];
    for (int j = 0; j < 16; j++) {
        v[j] = (blk[2 + j] & 0xF) ^ 8;
        v[j + 16] = (blk[2 + j] >> 4) ^ 8;
    }
    // block bi of the row: 128-value group bi / 4, pair (bi % 4) / 2, 8-byte slot bi % 2 of each chunk
    uint32_t * row = w + n * (n_in / 8);
    const int64_t base = (bi / 4) * 16 + ((bi % 4) >> 1) * 8 + (bi & 1) * 2;   // dwords
    for (int g = 0; g < 2; g++)
        for (int dw = 0; dw < 2; dw++) {
            uint32_t x = 0;
            for (int b = 0; b < 4; b++) x |= (uint32_t) (v[16 * g + 8 * dw + b] | (v[16 * g + 8 * dw + 4 + b] << 4)) << (8 * b);
            row[base + 4 * g + dw] = x;
        }
}

__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t * q, int & d, int & m) {
    if (j < 4) { d = q[j] & 63; m = q[j + 4] & 63; }
    else { d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

// q4_K for the int8 GEMM, still 4 bits per weight: w [n_out][n_in/2] codes, then wsc [n_out][n_in/256][8]
// sub-block scales (6-bit, as bytes), wd (d | dmin << 16) [n_in/256][n_out], wmin [n_out][n_in/256][16]
// f16 mins (m_{k/2}, the operand of the mins MFMA). Codes: each 16-value half g of a 32-value sub-block
// is 8 bytes, two dwords whose byte b holds values b (low nibble) and b + 4 (high nibble) of its first
// and of its second eight values, so that (w & 0x0F0F0F0F) and ((w >> 4) & 0x0F0F0F0F) are four
// consecutive codes each, in the byte order of the activation codes. The four sub-blocks of each 128
// values (64 B) lie as [g0: sb 0, 1] [g1: sb 0, 1] [g0: sb 2, 3] [g1: sb 2, 3], so that one 16-byte read
// gives a lane two sub-blocks' halves.
__global__ void k_repack_q4_K(const uint8_t * __restrict__ raw, int64_t n_out, int64_t n_in, uint8_t * w, uint8_t * wsc,
                              uint32_t * wd, _Float16 * wmin) {
    const int64_t nsb = n_in / 256;
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n_out * nsb) return;
    const int64_t n = id / nsb, sb = id % nsb;
    const uint8_t * blk = raw + id * 144;
    // (d, dmin) of the super-block as one word: d in the low half, dmin in the high half
    wd[sb * n_out + n] = (uint32_t) blk[0] | ((uint32_t) blk[1] << 8) | ((uint32_t) blk[2] << 16) | ((uint32_t) blk[3] << 24);
    const uint8_t * sc = blk + 4;
    const uint8_t * qs = blk + 16;
    uint8_t * dst = w + n * (n_in / 2) + sb * 128;
    for (int j = 0; j < 8; j++) {
        int s, m;
        q4k_scale_min(j, sc, s, m);
        wsc[id * 8 + j] = (uint8_t) s;
        wmin[id * 16 + 2 * j] = (_Float16) (float) m;
        wmin[id * 16 + 2 * j + 1] = (_Float16) (float) m;
        const uint8_t * qq = qs + 32 * (j / 2);
        uint8_t q[32];
        for (int l = 0; l < 32; l++) q[l] = (j & 1) ? (qq[l] >> 4) : (qq[l] & 0xF);
        const int jl = j & 3;   // sub-block within its 128 values
        uint8_t * d128 = dst + 64 * (j >> 2);
        for (int h = 0; h < 2; h++)
            for (int dw = 0; dw < 2; dw++)
                for (int b = 0; b < 4; b++) {
                    const int v = 16 * h + 8 * dw + b;
                    d128[16 * (2 * (jl >> 1) + h) + 8 * (jl & 1) + 4 * dw + b] = (uint8_t) (q[v] | (q[v + 4] << 4));
                }
    }
}

// ggml to_float of the block types (test hook for bit-exact dequantization)
__global__ void k_dequant(int gtype, const uint8_t * __restrict__ raw, int64_t n_rows, int64_t n_cols, float * y) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = n_rows * n_cols;
    if (id >= total) return;
    const int64_t r = id / n_cols, c = id % n_cols;
    if (gtype == T_Q8_0) {
        const uint8_t * blk = raw + (r * (n_cols / 32) + c / 32) * 34;
        y[id] = __fmul_rn((float) (int8_t) blk[2 + c % 32], h2f((uint16_t) (blk[0] | (blk[1] << 8))));
    } else if (gtype == T_Q4_0) {
        const uint8_t * blk = raw + (r * (n_cols / 32) + c / 32) * 18;
        const int j = (int) (c % 32);
        const int q = j < 16 ? (blk[2 + j] & 0xF) : (blk[2 + j - 16] >> 4);
        y[id] = __fmul_rn((float) (q - 8), h2f((uint16_t) (blk[0] | (blk[1] << 8))));
    } else if (gtype == T_Q4_K) {
        const uint8_t * blk = raw + (r * (n_cols / 256) + c / 256) * 144;
        const int e = (int) (c % 256), j = e / 32, l = e % 32;
        int s, m;
        q4k_scale_min(j, blk + 4, s, m);
        const uint8_t qq = blk[16 + 32 * (j / 2) + l];
        const int q = (j & 1) ? (qq >> 4) : (qq & 0xF);
        const float d = h2f((uint16_t) (blk[0] | (blk[1] << 8))), dmin = h2f((uint16_t) (blk[2] | (blk[3] << 8)));
        y[id] = __fsub_rn(__fmul_rn(__fmul_rn(d, (float) s), (float) q), __fmul_rn(dmin, (float) m));
    } else if (gtype == T_F16) {
        y[id] = h2f(((const uint16_t *) raw)[id]);
    } else if (gtype == T_BF16) {
        y[id] = __uint_as_float((uint32_t) ((const uint16_t *) raw)[id] << 16);
    } else {
        y[id] = ((const float *) raw)[id];
    }
}

// activation operand (int8 codes + scales) -> ggml block bytes (q8_0: 34 B, q8_K: 292 B)
__global__ void k_pack_act(act_view a, int64_t M, int64_t K, uint8_t * out) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (a.fmt == A_Q8_0) {
        const int64_t nb = K / 32;
        if (id >= M * nb) return;
        const int64_t m = id / nb, bi = id % nb;
        uint8_t * o = out + id * 34;
        const uint16_t d = ((const uint16_t *) a.d)[m * nb + bi];
        o[0] = (uint8_t) (d & 0xFF); o[1] = (uint8_t) (d >> 8);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) ((const int8_t *) a.q)[m * K + bi * 32 + j];
    } else if (a.fmt == A_Q8_K) {
        const int64_t nb = K / 256;
        if (id >= M * nb) return;
        const int64_t m = id / nb, bi = id % nb;
        uint8_t * o = out + id * 292;
        const float d = ((const float *) a.d)[m * nb + bi];
        const uint32_t db = __builtin_bit_cast(uint32_t, d);
        for (int k = 0; k < 4; k++) o[k] = (uint8_t) (db >> (8 * k));
        for (int j = 0; j < 256; j++) o[4 + j] = (uint8_t) ((const int8_t *) a.q)[m * K + bi * 256 + j];
        for (int j = 0; j < 16; j++) {
            const int16_t s = (int16_t) (float) ((const _Float16 *) a.bsum)[m * (K / 16) + bi * 16 + j];
            o[260 + 2 * j] = (uint8_t) (s & 0xFF); o[261 + 2 * j] = (uint8_t) ((uint16_t) s >> 8);
        }
    }
}

__global__ void k_fill_zero(uint32_t * p, size_t n) {
    const size_t id = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (id < n) p[id] = 0;
}

__global__ void k_copy_f32(const float * __restrict__ src, float * __restrict__ dst, int64_t n) {
    const int64_t id = ((int64_t) blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (id + 3 < n) *(float4 *) (dst + id) = *(const float4 *) (src + id);
    else for (int64_t i = id; i < n; i++) dst[i] = src[i];
}

// D = A . B with one v_mfma_f32_32x32x16_f16, stored with the (row, col) <- (lane, reg) map the
// GEMM epilogues rely on: row = 8*(r/4) + 4*(lane/32) + r%4, col = lane%32.
__global__ void k_mfma_probe(const float * a, const float * b, float * d) {
    const int lane = threadIdx.x & 63, l32 = lane & 31, g = lane >> 5;
    h8 av, bv;
    for (int s = 0; s < 8; s++) {
        av[s] = (_Float16) a[l32 * 16 + 8 * g + s];      // A[i][k]
        bv[s] = (_Float16) b[(8 * g + s) * 32 + l32];    // B[k][j]
    }
    const f16v z = {0};
    const f16v r = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, z, 0, 0, 0);
    for (int k = 0; k < 16; k++) d[(8 * (k / 4) + 4 * g + (k % 4)) * 32 + l32] = r[k];
}

inline unsigned nblk(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }

}  // namespace

void launch_rownorm_quant(const float * x, int64_t M, int64_t D, const float * w, const float * b, float eps,
                          bool normalize, const act_view & out, hipStream_t s) {
    if (M <= 0) return;
    if (!normalize && D > 512) {
        // Plain conversion: quantization blocks (32 / 256 values) never straddle a chunk of c columns
        // when c is a multiple of 256 dividing D, and [M][D] is [M*D/c][c] in memory for the codes,
        // the scales and the block sums alike. Chunks of 512 (one octet per lane) give the most
        // waves and the shortest dependency chain per wave.
        int64_t c = 0;
        if (D % 512 == 0) c = 512;
        else
            for (int64_t t = 64 * 8 * MAXOCT; t >= 256 && c == 0; t -= 256)
                if (D % t == 0) c = t;
        if (c > 0) { M = M * (D / c); D = c; }
    }
    const dim3 grid(nblk(M, 4));
    const int noct = D <= 512 ? 1 : D <= 1024 ? 2 : 4;
#define RN3(OUT, NORM) (noct == 1 ? (void) k_rownorm<OUT, NORM, 1><<<grid, 256, 0, s>>>(x, M, D, w, b, eps, out) \
                      : noct == 2 ? (void) k_rownorm<OUT, NORM, 2><<<grid, 256, 0, s>>>(x, M, D, w, b, eps, out) \
                                  : (void) k_rownorm<OUT, NORM, 4><<<grid, 256, 0, s>>>(x, M, D, w, b, eps, out))
#define RN(OUT) (normalize ? RN3(OUT, true) : RN3(OUT, false))
    switch (out.fmt) {
        case A_F32:  RN(A_F32); break;
        case A_F16:  RN(A_F16); break;
        case A_Q8_0: RN(A_Q8_0); break;
        case A_Q8_K: RN(A_Q8_K); break;
    }
#undef RN3
#undef RN
}

void launch_patchify(const float * in, void * rows, bool half_out, int64_t n_items, int C, int T, int H, int W, int P,
                     int tub, bool video, hipStream_t s) {
    const int GT = video ? T / tub : 1;
    const int64_t total = n_items * (int64_t) GT * (H / P) * (W / P) * C * tub * P;   // patch rows
    const int v = video ? 1 : 0;
    if (P % 8 == 0) {
        const int64_t n = total * (P / 8);
        if (half_out) k_patchify<true><<<nblk(n, 256), 256, 0, s>>>(in, rows, n_items, C, T, H, W, P, tub, v);
        else k_patchify<false><<<nblk(n, 256), 256, 0, s>>>(in, rows, n_items, C, T, H, W, P, tub, v);
    } else {
        if (half_out) k_patchify_rows<true><<<nblk(total, 256), 256, 0, s>>>(in, rows, n_items, C, T, H, W, P, tub, v);
        else k_patchify_rows<false><<<nblk(total, 256), 256, 0, s>>>(in, rows, n_items, C, T, H, W, P, tub, v);
    }
}

void launch_prefix_rows(float * x, const float * cls, const float * reg, int n_reg, const float * pos, int64_t n_items, int64_t R,
                        int64_t D, hipStream_t s) {
    const int np = (cls ? 1 : 0) + n_reg;
    if (np > 0) k_prefix_rows<<<nblk(n_items * np * D, 256), 256, 0, s>>>(x, cls, reg, n_reg, pos, n_items, R, D);
}

void launch_cls_rows(float * x, const float * cls, const float * pos, int64_t n_items, int64_t R, int64_t D, hipStream_t s) {
    k_cls_rows<<<nblk(n_items * D, 256), 256, 0, s>>>(x, cls, pos, n_items, R, D);
}

void launch_repack(int gtype, const void * raw, int64_t n_out, int64_t n_in, void * w, void * wd, void * wmin,
                   hipStream_t s, bool int8) {
    switch (gtype) {
        case T_Q8_0: k_repack_q8_0<<<nblk(n_out * (n_in / 32), 256), 256, 0, s>>>((const uint8_t *) raw, n_out, n_in, (int8_t *) w, (uint16_t *) wd); break;
        case T_Q4_0:
            if (!int8 && weight_format(T_Q4_0, n_in) == W_Q40)
                k_repack_q4_0_packed<<<nblk(n_out * (n_in / 32), 256), 256, 0, s>>>((const uint8_t *) raw, n_out, n_in, (uint32_t *) w,
                                                                                   (uint16_t *) wd);
            else
                k_repack_q4_0<<<nblk(n_out * (n_in / 32), 256), 256, 0, s>>>((const uint8_t *) raw, n_out, n_in, (int8_t *) w, (uint16_t *) wd);
            break;
        case T_Q4_K: k_repack_q4_K<<<nblk(n_out * (n_in / 256), 256), 256, 0, s>>>((const uint8_t *) raw, n_out, n_in, (uint8_t *) w,
                                                                                  (uint8_t *) w + n_out * (n_in / 2), (uint32_t *) wd,
                                                                                  (_Float16 *) wmin); break;
        default: break;
    }
}

void launch_dequant_rows(int gtype, const void * raw, int64_t n_rows, int64_t n_cols, float * y, hipStream_t s) {
    k_dequant<<<nblk(n_rows * n_cols, 256), 256, 0, s>>>(gtype, (const uint8_t *) raw, n_rows, n_cols, y);
}

void launch_pack_act_blocks(const act_view & a, int64_t M, int64_t K, void * blocks, hipStream_t s) {
    const int64_t nb = a.fmt == A_Q8_K ? M * (K / 256) : M * (K / 32);
    k_pack_act<<<nblk(nb, 256), 256, 0, s>>>(a, M, K, (uint8_t *) blocks);
}

void launch_fill_zero(void * p, size_t bytes, hipStream_t s) {
    const size_t n = bytes / 4;
    if (n) k_fill_zero<<<nblk((int64_t) n, 256), 256, 0, s>>>((uint32_t *) p, n);
}

void launch_copy_f32(const float * src, float * dst, int64_t n, hipStream_t s) {
    k_copy_f32<<<nblk((n + 3) / 4, 256), 256, 0, s>>>(src, dst, n);
}

// ------------------------------------------------------------------------------------------------
// The throughput ceiling of the q8_0 GEMM's inner step, measured from registers alone (no memory, no
// barriers): per 32x32x32 block and MFMA tile, one v_mfma_i32_32x32x32_i8 (exact block sum S), one
// v_mfma_f32_32x32x8_f16 (scale products dw * da) and 32 VALU ops (16 conversions of S, 16 fmas into
// the f32 accumulators). mode 0: the whole step in every wave, the MFMAs of step u+1 issued before the
// VALU work of step u (the kernels' pipeline); 1: the two MFMAs alone; 2: the 32 VALU ops alone;
// 3: the step split over waves, even waves running the MFMA half and odd waves the VALU half (the
// bound if the matrix unit overlapped VALU work of other waves; the waves of a SIMD alternate by their
// slot on it). Each wave runs 2 * iters half or whole
// steps; `sink` keeps the results live.
// ------------------------------------------------------------------------------------------------
typedef int i4v_ __attribute__((ext_vector_type(4)));
typedef int i16v_ __attribute__((ext_vector_type(16)));
template <int MODE>
__global__ __launch_bounds__(1024) void k_step_probe(float * sink, int iters) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    i4v_ A0 = {lane, lane * 3, lane * 5, lane * 7}, B0 = {lane + 1, lane * 2, lane * 9, lane * 11};
    i4v_ A1 = A0 + 1, B1 = B0 + 2;
    h4 sa, sb;
    for (int i = 0; i < 4; i++) { sa[i] = (_Float16) (0.001f * (lane + i)); sb[i] = (_Float16) (0.002f * (lane - i)); }
    f16v acc = {}, C[2] = {};
    i16v_ S[2] = {}, iv = {};
    for (int r = 0; r < 16; r++) iv[r] = (lane + r) & 63;
    float y[16];
    for (int r = 0; r < 16; r++) y[r] = 1.0f + r * 1e-3f;
    // mode 3 pairs the waves of each SIMD by their slot on it (HW_ID bits 3:0), whatever order the
    // workgroup's waves were dealt to the SIMDs in
    (void) wave;
    const int slot = MODE == 3 ? (int) (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 4) & 15) : 0;
    const bool mfma_wave = MODE == 3 ? (slot & 1) == 0 : MODE != 2;
    const bool valu_wave = MODE == 3 ? (slot & 1) == 1 : MODE != 1;
    if (MODE == 0) { S[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B0, i16v_{}, 0, 0, 0); C[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa, sb, f16v{}, 0, 0, 0); }
    // one loop per role (a role branch inside the loop body serialises the MFMAs)
    if (MODE == 0) {
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                asm volatile("" : "+v"(A0), "+v"(B0), "+v"(A1), "+v"(B1), "+v"(sa), "+v"(sb));
                S[u ^ 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(u ? A0 : A1, u ? B0 : B1, i16v_{}, 0, 0, 0);
                C[u ^ 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa, sb, f16v{}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[r] = fmaf((float) S[u][r], C[u][r], acc[r]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else if (mfma_wave) {
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                asm volatile("" : "+v"(A0), "+v"(B0), "+v"(A1), "+v"(B1), "+v"(sa), "+v"(sb));
                S[u ^ 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(u ? A0 : A1, u ? B0 : B1, i16v_{}, 0, 0, 0);
                C[u ^ 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa, sb, f16v{}, 0, 0, 0);
                asm volatile("" :: "v"(S[u]), "v"(C[u]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else if (valu_wave) {
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                asm volatile("" : "+v"(iv));
#pragma unroll
                for (int r = 0; r < 16; r++) acc[r] = fmaf((float) iv[r], y[r], acc[r]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    float t = 0.0f;
    for (int r = 0; r < 16; r++) t += acc[r] + (float) S[0][r] + C[0][r];
    sink[(size_t) blockIdx.x * blockDim.x + threadIdx.x] = t;
}

void launch_step_probe(int mode, int waves_per_simd, int iters, int n_wg, float * sink, hipStream_t s) {
    const dim3 block((unsigned) (256 * waves_per_simd));
    switch (mode) {
        case 0: k_step_probe<0><<<n_wg, block, 0, s>>>(sink, iters); break;
        case 1: k_step_probe<1><<<n_wg, block, 0, s>>>(sink, iters); break;
        case 2: k_step_probe<2><<<n_wg, block, 0, s>>>(sink, iters); break;
        default: k_step_probe<3><<<n_wg, block, 0, s>>>(sink, iters); break;
    }
}

void launch_mfma_probe(const float * a, const float * b, float * d, hipStream_t s) {
    k_mfma_probe<<<1, 64, 0, s>>>(a, b, d);
}
