// attention.hip - flash attention forward for head_dim 64 on gfx950 (f16 MFMA, f32 softmax).
//
// Computes softmax(Q K^T * scale) V per (item, head): the ggml_flash_attn_ext of reference
// src/jepa.cpp:416-442 (no mask, K/V in f16 as the reference's ggml_cast does, f32 softmax and f32
// accumulation). Q arrives with 3-D RoPE already applied by the QKV GEMM epilogue.
//
// Work split: one workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries and
// sweeps all keys in tiles of 64 (K and V^T tiles staged in LDS, shared by the 4 waves).
// MFMA roles are chosen so that softmax statistics need no cross-lane reduction beyond one
// xor-32 exchange:
//   S^T[key][q] = K . Q^T     A = K tile rows (keys), B = Q^T (held in registers for the sweep)
//                             -> lane (q = lane%32) holds 16 keys of its query column
//   O^T[d][q]  += V^T . P^T   A = V^T tile rows (d), B = P^T built in place from the S registers
// The B operand of the PV MFMA takes the 8 keys (4g..4g+3, 8+4g..8+4g+3 of each 16) that the S
// accumulator layout leaves in lane group g; V^T is stored with the same key order inside every
// 16-token group (written that way by the QKV epilogue), so both operands agree without shuffles.
#include "kernels.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

namespace {

constexpr int HD = 64, QB = 128, KT = 64, LDK = 72;

__global__ __launch_bounds__(256) void k_attn_hd64(const _Float16 * __restrict__ Q, const _Float16 * __restrict__ Kp,
                                                   const _Float16 * __restrict__ Vt, float * __restrict__ O,
                                                   int n_head, int64_t R, int64_t R_pad, float c) {
    __shared__ __attribute__((aligned(16))) _Float16 sK[KT * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 sV[HD * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int64_t head = blockIdx.y;
    const int64_t item = head / n_head;
    const int h = (int) (head - item * n_head);
    const int64_t q0 = (int64_t) blockIdx.x * QB + wave * 32;

    const _Float16 * Qh = Q + head * R_pad * HD;
    const _Float16 * Kh = Kp + head * R_pad * HD;
    const _Float16 * Vh = Vt + head * HD * R_pad;

    h8 qv[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) qv[kk] = *(const h8 *) (Qh + (q0 + l32) * HD + 16 * kk + 8 * g);

    const f16v zero = {0};
    f16v acc0 = zero, acc1 = zero;
    float m_run = -INFINITY, l_run = 0.0f;
    const int64_t kend = (R + KT - 1) / KT * KT;

    for (int64_t kt = 0; kt < kend; kt += KT) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int cidx = tid + 256 * i, row = cidx >> 3, col = (cidx & 7) * 8;
            *(uint4 *) &sK[row * LDK + col] = *(const uint4 *) (Kh + (kt + row) * HD + col);
            *(uint4 *) &sV[row * LDK + col] = *(const uint4 *) (Vh + (int64_t) row * R_pad + kt + col);
        }
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            f16v S = zero;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const h8 a = *(const h8 *) &sK[(32 * kb + l32) * LDK + 16 * kk + 8 * g];
                S = MFMA16(a, qv[kk], S);
            }
            const int64_t key0 = kt + 32 * kb + 4 * g;
            if (kt + 32 * kb + 32 > R) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (key0 + 8 * (r >> 2) + (r & 3) >= R) S[r] = -INFINITY;
            }
            float mloc = S[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, S[r]);
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = exp2f((m_run - m_new) * c);
            const float mc = m_new * c;
            float p[16], lsum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) { p[r] = exp2f(fmaf(S[r], c, -mc)); lsum += p[r]; }
            lsum += __shfl_xor(lsum, 32);
            l_run = fmaf(l_run, alpha, lsum);
            m_run = m_new;
            if (alpha != 1.0f) {
#pragma unroll
                for (int r = 0; r < 16; r++) { acc0[r] *= alpha; acc1[r] *= alpha; }
            }
#pragma unroll
            for (int kk2 = 0; kk2 < 2; kk2++) {
                h8 pb;
#pragma unroll
                for (int s = 0; s < 8; s++) pb[s] = (_Float16) p[8 * kk2 + s];
                const h8 a0 = *(const h8 *) &sV[(l32) * LDK + 32 * kb + 16 * kk2 + 8 * g];
                const h8 a1 = *(const h8 *) &sV[(32 + l32) * LDK + 32 * kb + 16 * kk2 + 8 * g];
                acc0 = MFMA16(a0, pb, acc0);
                acc1 = MFMA16(a1, pb, acc1);
            }
        }
    }
    const int64_t q = q0 + l32;
    if (q >= R) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float * orow = O + (item * R + q) * (int64_t) (n_head * HD) + h * HD;
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
        const int d = 8 * qq + 4 * g;
        *(float4 *) (orow + d) = make_float4(acc0[4 * qq] * inv, acc0[4 * qq + 1] * inv, acc0[4 * qq + 2] * inv, acc0[4 * qq + 3] * inv);
        *(float4 *) (orow + 32 + d) = make_float4(acc1[4 * qq] * inv, acc1[4 * qq + 1] * inv, acc1[4 * qq + 2] * inv, acc1[4 * qq + 3] * inv);
    }
}

}  // namespace

void launch_attention(const void * q, const void * k, const void * vt, float * o, int64_t n_items, int n_head,
                      int hd, int64_t R, int64_t R_pad, float scale, hipStream_t s) {
    (void) hd;   // only 64 (checked by the caller)
    const float c = scale * 1.4426950408889634f;   // exp(x*scale) = exp2(x*scale*log2(e))
    dim3 grid((unsigned) ((R + QB - 1) / QB), (unsigned) (n_items * n_head));
    k_attn_hd64<<<grid, 256, 0, s>>>((const _Float16 *) q, (const _Float16 *) k, (const _Float16 *) vt, o, n_head, R, R_pad, c);
}
