// pool.hip - the single-query cross-attention of the attentive-pool head on gfx950.
//
// Reference src/jepa.cpp:1047-1063: one learned query per head attends to all N encoder tokens,
// o_h = softmax(q_h . K_h^T * scale) V_h, with K and V kept in f32 (the CPU graph's kv_type), and
// the pooled token is y = o + q0 (the raw query; there is no output projection).
// One query makes this a bandwidth problem over K and V (2 * N * D * 4 bytes), not an MFMA one:
//   pass 1: grid (chunks of 256 keys) x heads; a thread scores one key (64-wide dot product with the
//           query held in LDS), the workgroup forms the chunk's max m, p = exp(s - m), l = sum p, and
//           the four waves accumulate P V with lane = output dimension (each V row read coalesced);
//           (m, l, acc[64]) of the chunk go to `part`;
//   pass 2: one wave per head merges its chunks (flash-decoding rescale by exp(m_c - M)), divides by
//           the total weight and adds q0.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int HD = 64, CH = 256;   // head width, keys per chunk (= threads per workgroup)
constexpr int PART = HD + 2;       // floats per (head, chunk) record: m, l, acc[64]

__device__ __forceinline__ float wave_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__global__ __launch_bounds__(CH) void k_pool_part(const float * __restrict__ q, const float * __restrict__ K,
                                                  const float * __restrict__ V, int64_t N, int64_t ld, float scale, int S,
                                                  float * __restrict__ part) {
    const int c = (int) blockIdx.x, h = (int) blockIdx.y, tid = (int) threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ float sq[HD], sp[CH], sred[2][4], sacc[4][HD];
    if (tid < HD) sq[tid] = q[(int64_t) h * HD + tid];
    __syncthreads();
    const int64_t t0 = (int64_t) c * CH;
    const int nc = (int) min<int64_t>(CH, N - t0);
    float s = -INFINITY;
    if (tid < nc) {
        const float4 * kr = (const float4 *) (K + (t0 + tid) * ld + (int64_t) h * HD);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 4; i++) {
            const float4 k4 = kr[i];
            a += k4.x * sq[4 * i];
            a += k4.y * sq[4 * i + 1];
            a += k4.z * sq[4 * i + 2];
            a += k4.w * sq[4 * i + 3];
        }
        s = a * scale;
    }
    float m = wave_max(s);
    if (lane == 0) sred[0][wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sred[0][0], sred[0][1]), fmaxf(sred[0][2], sred[0][3]));   // finite: nc >= 1
    const float p = tid < nc ? __expf(s - m) : 0.0f;
    sp[tid] = p;
    const float lw = wave_sum(p);
    if (lane == 0) sred[1][wv] = lw;
    __syncthreads();
    // P V: lane = output dimension, wave wv takes keys wv, wv + 4, ...
    const float * vc = V + t0 * ld + (int64_t) h * HD + lane;
    float acc = 0.0f;
    for (int j = wv; j < nc; j += 4) acc += sp[j] * vc[(int64_t) j * ld];
    sacc[wv][lane] = acc;
    __syncthreads();
    if (tid < HD) {
        float * o = part + ((int64_t) h * S + c) * PART;
        o[2 + tid] = (sacc[0][tid] + sacc[1][tid]) + (sacc[2][tid] + sacc[3][tid]);
        if (tid == 0) {
            o[0] = m;
            o[1] = (sred[1][0] + sred[1][1]) + (sred[1][2] + sred[1][3]);
        }
    }
}

__global__ __launch_bounds__(HD) void k_pool_combine(const float * __restrict__ part, int S, const float * __restrict__ q0,
                                                     float * __restrict__ y) {
    const int h = (int) blockIdx.x, d = (int) threadIdx.x;
    const float * p = part + (int64_t) h * S * PART;
    float M = -INFINITY;
    for (int c = 0; c < S; c++) M = fmaxf(M, p[(int64_t) c * PART]);
    float L = 0.0f, o = 0.0f;
    for (int c = 0; c < S; c++) {
        const float w = __expf(p[(int64_t) c * PART] - M);
        L += p[(int64_t) c * PART + 1] * w;
        o += p[(int64_t) c * PART + 2 + d] * w;
    }
    y[(int64_t) h * HD + d] = o / L + q0[(int64_t) h * HD + d];
}

}  // namespace

int64_t pool_attention_part_floats(int64_t N, int n_head) { return (int64_t) n_head * ((N + CH - 1) / CH) * PART; }

bool launch_pool_attention(const float * q, const float * K, const float * V, int64_t N, int64_t ld, int n_head, int hd, float scale,
                           const float * q0, float * y, float * part, int64_t part_floats, hipStream_t s) {
    if (hd != HD || N <= 0 || n_head <= 0 || ld % 4 != 0 || ld < (int64_t) n_head * HD ||
        ((uintptr_t) K | (uintptr_t) V) % 16 != 0 || part_floats < pool_attention_part_floats(N, n_head) ||
        (N + CH - 1) / CH > INT32_MAX || n_head > 65535) {
        jepa_log("jepa: pool attention: unsupported shape (N %lld, heads %d, head_dim %d, ld %lld)\n", (long long) N, n_head, hd,
                 (long long) ld);
        return false;
    }
    const int S = (int) ((N + CH - 1) / CH);
    k_pool_part<<<dim3(S, n_head), CH, 0, s>>>(q, K, V, N, ld, scale, S, part);
    k_pool_combine<<<n_head, HD, 0, s>>>(part, S, q0, y);
    return true;
}
