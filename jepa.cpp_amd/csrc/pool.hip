// pool.hip - the single-query cross-attention of the attentive-pool head on gfx950.
//
// Reference src/jepa.cpp:1047-1063: one learned query per head attends to all N encoder tokens,
// o_h = softmax(q_h . K_h^T * scale) V_h, with K and V kept in f32 (the CPU graph's kv_type), and
// the pooled token is y = o + q0 (the raw query; there is no output projection).
// One query makes this a bandwidth problem over K and V (2 * N * D * 4 bytes), not an MFMA one:
//   pass 1: grid (chunks of 64 keys) x heads, 256 threads. Scores: four threads per key, each a
//           16-wide slice of the dot product (one coalesced 256-byte row per four lanes), joined by
//           two lane shuffles; the workgroup forms the chunk's max m, p = exp(s - m) and l = sum p.
//           P V: lane = output dimension, wave w takes keys w, w + 4, ..., its 16 loads issued
//           together with the K loads; the four waves' sums are added in a fixed order; (m, l,
//           acc[64]) go to `part`;
//   pass 2: one workgroup per head merges its chunks (flash-decoding rescale by exp(m_c - M)): wave w
//           takes chunks w, w + 4, ..., the four waves' sums are added in a fixed order, the result is
//           divided by the total weight and q0 is added.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int HD = 64, CH = 64, NT = 256;   // head width, keys per chunk, threads per workgroup
constexpr int PART = HD + 2;                 // floats per (head, chunk) record: m, l, acc[64]

__device__ __forceinline__ float wave_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__global__ __launch_bounds__(NT) void k_pool_part(const float * __restrict__ q, const float * __restrict__ K,
                                                  const float * __restrict__ V, int64_t N, int64_t ld, float scale, int S,
                                                  float * __restrict__ part) {
    const int c = (int) blockIdx.x, h = (int) blockIdx.y, tid = (int) threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ float sq[HD], sp[CH], sred[2][4], sacc[4][HD];
    if (tid < HD) sq[tid] = q[(int64_t) h * HD + tid];
    __syncthreads();
    const int64_t t0 = (int64_t) c * CH;
    const int nc = (int) min<int64_t>(CH, N - t0);
    // scores: key kk = tid / 4, dims 16 * (tid % 4) .. + 15
    const int kk = tid >> 2, pq = tid & 3;
    float a = 0.0f;
    if (kk < nc) {
        const float4 * kr = (const float4 *) (K + (t0 + kk) * ld + (int64_t) h * HD + 16 * pq);
        float4 k4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) k4[i] = kr[i];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a += k4[i].x * sq[16 * pq + 4 * i];
            a += k4[i].y * sq[16 * pq + 4 * i + 1];
            a += k4[i].z * sq[16 * pq + 4 * i + 2];
            a += k4[i].w * sq[16 * pq + 4 * i + 3];
        }
    }
    // P V operands, issued before the score reductions so that their latency overlaps them:
    // lane = output dimension, wave wv takes keys wv, wv + 4, ..., wv + 60
    const float * vc = V + t0 * ld + (int64_t) h * HD + lane;
    float vv[CH / 4];
#pragma unroll
    for (int i = 0; i < CH / 4; i++) {
        const int j = wv + 4 * i;
        vv[i] = j < nc ? vc[(int64_t) j * ld] : 0.0f;
    }
    a += __shfl_xor(a, 1, 64);
    a += __shfl_xor(a, 2, 64);
    const float s = kk < nc ? a * scale : -INFINITY;
    float m = wave_max(s);
    if (lane == 0) sred[0][wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sred[0][0], sred[0][1]), fmaxf(sred[0][2], sred[0][3]));   // finite: nc >= 1
    const float p = kk < nc ? __expf(s - m) : 0.0f;
    if (pq == 0) sp[kk] = p;
    const float lw = wave_sum(pq == 0 ? p : 0.0f);
    if (lane == 0) sred[1][wv] = lw;
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CH / 4; i++) acc += sp[wv + 4 * i] * vv[i];
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

__global__ __launch_bounds__(NT) void k_pool_combine(const float * __restrict__ part, int S, const float * __restrict__ q0,
                                                     float * __restrict__ y) {
    const int h = (int) blockIdx.x, tid = (int) threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ float sred[4], sl[4], sacc[4][HD];
    const float * p = part + (int64_t) h * S * PART;
    float M = -INFINITY;
    for (int c = tid; c < S; c += NT) M = fmaxf(M, p[(int64_t) c * PART]);
    M = wave_max(M);
    if (lane == 0) sred[wv] = M;
    __syncthreads();
    M = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
    // wave wv merges chunks wv, wv + 4, ...; eight chunks' loads are in flight together
    float L = 0.0f, o = 0.0f;
    int c = wv;
    for (; c + 28 < S; c += 32) {
        float mm[8], ll[8], oo[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float * r = p + (int64_t) (c + 4 * i) * PART;
            mm[i] = r[0]; ll[i] = r[1]; oo[i] = r[2 + lane];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float w = __expf(mm[i] - M);
            L += ll[i] * w;
            o += oo[i] * w;
        }
    }
    for (; c < S; c += 4) {
        const float * r = p + (int64_t) c * PART;
        const float w = __expf(r[0] - M);
        L += r[1] * w;
        o += r[2 + lane] * w;
    }
    sacc[wv][lane] = o;
    if (lane == 0) sl[wv] = L;
    __syncthreads();
    if (tid < HD) {
        const float ot = (sacc[0][tid] + sacc[1][tid]) + (sacc[2][tid] + sacc[3][tid]);
        const float lt = (sl[0] + sl[1]) + (sl[2] + sl[3]);
        y[(int64_t) h * HD + tid] = ot / lt + q0[(int64_t) h * HD + tid];
    }
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
    k_pool_part<<<dim3(S, n_head), NT, 0, s>>>(q, K, V, N, ld, scale, S, part);
    k_pool_combine<<<n_head, NT, 0, s>>>(part, S, q0, y);
    return true;
}
