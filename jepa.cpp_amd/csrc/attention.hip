// attention.hip - flash attention forward on gfx950 (f16 MFMA, f32 softmax): head width 64 (and 32
// stored 64 wide) in the LDS-staged kernel below, other multiples of 16 up to 128 in k_attn_any.
//
// Computes softmax(Q K^T * scale) V per (item, head): the ggml_flash_attn_ext of reference
// src/jepa.cpp:416-442 (no mask, K/V in f16 as the reference's ggml_cast does, f32 softmax and f32
// accumulation). Q arrives with 3-D RoPE already applied by the QKV GEMM epilogue.
//
// Work split: one workgroup = 8 waves = 128 queries of one head. Waves 0-3 own 32 queries each and
// sweep the first half of the key tiles, waves 4-7 the same queries over the second half (two waves
// per SIMD: one wave's exp2 / VALU phase overlaps the other's MFMAs); the two halves are merged
// through LDS at the end. Keys come in tiles of 64: the K tile (64 keys x 64 dims) and the V^T tile
// (64 dims x 64 keys), 128 B per row, are copied HBM->LDS directly (buffer_load_dwordx4 ... lds) into
// a swizzled layout (lds_slot), NST - 1 tiles ahead of the one being used.
// MFMA roles are chosen so that softmax statistics need no cross-lane reduction beyond one
// xor-32 exchange:
//   S^T[key][q] = K . Q^T     A = K tile rows (keys), B = Q^T (held in registers for the sweep)
//                             -> lane (q = lane%32) holds 16 keys of its query column
//   O^T[d][q]  += V^T . P^T   A = V^T tile rows (d), B = P^T built in place from the S registers
// The B operand of the PV MFMA takes the 8 keys (4g..4g+3, 8+4g..8+4g+3 of each 16) that the S
// accumulator layout leaves in lane group g; V^T is stored with the same key order inside every
// 16-token group (written that way by the QKV epilogue), so both operands agree without shuffles.
// The running maximum is only moved when a tile's maximum exceeds it by more than 2^8 (in the
// exp2 domain), so the accumulators are rescaled a few times per sweep instead of every tile.
#include "kernels.h"
#include "model.h"
#include "lds_dma.h"
#include "lanes.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

namespace {

constexpr int HD = 64, QB = 128, KT = 64, NST = 4;
constexpr int TILE = KT * 128;                  // one K or V^T tile: 64 rows of 128 B
constexpr int STAGE = 2 * TILE;                 // K + V^T
constexpr int HALF = NST * STAGE;               // LDS of one key half
constexpr float LAZY = 8.0f;                    // keep the running max while growth <= 2^8

// 2^x by the hardware v_exp_f32 alone: exp2f adds a denormal-range fix-up (compare, select, add,
// ldexp) around it, which softmax weights do not need (a weight below 2^-126 next to a running
// sum >= 1 is lost to rounding either way; exp2(-inf) is still 0)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint16_t f2hbits(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

// 16-byte chunk c of LDS row r sits in slot c ^ ((r >> 1) & 7): the 16 rows one ds_read_b128 serves
// together land in 16 different 4-bank groups (128-B rows alternate between the two bank halves)
__device__ __forceinline__ int lds_slot(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ h8 lds_chunk(const unsigned char * base, int r, int c) {
    return *(const h8 *) (base + r * 128 + (lds_slot(r, c) << 4));
}

// s_waitcnt vmcnt(N) lgkmcnt(0), then a bare s_barrier (no fence: copies of later tiles stay in flight)
template <int N_>
__device__ __forceinline__ void tile_barrier() {
    static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit field");
    __builtin_amdgcn_s_waitcnt((N_ & 15) | ((N_ >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
}

// Keys visible to query row q of an item (block-causal attention, reference src/jepa.cpp:827-844):
// the np prefix rows read every key; a patch row of temporal slot f = (q - np) / tpf reads the patch
// keys of slots 0..f and no prefix key. tpf = 0: every query reads every key. Returns [lo, hi).
__device__ __forceinline__ int2 key_range(int q, int R, int np, int tpf) {
    if (tpf <= 0 || q < np) return make_int2(0, R);
    return make_int2(np, min(R, np + ((q - np) / tpf + 1) * tpf));
}

// OUT: A_F32 writes O f32 [item*R][H*HDO]; A_Q8_0 writes the q8_0 activation of the next linear
// (int8 codes [item*R][H*HDO] + f16 d per 32), the same values the separate quantizer would produce.
// HDO: the heads' real width, 64, or 32 for heads stored 64 wide with a zero upper half (their
// second Q.K^T dim pair and second P.V row block are skipped: both are zero).
// np / tpf select the block-causal mask (tpf = 0: none); key tiles that no query of the workgroup
// sees are not visited, 32-key blocks that no query of a wave sees are skipped by that wave.
template <int OUT, int HDO>
__global__ __launch_bounds__(512, 1) void k_attn_hd64(const _Float16 * __restrict__ Q, const _Float16 * __restrict__ Kp,
                                                      const _Float16 * __restrict__ Vt, void * __restrict__ O,
                                                      void * __restrict__ Od, int n_head, int64_t R, int64_t R_pad,
                                                      float c, int np, int tpf) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * HALF];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, g = lane >> 5;
    const int qg = wave & 3, kh = wave >> 2;            // query group, key half
    const int hw = wave & 3;                            // wave index inside its half (loads)
    // XCD-aware order: workgroups go to the 8 XCDs round-robin by linear id, so linear id L runs on
    // XCD L % 8. Renumber so that each XCD's share is a contiguous range of (head, query block): the
    // query blocks of one head then share one XCD's L2 for that head's K / V^T instead of all eight
    // fetching it (the identity when the grid is not a multiple of 8).
    const uint32_t gx = gridDim.x, total = gridDim.x * gridDim.y, lin = blockIdx.x + gx * blockIdx.y;
    const uint32_t rl = total % 8 == 0 ? (lin % 8) * (total / 8) + lin / 8 : lin;
    const uint32_t qblk = rl % gx;
    const int64_t head = rl / gx;
    const int64_t item = head / n_head;
    const int h = (int) (head - item * n_head);
    const int64_t q0 = (int64_t) qblk * QB + qg * 32;

    const _Float16 * Qh = Q + head * R_pad * HD;
    // buffer resources over this head's K rows and V^T rows (offsets below 4 GiB per head)
    const brsrc rK = make_brsrc(Kp + head * R_pad * HD, R_pad * HD * 2);
    const brsrc rV = make_brsrc(Vt + head * HD * R_pad, R_pad * HD * 2);

    // key tiles of this workgroup: the union of its queries' key ranges (the first query has the
    // lowest bound, the last the highest; a prefix row among them reads everything)
    const int qa = (int) qblk * QB, qz = min((int) R, qa + QB) - 1;
    const int klo_wg = key_range(qa, (int) R, np, tpf).x;
    const int khi_wg = qa < np ? (int) R : key_range(qz, (int) R, np, tpf).y;
    const int tfirst = klo_wg / KT;
    const int ntile = (khi_wg + KT - 1) / KT - tfirst;
    const int nt = (ntile + 1) / 2;                     // tiles per half (the second may have one less)
    const int t0 = tfirst + kh * nt;                    // first tile of this half
    const int my_nt = kh == 0 ? nt : ntile - nt;
    unsigned char * hbase = smem + kh * HALF;

    // stage s of this half: tile t0 + s. Each of the half's 4 waves copies 4 of the 16 row-groups.
    auto issue = [&](int s) {
        if (s >= my_nt) return;
        unsigned char * base = hbase + (s % NST) * STAGE;
        const int64_t key0 = (int64_t) (t0 + s) * KT;
        // lane fills slot lane % 8 of row r; all rows this wave copies are 8 hw + lane / 8 modulo 32
        const int cch = lds_slot(8 * hw + (lane >> 3), lane & 7);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int L = 4 * i + hw;                   // 0..7: K rows 8L..8L+7; 8..15: V^T rows
            const uint32_t r = 8 * (L & 7) + (lane >> 3);
            if (i < 2) dma_to_lds<16>(rK, r * (HD * 2) + 16 * cch, (uint32_t) key0 * (HD * 2), base + 1024 * (L & 7));
            else dma_to_lds<16>(rV, r * (uint32_t) R_pad * 2 + 16 * cch, (uint32_t) key0 * 2, base + TILE + 1024 * (L & 7));
        }
    };

    h8 qv[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) qv[kk] = *(const h8 *) (Qh + (q0 + l32) * HD + 16 * kk + 8 * g);

    const f16v zero = {0};
    f16v acc0 = zero, acc1 = zero;
    float m_run = -INFINITY, l_run = 0.0f;

    // this lane's key range, and the wave's bounds on it: a 32-key block below lo_max or reaching
    // past hi_min needs the per-key mask, one below lo_min or past hi_max is invisible to all lanes
    const int2 kr = key_range((int) q0 + l32, (int) R, np, tpf);
    const int qw = (int) q0, qp = max(qw, np);
    const int lo_min = key_range(qw, (int) R, np, tpf).x, lo_max = key_range(qw + 31, (int) R, np, tpf).x;
    const int hi_min = qp <= qw + 31 ? key_range(qp, (int) R, np, tpf).y : (int) R;
    const int hi_max = qw < np ? (int) R : key_range(qw + 31, (int) R, np, tpf).y;

    for (int s = 0; s < NST - 1; s++) issue(s);
    for (int s = 0; s < nt; s++) {
        // tile s has landed once only the copies of the NST - 2 younger tiles are outstanding; the
        // half with fewer tiles issues fewer, so its waits are conservative
        if (s + NST - 2 < my_nt) tile_barrier<(NST - 2) * 4>();
        else tile_barrier<0>();
        issue(s + NST - 1);
        if (s >= my_nt) continue;                       // (second half, odd tile count) barrier only
        const unsigned char * sK = hbase + (s % NST) * STAGE;
        const unsigned char * sV = sK + TILE;
        const int64_t kt = (int64_t) (t0 + s) * KT;
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const int kb0 = (int) kt + 32 * kb;
            if (kb0 + 32 <= lo_min || kb0 >= hi_max) continue;     // no query of this wave sees them
            f16v S = zero;
#pragma unroll
            for (int kk = 0; kk < HDO / 16; kk++) S = MFMA16(lds_chunk(sK, 32 * kb + l32, 2 * kk + g), qv[kk], S);
            if (kb0 < lo_max || kb0 + 32 > hi_min) {                 // keys past R or outside a lane's range
                const int key0 = kb0 + 4 * g;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = key0 + 8 * (r >> 2) + (r & 3);
                    if (key < kr.x || key >= kr.y) S[r] = -INFINITY;
                }
            }
            float mloc = S[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, S[r]);
            mloc = halves_max(mloc);
            if (mloc > m_run && (m_run == -INFINITY || (mloc - m_run) * c > LAZY)) {
                // move the reference maximum; rescale what was accumulated against the old one
                const float alpha = fast_exp2((m_run - mloc) * c);
                l_run *= alpha;
#pragma unroll
                for (int r = 0; r < 16; r++) { acc0[r] *= alpha; acc1[r] *= alpha; }
                m_run = mloc;
            }
            const float mc = m_run == -INFINITY ? 0.0f : m_run * c;   // no key seen yet: S is -inf too
            float p[16], lsum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) { p[r] = fast_exp2(fmaf(S[r], c, -mc)); lsum += p[r]; }
            lsum = halves_sum(lsum);
            l_run += lsum;
#pragma unroll
            for (int kk2 = 0; kk2 < 2; kk2++) {
                h8 pb;
#pragma unroll
                for (int e = 0; e < 8; e++) pb[e] = (_Float16) p[8 * kk2 + e];
                const int ch = 4 * kb + 2 * kk2 + g;
                acc0 = MFMA16(lds_chunk(sV, l32, ch), pb, acc0);
                if constexpr (HDO == 64) acc1 = MFMA16(lds_chunk(sV, 32 + l32, ch), pb, acc1);
            }
        }
    }

    // merge the two key halves: the second half's waves publish (m, l, acc) through LDS
    __syncthreads();
    float * xs = (float *) smem + (size_t) (qg * 64 + lane) * 34;
    if (kh == 1) {
        xs[0] = m_run; xs[1] = l_run;
#pragma unroll
        for (int r = 0; r < 16; r++) { xs[2 + r] = acc0[r]; xs[18 + r] = acc1[r]; }
    }
    __syncthreads();
    if (kh == 1) return;
    {
        const float m1 = xs[0], l1 = xs[1];
        const float m = fmaxf(m_run, m1);
        const float a0 = m_run == -INFINITY ? 0.0f : fast_exp2((m_run - m) * c);
        const float a1 = m1 == -INFINITY ? 0.0f : fast_exp2((m1 - m) * c);
        l_run = fmaf(l_run, a0, l1 * a1);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            acc0[r] = fmaf(acc0[r], a0, xs[2 + r] * a1);
            acc1[r] = fmaf(acc1[r], a0, xs[18 + r] * a1);
        }
    }

    const int64_t q = q0 + l32;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float o0[16], o1[16];
#pragma unroll
    for (int r = 0; r < 16; r++) { o0[r] = acc0[r] * inv; o1[r] = acc1[r] * inv; }
    const int64_t DD = (int64_t) n_head * HDO;
    if constexpr (OUT == A_Q8_0) {
        // dims 0-31 (acc0) and 32-63 (acc1) are one q8_0 block each, split over lanes l32 and l32+32
        float am0 = 0.0f, am1 = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) { am0 = fmaxf(am0, fabsf(o0[r])); am1 = fmaxf(am1, fabsf(o1[r])); }
        am0 = halves_max(am0);
        am1 = halves_max(am1);
        if (q >= R) return;
        const float id0 = am0 != 0.0f ? 127.0f / am0 : 0.0f, id1 = am1 != 0.0f ? 127.0f / am1 : 0.0f;
        int8_t * crow = (int8_t *) O + (item * R + q) * DD + h * HDO;
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int c0 = (int) fminf(fmaxf(rintf(o0[4 * qq + e] * id0), -128.0f), 127.0f);
                const int c1 = (int) fminf(fmaxf(rintf(o1[4 * qq + e] * id1), -128.0f), 127.0f);
                w0 |= ((uint32_t) c0 & 0xffu) << (8 * e);
                w1 |= ((uint32_t) c1 & 0xffu) << (8 * e);
            }
            const int d = 8 * qq + 4 * g;
            *(uint32_t *) (crow + d) = w0;
            if constexpr (HDO == 64) *(uint32_t *) (crow + 32 + d) = w1;
        }
        if (g == 0) {
            uint16_t * drow = (uint16_t *) Od + (item * R + q) * (DD / 32) + h * (HDO / 32);
            drow[0] = f2hbits(am0 / 127.0f);
            if constexpr (HDO == 64) drow[1] = f2hbits(am1 / 127.0f);
        }
    } else {
        if (q >= R) return;
        float * orow = (float *) O + (item * R + q) * DD + h * HDO;
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int d = 8 * qq + 4 * g;
            *(float4 *) (orow + d) = make_float4(o0[4 * qq], o0[4 * qq + 1], o0[4 * qq + 2], o0[4 * qq + 3]);
            if constexpr (HDO == 64)
                *(float4 *) (orow + 32 + d) = make_float4(o1[4 * qq], o1[4 * qq + 1], o1[4 * qq + 2], o1[4 * qq + 3]);
        }
    }
}

// Head widths other than 32 and 64 (80 for I-JEPA ViT-H/14): heads stored HDS = 32 * NDT wide with
// zero padding past hd (Q, K [head][R_pad][HDS], V^T [head][HDS][R_pad] in the PV order of the 16-token
// groups, as the QKV epilogue writes them). One workgroup = 4 waves = 128 queries of one head, each wave
// 32 queries over every key; K and V^T operands are read straight from global memory (L2), which suits
// the short sequences these models run (256 tokens at 224^2). The arithmetic per 32-key block is the
// fast kernel's: S^T = K . Q^T over NKK = ceil(hd / 16) dim steps (the padded dims are zero), the lazy
// online softmax in the exp2 form, O^T += V^T . P^T over NDT 32-dim row blocks. f32 output only: q8_0
// blocks of 32 dims would span heads.
template <int NKK, int NDT>
__global__ __launch_bounds__(256) void k_attn_any(const _Float16 * __restrict__ Q, const _Float16 * __restrict__ Kp,
                                                  const _Float16 * __restrict__ Vt, float * __restrict__ O, int n_head,
                                                  int hd, int64_t R, int64_t R_pad, float c, int np, int tpf) {
    constexpr int HDS = 32 * NDT;
    static_assert(NKK * 16 <= HDS, "dim steps inside the stored width");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int64_t head = blockIdx.y;
    const int64_t item = head / n_head;
    const int h = (int) (head - item * n_head);
    const int64_t q0 = (int64_t) blockIdx.x * 128 + 32 * wave;
    if (q0 >= R) return;                                  // whole wave past the last query
    const _Float16 * Qh = Q + head * R_pad * HDS;
    const _Float16 * Kh = Kp + head * R_pad * HDS;
    const _Float16 * Vh = Vt + head * HDS * R_pad;

    h8 qv[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; kk++) qv[kk] = *(const h8 *) (Qh + (q0 + l32) * HDS + 16 * kk + 8 * g);

    const f16v zero = {0};
    f16v acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = zero;
    float m_run = -INFINITY, l_run = 0.0f;
    const int2 kr = key_range((int) q0 + l32, (int) R, np, tpf);
    const int qw = (int) q0;
    const int lo_min = key_range(qw, (int) R, np, tpf).x;
    const int hi_max = qw < np ? (int) R : key_range(min(qw + 31, (int) R - 1), (int) R, np, tpf).y;
    for (int kb0 = (lo_min / 32) * 32; kb0 < hi_max; kb0 += 32) {
        f16v S = zero;
#pragma unroll
        for (int kk = 0; kk < NKK; kk++) S = MFMA16(*(const h8 *) (Kh + (int64_t) (kb0 + l32) * HDS + 16 * kk + 8 * g), qv[kk], S);
        const int key0 = kb0 + 4 * g;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = key0 + 8 * (r >> 2) + (r & 3);
            if (key < kr.x || key >= kr.y) S[r] = -INFINITY;
        }
        float mloc = S[0];
#pragma unroll
        for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, S[r]);
        mloc = halves_max(mloc);
        if (mloc > m_run && (m_run == -INFINITY || (mloc - m_run) * c > LAZY)) {
            const float alpha = fast_exp2((m_run - mloc) * c);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[dt][r] *= alpha;
            m_run = mloc;
        }
        const float mc = m_run == -INFINITY ? 0.0f : m_run * c;
        float p[16], lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) { p[r] = fast_exp2(fmaf(S[r], c, -mc)); lsum += p[r]; }
        lsum = halves_sum(lsum);
        l_run += lsum;
#pragma unroll
        for (int kk2 = 0; kk2 < 2; kk2++) {
            h8 pb;
#pragma unroll
            for (int e = 0; e < 8; e++) pb[e] = (_Float16) p[8 * kk2 + e];
            // V^T row d, keys kb0 + 16 kk2 + 8 g .. + 8 in the order of the S lanes (see the header)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                acc[dt] = MFMA16(*(const h8 *) (Vh + (int64_t) (32 * dt + l32) * R_pad + kb0 + 16 * kk2 + 8 * g), pb, acc[dt]);
        }
    }
    const int64_t q = q0 + l32;
    if (q >= R) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float * orow = O + (item * R + q) * ((int64_t) n_head * hd) + (int64_t) h * hd;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int d = 32 * dt + 8 * qq + 4 * g;
            if (d < hd)   // hd is a multiple of 16: a group of four is inside or outside as a whole
                *(float4 *) (orow + d) = make_float4(acc[dt][4 * qq] * inv, acc[dt][4 * qq + 1] * inv, acc[dt][4 * qq + 2] * inv,
                                                     acc[dt][4 * qq + 3] * inv);
        }
}

}  // namespace

int attention_stored_width(int hd) { return hd <= 64 ? 64 : (hd + 31) / 32 * 32; }

bool attention_supports(int hd) { return hd == 32 || hd == 64 || (hd > 0 && hd <= 128 && hd % 16 == 0); }

void launch_attention(const void * q, const void * k, const void * vt, const act_view & out, int64_t n_items,
                      int n_head, int hd, int64_t R, int64_t R_pad, float scale, int n_prefix, int64_t tokens_per_slot,
                      hipStream_t s) {
    // hd: 64, or 32 (stored 64 wide), or a multiple of 16 up to 128 stored attention_stored_width(hd)
    // wide (f32 output; checked by the callers)
    const float c = scale * 1.4426950408889634f;   // exp(x*scale) = exp2(x*scale*log2(e))
    const int tpf = (int) tokens_per_slot;
    dim3 grid((unsigned) ((R + QB - 1) / QB), (unsigned) (n_items * n_head));
    const _Float16 * Q = (const _Float16 *) q, * K = (const _Float16 *) k, * V = (const _Float16 *) vt;
    if (hd != 32 && hd != 64) {
        float * o = (float *) out.q;
        switch ((hd + 15) / 16) {
            case 1: k_attn_any<1, 2><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            case 3: k_attn_any<3, 2><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            case 5: k_attn_any<5, 3><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            case 6: k_attn_any<6, 3><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            case 7: k_attn_any<7, 4><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            case 8: k_attn_any<8, 4><<<grid, 256, 0, s>>>(Q, K, V, o, n_head, hd, R, R_pad, c, n_prefix, tpf); break;
            default: break;
        }
        return;
    }
    if (out.fmt == A_Q8_0) {
        if (hd == 32) k_attn_hd64<A_Q8_0, 32><<<grid, 512, 0, s>>>(Q, K, V, out.q, out.d, n_head, R, R_pad, c, n_prefix, tpf);
        else k_attn_hd64<A_Q8_0, 64><<<grid, 512, 0, s>>>(Q, K, V, out.q, out.d, n_head, R, R_pad, c, n_prefix, tpf);
    } else {
        if (hd == 32) k_attn_hd64<A_F32, 32><<<grid, 512, 0, s>>>(Q, K, V, out.q, nullptr, n_head, R, R_pad, c, n_prefix, tpf);
        else k_attn_hd64<A_F32, 64><<<grid, 512, 0, s>>>(Q, K, V, out.q, nullptr, n_head, R, R_pad, c, n_prefix, tpf);
    }
}
