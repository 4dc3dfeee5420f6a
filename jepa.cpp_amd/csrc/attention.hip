// attention.hip - flash attention forward on gfx950 (f16 MFMA, f32 softmax): head width 64 (and 32
// stored 64 wide) in the LDS-staged kernel below, other multiples of 16 up to 128 in k_attn_any.
//
// Computes softmax(Q K^T * scale) V per (item, head): the ggml_flash_attn_ext of reference
// src/jepa.cpp:416-442 (no mask, K/V in f16 as the reference's ggml_cast does, f32 softmax and f32
// accumulation). Q arrives with 3-D RoPE already applied by the QKV GEMM epilogue.
//
// Work split: one workgroup = 128 queries of one head, in QG query groups of QT 32-query MFMA tiles
// (QG x QT = 4) times KS key splits (1, 2 or 4 by the key count: attention_key_splits), one wave
// each. With QT = 1 and KS = 4 that is 16 waves (four per SIMD, 128 VGPRs each); QT = 2 (8 waves
// whose every K and V^T read from LDS feeds two MFMAs) measured slower (32.9 against 30.3 us at 2048
// tokens x 16 heads). The splits are merged through LDS at the end. Keys come in
// tiles of 64: the K tile (64 keys x 64 dims) and the V^T tile (64 dims x 64 keys), 128 B per row, are
// copied HBM->LDS directly (buffer_load_dwordx4 ... lds) into a swizzled layout (lds_slot),
// double-buffered per split: tile s + 1 is copied while tile s is used.
// MFMA roles are chosen so that softmax statistics need no cross-lane reduction beyond one
// xor-32 exchange:
//   S^T[key][q] = K . Q^T     A = K tile rows (keys), B = Q^T (held in registers for the sweep)
//                             -> lane (q = lane%32) holds 16 keys of its query column
//   O^T[d][q]  += V^T . P^T   A = V^T tile rows (d), B = P^T built in place from the S registers
// The B operand of the PV MFMA takes the 8 keys (4g..4g+3, 8+4g..8+4g+3 of each 16) that the S
// accumulator layout leaves in lane group g; V^T is stored with the same key order inside every
// 16-token group (written that way by the QKV epilogue), so both operands agree without shuffles.
// Scores become exponents t = s c - M in one fma (c = scale log2 e, M the running maximum already
// scaled by c), the weights are 2^t; M is only moved when a block's largest t exceeds 8 (weights up to
// 2^8), so the accumulators are rescaled a few times per sweep instead of every block. The row sums
// add the f16 weights that the P.V MFMA uses (v_dot2_f32_f16 against (1, 1)).
#include "kernels.h"
#include "model.h"
#include "lds_dma.h"
#include "lanes.h"
#include "quant_dev.h"

#include <type_traits>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

namespace {

constexpr int HD = 64, QB = 128, KT = 64;
constexpr int TILE = KT * 128;                  // one K or V^T tile: 64 rows of 128 B
constexpr int STAGE = 2 * TILE;                 // K + V^T
constexpr int SPLIT = 2 * STAGE;                // LDS of one key split: two stages
constexpr float LAZY = 8.0f;                    // keep the running max while growth <= 2^8
constexpr int ATTN_QT = 1;                      // query tiles per wave (see the work split above)

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

// OUT: A_F32 writes O f32 [item*R][H*HDO], A_F16 the same rounded to f16; A_Q8_0 writes the q8_0 activation of the next linear
// (int8 codes [item*R][H*HDO] + f16 d per 32), the same values the separate quantizer would produce.
// HDO: the heads' real width, 64, or 32 for heads stored 64 wide with a zero upper half (their
// second Q.K^T dim pair and second P.V row block are skipped: both are zero).
// np / tpf select the block-causal mask (tpf = 0: none); key tiles that no query of the workgroup
// sees are not visited. MASKED = false (no block-causal mask, R a multiple of 64: every key of every
// visited tile is visible to every query) drops the per-key mask code from the loop.
template <int OUT, int HDO, bool MASKED, int QT, int KS>
__global__ __launch_bounds__(64 * KS * 4 / QT, 1) void k_attn_hd64(const _Float16 * __restrict__ Q, const _Float16 * __restrict__ Kp,
                                                                   const _Float16 * __restrict__ Vt, void * __restrict__ O,
                                                                   void * __restrict__ Od, int n_head, int64_t R, int64_t R_pad,
                                                                   float c, int np, int tpf) {
    static_assert(KS == 1 || KS == 2 || KS == 4, "key splits");
    constexpr int NKK = HDO / 16, NDT = HDO / 32;       // Q.K^T dim steps, P.V row blocks
    constexpr int QG = 4 / QT;                          // query groups: QG x QT x 32 = 128 queries
    constexpr int QW = 32 * QT;                         // queries per wave
    constexpr int CPW = 16 / QG;                        // 1 KB copies per wave per tile
    __shared__ __attribute__((aligned(16))) unsigned char smem[KS * SPLIT];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, g = lane >> 5;
    const int qg = wave % QG, ks = wave / QG;           // query group, key split
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
    const int64_t q0 = (int64_t) qblk * QB + qg * QW;   // this wave's queries: q0 .. q0 + QW - 1

    const _Float16 * Qh = Q + head * R_pad * HD;
    // buffer resources over this head's K rows and V^T rows (offsets below 4 GiB per head)
    const brsrc rK = make_brsrc(Kp + head * R_pad * HD, R_pad * HD * 2);
    const brsrc rV = make_brsrc(Vt + head * HD * R_pad, R_pad * HD * 2);

    // key tiles of this workgroup: the union of its queries' key ranges (the first query has the
    // lowest bound, the last the highest; a prefix row among them reads everything), dealt to the
    // KS splits in contiguous runs (the first ntile % KS splits take one more)
    const int qa = (int) qblk * QB, qz = min((int) R, qa + QB) - 1;
    const int klo_wg = key_range(qa, (int) R, np, tpf).x;
    const int khi_wg = qa < np ? (int) R : key_range(qz, (int) R, np, tpf).y;
    const int tfirst = klo_wg / KT;
    const int ntile = (khi_wg + KT - 1) / KT - tfirst;
    const int nbase = ntile / KS, nrem = ntile % KS;
    const int nt = nbase + (nrem > 0);                  // loop trips (the longest split)
    const int my_nt = nbase + (ks < nrem);
    const int t0 = tfirst + ks * nbase + min(ks, nrem); // first tile of this split
    unsigned char * sbase = smem + ks * SPLIT;

    // tile s of this split into stage s % 2, copied by the split's QG waves: 16 row-groups of 8 rows
    // (K rows, then V^T rows), row-group L = QG i + qg for this wave
    auto issue = [&](int s) {
        if (s >= my_nt) return;
        unsigned char * base = sbase + (s & 1) * STAGE;
        const int64_t key0 = (int64_t) (t0 + s) * KT;
        // lane fills slot lane % 8 of row r; all rows this wave copies agree modulo 16 (QG is even)
        const int cch = lds_slot(8 * (qg & 1) + (lane >> 3), lane & 7);
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const int L = QG * i + qg;                  // 0..7: K rows 8L..8L+7; 8..15: V^T rows
            const uint32_t r = 8 * (L & 7) + (lane >> 3);
            if (L < 8) dma_to_lds<16>(rK, r * (HD * 2) + 16 * cch, (uint32_t) key0 * (HD * 2), base + 1024 * (L & 7));
            else dma_to_lds<16>(rV, r * (uint32_t) R_pad * 2 + 16 * cch, (uint32_t) key0 * 2, base + TILE + 1024 * (L & 7));
        }
    };
    issue(0);

    // Q^T operands of the query tiles (rows past R are zero in the padded layout)
    h8 qv[QT][NKK];
#pragma unroll
    for (int qt = 0; qt < QT; qt++)
#pragma unroll
        for (int kk = 0; kk < NKK; kk++) qv[qt][kk] = *(const h8 *) (Qh + (q0 + 32 * qt + l32) * HD + 16 * kk + 8 * g);

    const f16v zero = {0};
    f16v acc[QT][NDT];
    // running maximum in the exp2 domain: mcs = max(s) * c (-inf before the first visible key) and
    // nm = -mcs (0 before the first key), the addend of every score's fma; a block moves it when its
    // largest exponent exceeds thr (-inf before the first visible key, LAZY after)
    float mcs[QT], nm[QT], thr[QT], l_run[QT];
    int2 kr[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) acc[qt][dt] = zero;
        mcs[qt] = -INFINITY; nm[qt] = 0.0f; thr[qt] = -INFINITY; l_run[qt] = 0.0f;
        kr[qt] = key_range((int) q0 + 32 * qt + l32, (int) R, np, tpf);   // this lane's key range per tile
    }
    // the wave's bounds on its queries' ranges: a 32-key block below lo_max or reaching past hi_min
    // needs the per-key mask (blocks no query of the wave sees are masked whole)
    const int qw = (int) q0, qp = max(qw, np);
    const int lo_max = key_range(qw + QW - 1, (int) R, np, tpf).x;
    const int hi_min = qp <= qw + QW - 1 ? key_range(qp, (int) R, np, tpf).y : (int) R;

    // One 32-key block kb of a tile and one query tile qt form a unit with four phases: A (S = K.Q^T,
    // NKK chained MFMAs), M (mask, row maximum, the rare lazy rescale), E (exp2, row sum, f16 weights:
    // VALU only) and P (O^T += V^T.P^T, MFMAs). The units of a tile, kb-major, are software-pipelined
    // so that each unit's E runs while the next unit's A MFMAs execute and its P MFMAs while the next
    // unit's M runs: a wave keeps the matrix core and the VALU busy together.
    auto qk = [&](int qt, const h8 (&kc)[NKK]) {
        f16v S = zero;
#pragma unroll
        for (int kk = 0; kk < NKK; kk++) S = MFMA16(kc[kk], qv[qt][kk], S);
        return S;
    };
    // M: keys past R or outside a lane's range (block-causal) to -inf, the exponents t = s c - mcs
    // (in place of the scores), then the lazy maximum. The maximum is taken over the fma results, which
    // the compiler knows to be canonical floats: over the raw MFMA results it would first canonicalize
    // every value (an extra v_max_f32 each, for IEEE NaN semantics).
    auto mx = [&](int qt, f16v & S, int kb0) {
        if (MASKED && (kb0 < lo_max || kb0 + 32 > hi_min)) {
            const int key0 = kb0 + 4 * g;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = key0 + 8 * (r >> 2) + (r & 3);
                if (key < kr[qt].x || key >= kr[qt].y) S[r] = -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) S[r] = fmaf(S[r], c, nm[qt]);
        // a chain of three-input maxima (v_max3_f32): 8 ops for 16 values
        float tl = fmaxf(fmaxf(S[0], S[1]), S[2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) tl = fmaxf(fmaxf(tl, S[r]), S[r + 1]);
        tl = halves_max_nonan(fmaxf(tl, S[15]));
        // the first visible key sets the maximum; later, it moves when a block's exceeds it by 2^LAZY
        const bool move = tl > thr[qt];
        if (__builtin_amdgcn_ballot_w64(move) != 0) {   // rare after the first blocks: a uniform branch
            // move the reference maximum by tl; rescale what was accumulated against the old one and
            // shift this block's exponents (the empty volatile asm keeps the compiler from executing
            // this block speculatively on every block)
            asm volatile("");
            const bool first = mcs[qt] == -INFINITY;
            const float sh = move ? tl : 0.0f;
            const float alpha = first ? 0.0f : fast_exp2(-sh);   // nothing accumulated yet: 0, not 2^-sh
            l_run[qt] *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[qt][dt][r] *= alpha;
#pragma unroll
            for (int r = 0; r < 16; r++) S[r] = __fsub_rn(S[r], sh);
            mcs[qt] = move ? (first ? tl : mcs[qt] + tl) : mcs[qt];
            nm[qt] = mcs[qt] == -INFINITY ? 0.0f : -mcs[qt];
            thr[qt] = mcs[qt] == -INFINITY ? -INFINITY : LAZY;
        }
    };
    // E: weights 2^t as the f16 B operand of the P.V MFMA, and the f32 sum of those f16 weights into
    // l (v_dot2_f32_f16 against (1, 1): eight ops instead of fifteen adds, and the normalizer is the
    // sum of the weights the P.V products actually used)
    const h2 one2 = {(_Float16) 1.0f, (_Float16) 1.0f};
    auto ex = [&](int qt, const f16v & S, h8 (&pb)[2]) {
#pragma unroll
        for (int r = 0; r < 16; r++) pb[r >> 3][r & 7] = (_Float16) fast_exp2(S[r]);
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s0 = __builtin_amdgcn_fdot2(h2{pb[0][2 * k], pb[0][2 * k + 1]}, one2, s0, false);
            s1 = __builtin_amdgcn_fdot2(h2{pb[1][2 * k], pb[1][2 * k + 1]}, one2, s1, false);
        }
        l_run[qt] += halves_sum(s0 + s1);
    };
    auto pv = [&](int qt, const h8 (&pb)[2], const h8 (&vc)[2][NDT]) {
#pragma unroll
        for (int kk2 = 0; kk2 < 2; kk2++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[qt][dt] = MFMA16(vc[kk2][dt], pb[kk2], acc[qt][dt]);
    };
    // one MFMA, then n VALU instructions, four times: the interleave of an A phase with E's VALU work
    auto interleave = [] {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
        }
    };
    constexpr int U = 2 * QT;                           // units per tile

    for (int s = 0; s < nt; s++) {
        // tile s has landed (this wave's copies: vmcnt(0); the other waves': the barrier), and every
        // wave is past tile s - 1, whose stage tile s + 1 now refills
        tile_barrier<0>();
        // a wave raises its issue priority for the first half of the tile and drops it after: the
        // waves of a SIMD otherwise share it by age, and the oldest would idle at the next barrier
        // while the youngest finishes (measured 30.0 -> 29.5 us at 2048 tokens x 16 heads)
        __builtin_amdgcn_s_setprio(1);
        issue(s + 1);
        if (s >= my_nt) continue;                       // (a split with one tile less) barrier only
        const unsigned char * sK = sbase + (s & 1) * STAGE;
        const unsigned char * sV = sK + TILE;
        const int kt = (t0 + s) * KT;
        h8 kc[NKK], vc[2][2][NDT], pb[2];
        f16v S[U];
        auto load_k = [&](int kb) {
#pragma unroll
            for (int kk = 0; kk < NKK; kk++) kc[kk] = lds_chunk(sK, 32 * kb + l32, 2 * kk + g);
        };
        auto load_v = [&](int kb) {
#pragma unroll
            for (int kk2 = 0; kk2 < 2; kk2++)
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) vc[kb][kk2][dt] = lds_chunk(sV, 32 * dt + l32, 4 * kb + 2 * kk2 + g);
        };
        load_k(0);
        load_v(0);
        S[0] = qk(0, kc);                               // A(0)
        mx(0, S[0], kt);                                // M(0)
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int qt = u % QT, kb = u / QT;
            if (u + 1 < U) {
                const int qn = (u + 1) % QT, kn = (u + 1) / QT;
                if (kn != kb) load_k(kn);
                S[u + 1] = qk(qn, kc);                  // A(u+1) with E(u)
                ex(qt, S[u], pb);
                interleave();
                if (kn != kb) load_v(kn);
                pv(qt, pb, vc[kb]);                     // P(u) with M(u+1)
                if (u == U / 2 - 1) __builtin_amdgcn_s_setprio(0);
                mx(qn, S[u + 1], kt + 32 * kn);
            } else {
                ex(qt, S[u], pb);                       // E, P of the tile's last unit
                pv(qt, pb, vc[kb]);
            }
        }
    }

    // merge the key splits: splits 1..KS-1 publish (m, l, acc) through LDS (value-major, one float
    // per lane per bank), split 0 combines them in split order
    constexpr int NV = QT * (2 + 16 * NDT);             // floats per lane: per query tile m, l, acc
    __builtin_amdgcn_s_setprio(0);
    if constexpr (KS > 1) {
        __syncthreads();                                // every wave is past its last stage read
        if (ks > 0) {
            float * xs = (float *) smem + (size_t) ((ks - 1) * QG + qg) * NV * 64 + lane;
#pragma unroll
            for (int qt = 0; qt < QT; qt++) {
                float * x = xs + (size_t) qt * (NV / QT) * 64;
                x[0] = mcs[qt]; x[64] = l_run[qt];
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) x[(2 + 16 * dt + r) * 64] = acc[qt][dt][r];
            }
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            float mi[KS], ai[KS];
            mi[0] = mcs[qt];
            float m = mcs[qt];
#pragma unroll
            for (int k = 1; k < KS; k++) {
                mi[k] = ((const float *) smem)[(size_t) ((k - 1) * QG + qg) * NV * 64 + (size_t) qt * (NV / QT) * 64 + lane];
                m = fmaxf(m, mi[k]);
            }
#pragma unroll
            for (int k = 0; k < KS; k++) ai[k] = mi[k] == -INFINITY ? 0.0f : fast_exp2(mi[k] - m);
            float l = l_run[qt] * ai[0];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[qt][dt][r] *= ai[0];
#pragma unroll
            for (int k = 1; k < KS; k++) {
                const float * x = (const float *) smem + (size_t) ((k - 1) * QG + qg) * NV * 64 + (size_t) qt * (NV / QT) * 64 + lane;
                l = fmaf(x[64], ai[k], l);
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[qt][dt][r] = fmaf(x[(2 + 16 * dt + r) * 64], ai[k], acc[qt][dt][r]);
            }
            l_run[qt] = l;
        }
    }

    const int64_t DD = (int64_t) n_head * HDO;
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        const int64_t q = q0 + 32 * qt + l32;
        const float inv = l_run[qt] > 0.0f ? 1.0f / l_run[qt] : 0.0f;
        float o[NDT][16];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[dt][r] = acc[qt][dt][r] * inv;
        if constexpr (OUT == A_Q8_0) {
            // each 32-dim row block is one q8_0 block, split over lanes l32 and l32 + 32
            float am[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                am[dt] = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) am[dt] = fmaxf(am[dt], fabsf(o[dt][r]));
                am[dt] = halves_max(am[dt]);
            }
            if (q < R) {
                int8_t * crow = (int8_t *) O + (item * R + q) * DD + h * HDO;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
                    const float id = am[dt] != 0.0f ? 127.0f / am[dt] : 0.0f;
#pragma unroll
                    for (int qq = 0; qq < 4; qq++) {
                        uint32_t w = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            w |= q8_byte(o[dt][4 * qq + e], id) << (8 * e);
                        }
                        *(uint32_t *) (crow + 32 * dt + 8 * qq + 4 * g) = w;
                    }
                }
                if (g == 0) {
                    uint16_t * drow = (uint16_t *) Od + (item * R + q) * (DD / 32) + h * (HDO / 32);
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++) drow[dt] = f2hbits(am[dt] / 127.0f);
                }
            }
        } else if constexpr (OUT == A_F16) {
            // the f16 input of an f16 out-projection: the f32 values rounded to nearest, as the
            // separate conversion would
            if (q < R) {
                _Float16 * orow = (_Float16 *) O + (item * R + q) * DD + h * HDO;
                typedef _Float16 h4o __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int qq = 0; qq < 4; qq++)
                        *(h4o *) (orow + 32 * dt + 8 * qq + 4 * g) = h4o{(_Float16) o[dt][4 * qq], (_Float16) o[dt][4 * qq + 1],
                                                                          (_Float16) o[dt][4 * qq + 2], (_Float16) o[dt][4 * qq + 3]};
            }
        } else {
            if (q < R) {
                float * orow = (float *) O + (item * R + q) * DD + h * HDO;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int qq = 0; qq < 4; qq++)
                        *(float4 *) (orow + 32 * dt + 8 * qq + 4 * g) =
                            make_float4(o[dt][4 * qq], o[dt][4 * qq + 1], o[dt][4 * qq + 2], o[dt][4 * qq + 3]);
            }
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
    // the running maximum in the exp2 domain, as in k_attn_hd64: mcs, its negation nm, threshold thr
    float mcs = -INFINITY, nm = 0.0f, thr = -INFINITY, l_run = 0.0f;
    const int2 kr = key_range((int) q0 + l32, (int) R, np, tpf);
    const int qw = (int) q0;
    const int lo_min = key_range(qw, (int) R, np, tpf).x;
    const int hi_max = qw < np ? (int) R : key_range(min(qw + 31, (int) R - 1), (int) R, np, tpf).y;
    const h2 one2 = {(_Float16) 1.0f, (_Float16) 1.0f};
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
#pragma unroll
        for (int r = 0; r < 16; r++) S[r] = fmaf(S[r], c, nm);
        float tl = fmaxf(fmaxf(S[0], S[1]), S[2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) tl = fmaxf(fmaxf(tl, S[r]), S[r + 1]);
        tl = halves_max_nonan(fmaxf(tl, S[15]));
        if (tl > thr) {
            const bool first = mcs == -INFINITY;
            const float alpha = first ? 0.0f : fast_exp2(-tl);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[dt][r] *= alpha;
#pragma unroll
            for (int r = 0; r < 16; r++) S[r] = __fsub_rn(S[r], tl);
            mcs = first ? tl : mcs + tl;
            nm = -mcs;
            thr = LAZY;
        }
        float lsum = 0.0f;
#pragma unroll
        for (int kk2 = 0; kk2 < 2; kk2++) {
            h8 pb;
#pragma unroll
            for (int e = 0; e < 8; e++) pb[e] = (_Float16) fast_exp2(S[8 * kk2 + e]);
#pragma unroll
            for (int e = 0; e < 4; e++) lsum = __builtin_amdgcn_fdot2(h2{pb[2 * e], pb[2 * e + 1]}, one2, lsum, false);
            // V^T row d, keys kb0 + 16 kk2 + 8 g .. + 8 in the order of the S lanes (see the header)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                acc[dt] = MFMA16(*(const h8 *) (Vh + (int64_t) (32 * dt + l32) * R_pad + kb0 + 16 * kk2 + 8 * g), pb, acc[dt]);
        }
        l_run += halves_sum(lsum);
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

// Key splits by the key count R only (so an item's result does not depend on the batch). Fewer
// splits mean fewer waves per workgroup, less LDS (32 KB per split) and no merge, and more workgroups
// per CU. Measured (us per launch, q8_0 output, splits 1 / 2 / 4): 197 keys x 6 heads 8.1 / 8.0 /
// 10.4, 576 x 96 17.7 / 18.2 / 24.9, 2048 x 16 34.1 / 27.8 / 27.9, 8192 x 22 461 / 461 / 481.
int attention_key_splits(int64_t R) {
    return R <= 1024 ? 1 : R <= 4096 ? 4 : 2;
}

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
    const bool masked = tpf > 0 || R % KT != 0;
    const int ks = attention_key_splits(R);
    constexpr int QT = ATTN_QT;
    static_assert(QT == 1 || QT == 2, "one or two query tiles per wave");
    // kernel instance by output format, stored head width, mask and key splits
    auto go = [&](auto out_c, auto hdo_c, auto masked_c, void * od) {
        constexpr int OUT = decltype(out_c)::value, HDO = decltype(hdo_c)::value;
        constexpr bool MK = decltype(masked_c)::value;
        auto run = [&](auto kern, int ks_) { kern<<<grid, 64 * ks_ * 4 / QT, 0, s>>>(Q, K, V, out.q, od, n_head, R, R_pad, c, n_prefix, tpf); };
        if (ks == 1) run(k_attn_hd64<OUT, HDO, MK, QT, 1>, 1);
        else if (ks == 2) run(k_attn_hd64<OUT, HDO, MK, QT, 2>, 2);
        else run(k_attn_hd64<OUT, HDO, MK, QT, 4>, 4);
    };
    auto by_width = [&](auto out_c, void * od) {
        using T = std::true_type;
        using F = std::false_type;
        using W32 = std::integral_constant<int, 32>;
        using W64 = std::integral_constant<int, 64>;
        if (hd == 32) masked ? go(out_c, W32{}, T{}, od) : go(out_c, W32{}, F{}, od);
        else masked ? go(out_c, W64{}, T{}, od) : go(out_c, W64{}, F{}, od);
    };
    if (out.fmt == A_Q8_0) by_width(std::integral_constant<int, A_Q8_0>{}, out.d);
    else if (out.fmt == A_F16) by_width(std::integral_constant<int, A_F16>{}, nullptr);
    else by_width(std::integral_constant<int, A_F32>{}, nullptr);
}
