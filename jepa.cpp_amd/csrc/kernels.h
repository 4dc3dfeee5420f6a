// kernels.h - launchers of the hand-written gfx950 kernels (host-callable, stream-ordered).
//
// Data layouts in HBM (row-major unless stated):
//   residual stream  x      f32 [rows][D]
//   GEMM operands    W      int8 [N][K] codes (q8_0 q, q4_0 q-8); 4-bit [N][K/2] q4_K codes; f16 weights
//                    X      int8 [M][K] q8_0 / q8_K activation codes; f16 [M][K] f16-rounded values
//   scales           q8_0   f16 [rows][K/32];  q8_K  f32 d [rows][K/256] + f16 bsums [rows][K/16]
//   attention        Q, K   f16 [item*H][R_pad][hd];  V^T f16 [item*H][hd][R_pad] with the tokens of
//                    every 16-token group stored in the order the PV MFMA reads them
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

struct act_view {            // a GEMM activation operand / a quantizer output
    int       fmt = 0;       // afmt
    void *    q = nullptr;   // int8 [M][K] (A_Q8_0 / A_Q8_K), f16 [M][K] (A_F16) or f32 [M][K] (A_F32)
    void *    d = nullptr;   // A_Q8_0: f16 [M][K/32]; A_Q8_K: f32 [M][K/256]
    void *    bsum = nullptr;// A_Q8_K: f16 [M][K/16]
    int64_t   ld = 0;        // K
};

enum epi_kind {
    EPI_F32 = 0,      // y[map(m)][n] = acc + bias (+ addvec[n]) (+ addrows[pre + m%rin][n])
    EPI_RESID,        // x[m][n] += (acc + bias) (* ls[n])
    EPI_GELU_F32,     // y[m][n] = gelu(acc + bias)
    EPI_GELU_F16,     // oh[m][n] = f16(gelu(acc + bias))
    EPI_GELU_Q8_0,    // q8_0-quantize gelu(acc + bias) into (oq, od)
    EPI_QKV,          // split into Q, K (RoPE'd) and V^T f16 attention operands
    EPI_GELU_Q8_K,    // q8_K-quantize gelu(acc + bias) into (oh codes, od d, ob bsums); 256-wide tiles
};

struct gemm_epi {
    int kind = EPI_F32;
    float * y = nullptr; int64_t ldy = 0;
    int64_t rin = 0, rout = 0, pre = 0;     // EPI_F32 row map: row = (m/rin)*rout + pre + m%rin (rin 0: row = m)
    const float * addvec = nullptr;
    const float * addrows = nullptr;
    const float * ls = nullptr;
    void * oq = nullptr; void * od = nullptr; void * oh = nullptr; void * ob = nullptr;
    // EPI_QKV
    void * q = nullptr; void * k = nullptr; void * vt = nullptr;
    const float * rope_c = nullptr; const float * rope_s = nullptr;
    int n_head = 0, hd = 0, D = 0;
    int hds = 0;                            // stored head width of Q / K / V^T (0: hd); 64 for hd 32 heads,
                                            // whose upper 32 dims stay zero
    int64_t R = 0, R_pad = 0;
    int64_t col0 = 0;                       // this launch's outputs are columns col0.. of the [q | k | v]
                                            // layout (one part of separate q / k / v linears; else 0)
};

struct dev_linear;

// Scratch of the split-K GEMMs (int8 / 4-bit weights with N <= 1024: two workgroups per output tile,
// one per K half; f16 weights over few rows: up to four K parts): the raw accumulators of every part
// and one arrival counter per tile, which must be zero before the first launch (every launch leaves
// them zero). Sizes from gemm_split_ws_size.
struct gemm_split_ws {
    float * part = nullptr;
    int * cnt = nullptr;
    int64_t part_floats = 0, cnt_n = 0;
    // f16 residual GEMMs may split K by the launch's tile count, so that an output's rounding can
    // depend on the number of rows (false: only a forced split, for workspaces whose batched items
    // must equal one-item calls bit for bit)
    bool f16_by_tiles = true;
};
void gemm_split_ws_size(int64_t max_rows, int64_t * part_floats, int64_t * cnt_n);

// Y = X W^T (+ epilogue). M = rows of X. Without split scratch every tile is one workgroup.
void launch_gemm(const dev_linear & W, const act_view & X, int64_t M, const gemm_epi & ep, hipStream_t s,
                 const gemm_split_ws * sw = nullptr);
// K halves the int8 / 4-bit GEMM of this weight format and shape runs in (1 or 2); depends on N and K
// only, so that the summation order of an output never depends on the number of rows (f16 weights:
// chosen per launch from the tile count, 1 here)
int gemm_split_for(int wf, int64_t N, int64_t K);

// LayerNorm (ggml_norm + affine) of x [M][D] written in `out` format; w/b may be null (no affine).
// out.fmt A_F32 writes f32 rows into out.q. When normalize == false the rows are only quantized.
void launch_rownorm_quant(const float * x, int64_t M, int64_t D, const float * w, const float * b, float eps,
                          bool normalize, const act_view & out, hipStream_t s);

// Flash attention over (items*H) heads into `out` [item*R][H*hd]: hd 64, or hd 32 with Q / K / V^T
// stored 64 wide (zero upper half, gemm_epi::hds). A_F32 (f32 rows in out.q) or
// A_Q8_0 (the next linear's q8_0 activation: int8 codes in out.q, f16 d per 32 in out.d).
// tokens_per_slot > 0 applies the block-causal mask: n_prefix leading rows read every key, a patch row
// reads the patch keys of its own and earlier temporal slots (tokens_per_slot rows each) and no prefix
// key. tokens_per_slot = 0: full attention.
// key splits (waves per query group, merged through LDS) of the head-width-64 attention for R keys
int attention_key_splits(int64_t R);
void launch_attention(const void * q, const void * k, const void * vt, const act_view & out, int64_t n_items, int n_head,
                      int hd, int64_t R, int64_t R_pad, float scale, int n_prefix, int64_t tokens_per_slot, hipStream_t s);
// Head widths the attention runs: 32, 64, and other multiples of 16 up to 128 (f32 output only); the
// width Q, K and V^T are stored with (64 for hd <= 64, else hd rounded up to 32; the rest zero).
bool attention_supports(int hd);
int attention_stored_width(int hd);

// Single-query attention of the attentive-pool head: y = softmax(q . K^T * scale) V + q0 per head
// (hd 64), q / q0 / y [n_head * hd], K / V f32 rows [N][ld]. `part` holds pool_attention_part_floats
// floats of per-chunk partial results. Returns false (logged) on an unsupported shape.
int64_t pool_attention_part_floats(int64_t N, int n_head);
bool launch_pool_attention(const float * q, const float * K, const float * V, int64_t N, int64_t ld, int n_head, int hd, float scale,
                           const float * q0, float * y, float * part, int64_t part_floats, hipStream_t s);

// Patch rows from NCTHW input: rows [items*Np][C*tub*P*P] in f16 (half_out) or f32.
void launch_patchify(const float * in, void * rows, bool half_out, int64_t n_items, int C, int T, int H, int W,
                     int P, int tub, bool video, hipStream_t s);

// prefix (CLS) rows: x[it*R + 0][n] = cls[n] (+ pos[n])
void launch_cls_rows(float * x, const float * cls, const float * pos, int64_t n_items, int64_t R, int64_t D, hipStream_t s);
// rows 0 .. (cls ? 1 : 0) + n_reg - 1 of every item of R rows: CLS, then the register rows [n_reg][D],
// each plus its row of pos when pos is not null
void launch_prefix_rows(float * x, const float * cls, const float * reg, int n_reg, const float * pos, int64_t n_items, int64_t R,
                        int64_t D, hipStream_t s);

// f32 values -> ggml blocks of dst_type (q8_0, q4_0, q4_K) or f16, bit-exact with ggml's reference
// quantizers; n a multiple of the block size. Returns false for another type or a ragged n.
bool launch_quantize_rows(int dst_type, const float * x, int64_t n, void * y, hipStream_t s);

// weight expansion at load: raw ggml blocks (device) -> dev_linear operand arrays (int8: q4_0 rows
// go to the int8 layout of q8_0 whatever their length, for a linear whose parts mix the two)
void launch_repack(int gtype, const void * raw, int64_t n_out, int64_t n_in, void * w, void * wd,
                   void * wmin, hipStream_t s, bool int8 = false);

// test hooks
// force the MFMA GEMM onto workgroup tile `index` (0..8) for every later launch whose N it divides;
// -1 restores the automatic choice. Returns -1 for an index past the table.
int gemm_force_tile(int index);
// force the split-K choice: 1 off, 2 on where the shape allows it, -1 automatic
int gemm_force_split(int split);
void launch_qkv_split(const float * qkv, int64_t M, int64_t N, const gemm_epi & ep, hipStream_t s);
void launch_dequant_rows(int gtype, const void * raw, int64_t n_rows, int64_t n_cols, float * y, hipStream_t s);
void launch_pack_act_blocks(const act_view & a, int64_t M, int64_t K, void * blocks, hipStream_t s);
void launch_fill_zero(void * p, size_t bytes, hipStream_t s);
void launch_copy_f32(const float * src, float * dst, int64_t n, hipStream_t s);

// MFMA layout probe (test hook): D = A * B for 32x32x16 f16 with A [32][16], B [16][32] row-major f32
// inputs; writes D [32][32] using the register layout the GEMM epilogues assume.
void launch_mfma_probe(const float * a, const float * b, float * d, hipStream_t s);
// the q8_0 GEMM step from registers alone (jepa_amd_gemm_step_probe); sink: n_wg * 256 * waves_per_simd floats
void launch_step_probe(int mode, int waves_per_simd, int iters, int n_wg, float * sink, hipStream_t s);
