/*
 * oracle.h - CPU restatement of the jepa.cpp encoder path with ggml's CPU semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libjepa.so, bench.py's measured leg) links or
 * calls this; it is the checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use. It restates, in plain C, what the reference computes through ggml @36da5713 on the CPU:
 *
 *   - ggml block formats Q8_0 / Q4_0 / Q4_K / Q8_K (ggml-common.h layouts) and their dequantization
 *   - weight quantizers (quantize_row_q8_0_ref / q4_0_ref style) used to write fixtures
 *   - activation quantization as the x86 CPU backend does it inside mul_mat:
 *       q8_0: d = amax/127 stored f16, q = round_half_even(x * (127/amax))   (AVX2 quantize_row_q8_0)
 *       q8_K: iscale = -127/max, q = min(127, nearest_int(iscale*x)), d = 1/iscale (f32), bsums
 *   - per-block integer dots with float scale epilogues (vec_dot_q8_0_q8_0, q4_0_q8_0, q4_K_q8_K)
 *   - F16 weights: activations rounded to F16, f32 accumulation (docs/parity.md:151-154)
 *   - ggml_norm (two-pass, centred variance), gelu_erf, flash attention with F32 Q and F16 K/V
 *   - the 3-D RoPE tables and x*C + swap(x)*S' application (src/rope3d.cpp:9-164)
 *   - the encoder graphs of src/jepa.cpp:444-471 (block), 586-627 (image), 846-895 (video)
 *
 * Each function cites the reference file:line it follows. Pinning of each part is listed in the
 * test files (tests/test_oracle_*.py): golden RoPE vectors, closed forms, invariants and
 * double-precision references.
 */
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (ggml_type) as stored in GGUF tensor infos */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q8_K = 15 };

uint16_t or_fp32_to_fp16(float f);
float    or_fp16_to_fp32(uint16_t h);
void     or_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n);
void     or_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n);

/* bytes of one row of n elements of a type (0 if n is not a multiple of the block) */
size_t or_row_size(int type, int64_t n);

/* weight quantizers (ggml *_ref formulas); q4_K uses this oracle's own min/max search */
void or_quantize_q8_0_ref(const float * x, void * blocks, int64_t n);
void or_quantize_q4_0_ref(const float * x, void * blocks, int64_t n);
void or_quantize_q4_K(const float * x, void * blocks, int64_t n);
float or_make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                          float rmin, float rdelta, int nstep);
/* activation quantizers as the x86 CPU backend runs them inside mul_mat */
void or_quantize_q8_0_act(const float * x, void * blocks, int64_t n);
void or_quantize_q8_K_act(const float * x, void * blocks, int64_t n);

void or_dequantize(int type, const void * blocks, float * y, int64_t n);

/* dot of one weight row (type) with one activation row already in the matching vec-dot type */
float or_vec_dot(int wtype, int64_t n, const void * wrow, const void * arow);

/* Y[m, o] = sum_k W[o, k] X[m, k] (+ bias[o]); W rows in `wtype` blocks, X f32.
 * Activation conversion follows the weight type exactly as ggml_compute_forward_mul_mat does. */
int or_mul_mat(int wtype, const void * w, int64_t n_out, int64_t n_in,
               const float * x, int64_t n_rows, const float * bias, float * y, int n_threads);

/* 1: sum the per-block terms of quantized dots from the last K-block to the first (see oracle.c) */
void or_set_reverse_block_order(int on);
void or_set_k_split(int s);
/* 1: quantized dots summed in ggml's x86 lane order (AVX2 vec_dot / llamafile tinyBLAS), 0: one chain */
void or_set_ggml_lanes(int on);
int  or_get_ggml_lanes(void);
/* 1: with f16 K/V, round q and the softmax weights to f16 too (an f16 matrix-core attention) */
void or_set_attn_f16(int on);
/* rounding switches (bits: 1 f16 q, 2 f16 softmax weights, 4 exp2 form, 8 GPU erf polynomial) */
void or_set_rounding(int bits);
int  or_get_rounding(void);
/* teacher forcing of the encoder: block l starts from trace entry l (NULL: off) */
void or_set_teacher(const float * trace, int64_t n_floats);
/* teacher forcing only: blocks before l0 are skipped (their trace entries are the teacher's) */
void or_set_first_block(int l0);

void or_layer_norm(const float * x, int64_t n_rows, int64_t d, const float * w, const float * b,
                   float eps, float * y);
float or_gelu_erf(float x);
void or_gelu_erf_n(const float * x, float * y, int64_t n);

typedef struct {
    int   grid_t, grid_h, grid_w, head_dim;
    float theta;
    int   interpolate, train_grid_h, train_grid_w;
    int   variant;   /* 0 tiled (V-JEPA 2), 1 interleaved (V-JEPA 2.1) */
} or_rope_params;

/* [n_rows, head_dim] tables; ids == NULL means rows 0..n-1 of the full grid */
void or_rope_tables(const or_rope_params * p, const int32_t * ids, int64_t n_rows,
                    float * cos_out, float * sin_out, int signed_sin);
/* x [n_tok, n_head, head_dim] in place: x*C + swap(x)*S' with the signed table */
void or_rope_apply(float * x, int64_t n_tok, int n_head, int head_dim, const float * cos_t, const float * sin_t);

/* softmax(q k^T * scale + mask) v per head. q f32 [n_q, n_head*hd] rows, k/v [n_kv, n_head*hd]; when
 * kv_f16 the K/V values are rounded to f16 first (ggml_cast). mask (optional): additive [n_q][n_kv]
 * (0 / -inf), the flash_attn_ext mask argument; a row with no visible key gives zeros. Output
 * [n_q, n_head*hd]. */
void or_attention(const float * q, const float * k, const float * v, int64_t n_q, int64_t n_kv,
                  int n_head, int hd, float scale, int kv_f16, const float * mask, float * out, int n_threads);

/* LeVJEPA block-causal mask [N][N], N = n_prefix + gt*gh*gw (src/jepa.cpp:827-844): 0 where query i
 * sees key j, -inf elsewhere. Prefix rows see every key; a patch query sees the patch keys of its own
 * and earlier temporal slots and no prefix key. */
void or_block_causal_mask(int gt, int gh, int gw, int n_prefix, float * out);

/* Encoder forward of a GGUF file on NCTHW input (what jepa_encode returns).
 * trace (optional): [n_items][n_layer + 1][rows][D] residual stream after the patch embedding /
 * prefix tokens and after every block (before the final norm). Returns rows written per item, or
 * -1 on error (message on stderr). */
int64_t or_encode_file(const char * gguf_path, const float * in, int n_batch, int n_chans, int n_frames,
                       int height, int width, float * out, int64_t out_cap_floats,
                       float * trace, int64_t trace_cap_floats, int n_layers_limit, int n_threads);

/* Attentive-pool head of a GGUF file on encoder rows x [N][D] (what jepa_head_ex returns): pooled
 * [D] and logits [n_classes] (either may be NULL). Returns n_classes, or -1 on error. */
int64_t or_head_file(const char * gguf_path, const float * x, int64_t n_tokens, float * pooled, float * logits,
                     int64_t logits_cap, int n_threads);

/* Masked predictor of a GGUF file (what jepa_predict_mod returns): encoder rows enc [n_tok][enc_dim],
 * context ids (NULL: 0..n_ctx-1, rows of enc) and target ids (NULL: 0..n_tgt-1), modality 1 video /
 * 2 image. out [n_tgt][out_dim]. Returns out_dim, or -1. */
int64_t or_predict_file(const char * gguf_path, const float * enc, int64_t n_tok, const int32_t * ctx_ids, int n_ctx,
                        const int32_t * tgt_ids, int n_tgt, int mask_index, int modality, float * out, int64_t out_cap,
                        int n_threads);

#ifdef __cplusplus
}
#endif
