/*
 * jepa_amd.h - entry points of libjepa.so beyond the reference API (include/jepa.h).
 *
 * The reference has no counterpart for these; they exist for callers that keep data on the GPU
 * (benchmarks, pipelines feeding decoded frames from device memory) and for parity tests that check
 * one kernel at a time against the CPU oracle. Pointers named *_dev are HIP device pointers on the
 * given device; every call is synchronous (it returns after its kernels finished) unless stated.
 * Return values: >= 0 on success, -1 on failure with the reason in jepa_error_text().
 */
#pragma once
#include "jepa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- encoder on device-resident data -------------------------------------------------------- */
/* jepa_encode without the host copies: in_dev is the NCTHW float32 input already on the model's
 * device, out_dev receives [rows, embed_dim] float32 rows (same order as jepa_encode). Replaces the
 * host-side patchify + tensor_set / tensor_get of reference src/jepa.cpp:990-1019 with device data.
 * Returns the rows per item (jepa_token_grid) or -1. last_compute_ms is set as for jepa_encode. */
int64_t jepa_amd_encode_device(jepa_context * ctx, const float * in_dev, int n_batch, int n_chans, int n_frames,
                               int height, int width, float * out_dev, int64_t out_cap_floats);

/* jepa_head_ex on device-resident encoder rows: x_dev [n_tokens][embed_dim] float32 on the model's
 * device; pooled_dev [embed_dim] and logits_dev [n_classes] (device, either may be NULL) receive
 * the pooled token and the classifier logits. Replaces the tensor_set / tensor_get of reference
 * src/jepa.cpp:1093-1110 with device data. Returns n_classes, or -1 with the reason in
 * jepa_error_text(). last_compute_ms covers the head's kernels. */
int jepa_amd_head_device(jepa_context * ctx, const float * x_dev, int64_t n_tokens, float * pooled_dev, float * logits_dev);

/* jepa_encode that also returns the residual stream after the patch embedding and after every
 * block (before the final norm): trace [n_items][n_layer + 1][rows][dim] on the host. For per-layer
 * parity checks; runs without graph replay. */
int64_t jepa_amd_encode_trace(jepa_context * ctx, const jepa_input * in, float * out, int64_t out_cap_floats,
                              float * trace, int64_t trace_cap_floats);

/* ---- context knobs --------------------------------------------------------------------------- */
/* Record hipEvents around every kernel launch of the next encodes (disables graph replay) and sum
 * their device time per kernel class: "patchify", "patch_embed", "layernorm", "gemm_q8",
 * "gemm_q4k", "gemm_f16", "gemm_f32", "attention", "quantize", "cls". */
void jepa_amd_context_set_kernel_timing(jepa_context * ctx, bool on);
int  jepa_amd_context_kernel_stats(const jepa_context * ctx, const char * kernel_class, int64_t * n_launches, double * total_ms);
void jepa_amd_context_reset_kernel_stats(jepa_context * ctx);
/* Capture the forward into a hipGraph and replay it (default on; $JEPA_HIP_GRAPH=0 turns it off). */
void jepa_amd_context_set_graph(jepa_context * ctx, bool on);
/* The HIP stream (hipStream_t) the context launches on. */
void * jepa_amd_context_stream(const jepa_context * ctx);

/* ---- single-kernel hooks (parity tests, micro-benchmarks) ------------------------------------ */
/* ggml to_float of q8_0 / q4_0 / q4_K / f16 rows: blocks_dev holds n_rows rows of n_cols values in
 * the ggml block layout (ggml_type ids 8 / 2 / 12 / 1). */
int jepa_amd_dequantize(int device, int ggml_type, const void * blocks_dev, int64_t n_rows, int64_t n_cols, float * y_dev);

/* Row-wise LayerNorm (ggml_norm + optional affine, normalize = 1) or plain conversion (normalize = 0)
 * of x_dev [n_rows][n_cols], written as out_type: 0 f32 rows, 1 f16 rows, 8 q8_0 blocks (34 B per 32),
 * 15 q8_K blocks (292 B per 256) in ggml's block layout - the activation quantization the GEMMs
 * consume (x86 quantize_row_q8_0 / quantize_row_q8_K_ref semantics). */
int jepa_amd_rownorm(int device, const float * x_dev, int64_t n_rows, int64_t n_cols, const float * w_dev,
                     const float * b_dev, float eps, int normalize, int out_type, void * out_dev);

/* Y = X W^T (+ bias): W_dev in ggml blocks of wtype (8 q8_0, 2 q4_0, 12 q4_K, 1 f16, 0 f32) [n_out][n_in],
 * X_dev f32 [n_rows][n_in], Y_dev f32 [n_rows][n_out]; the activations are quantized to the weight's
 * vec-dot type first, like ggml_mul_mat (reference src/jepa.cpp:365-375). reps > 1 repeats the GEMM
 * (same result); *gemm_ms (optional) receives the mean device time of one GEMM launch. */
int jepa_amd_matmul(int device, int wtype, const void * w_dev, int64_t n_out, int64_t n_in, const float * bias_dev,
                    const float * x_dev, int64_t n_rows, float * y_dev, int reps, double * gemm_ms);

/* The MLP's first linear with its fused epilogue: out = gelu_erf(X W^T + bias) (reference
 * src/jepa.cpp:365-385), written the way the encoder hands it to the second linear. out_type 0 (f32):
 * out_dev f32 [n_rows][n_out]; 1 (f16): f16 values; 8 (q8_0) / 15 (q8_K): ggml blocks of the quantized
 * rows (q8_K needs n_out % 256 == 0). W, X, bias as for jepa_amd_matmul. reps > 1 repeats the GEMM
 * (same result); *gemm_ms (optional) receives the mean device time of one repeat. */
int jepa_amd_matmul_gelu(int device, int wtype, const void * w_dev, int64_t n_out, int64_t n_in, const float * bias_dev,
                         const float * x_dev, int64_t n_rows, int out_type, void * out_dev, int reps, double * gemm_ms);

/* Attention of one block from its fused qkv rows: qkv_dev f32 [n_items*n_tok][3*n_head*hd] (rows
 * [q | k | v], head-major), head width hd 64 or 32, optional RoPE tables rope_c/rope_s [n_tok][hd]
 * (signed sine). Runs the QKV epilogue's split/RoPE/f16 cast and the attention kernel. tokens_per_slot
 * > 0 applies the LeVJEPA block-causal mask (reference src/jepa.cpp:827-844): the n_prefix leading
 * rows read every key, a patch row reads the patch keys of its own and earlier temporal slots of
 * tokens_per_slot rows, and no prefix key; 0 is full attention. out_type 0 (f32): out_dev f32
 * [n_items*n_tok][n_head*hd]; 8 (q8_0): out_dev ggml q8_0 blocks of those rows, as the attention
 * kernel's fused epilogue quantizes them for the out-projection; 1 (f16, head widths 32 and 64):
 * out_dev f16 rows, the f32 values rounded to nearest, the input of an f16 out-projection. */
int jepa_amd_attention(int device, const float * qkv_dev, int64_t n_items, int64_t n_tok, int n_head, int hd,
                       const float * rope_c_dev, const float * rope_s_dev, int n_prefix, int64_t tokens_per_slot,
                       int out_type, void * out_dev);

/* jepa_preprocess_frames_rgb_ex on the device: n_frames RGB8 HWC frames of h x w, contiguous in device
 * memory ([n_frames][h][w][3]), are resized (uint8 antialias), centre-cropped and normalised into
 * out_dev, NCTHW f32 [3][n_frames][crop][crop] (N = 1), bit-identical to the host function. The clip
 * then goes to jepa_amd_encode_device without a host round trip, and only uint8 frames cross PCIe.
 * out_cap is out_dev's size in floats; out_h / out_w receive the crop. Returns 0, or -1 with the
 * reason in jepa_error_text(). Replaces the host half of reference src/preprocess.cpp:233-300. */
int jepa_amd_preprocess_frames_device(int device, const jepa_preprocess_params * p, const uint8_t * frames_dev, int n_frames, int h,
                                      int w, float * out_dev, int64_t out_cap, int * out_h, int * out_w);

/* jepa_amd_preprocess_frames_device without any allocation: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The tap tables and the horizontal-pass image live in a static
 * device array of 32 MiB that every GPU the library runs on holds until the process ends; a call
 * whose scratch would exceed it (about n_frames * h * crop * 3 bytes plus the tables) is refused
 * with -1 and a message. Work is queued on `stream` (a hipStream_t of `device`; NULL: the null
 * stream) and the call returns without waiting for it; the output is, bit for bit, that of
 * jepa_amd_preprocess_frames_device. Nothing is copied from host memory: the tables reach the
 * device as kernel arguments, so the call can be captured into a HIP graph (make one call on the
 * device before capturing, which looks up the array's address) and the graph replayed on new frames
 * of the same geometry. Calls on one GPU share the array: calls whose work overlaps on one GPU (on
 * different streams, or graph replays beside eager calls) race, and the caller orders them. */
int jepa_amd_preprocess_frames_device_noalloc(int device, const jepa_preprocess_params * p, const uint8_t * frames_dev, int n_frames,
                                              int h, int w, float * out_dev, int64_t out_cap, int * out_h, int * out_w, void * stream);

/* Split-K of the GEMMs with the residual or plain f32 epilogue (S workgroups per output tile, one per
 * K part; the last to finish adds the parts' sums in part order): q8_0 / q4_0 / q4_K run in 1 or 2
 * halves chosen from n_out and n_in only; f16 weights in 1 to 4 parts when the tiles leave most CUs
 * idle (few rows) and K >= 1024. jepa_amd_gemm_split forces S for later launches (1 = off; 2 for the
 * int8 / 4-bit types; 2, 3 or 4 for f16 where K allows, else unsplit) or restores the automatic choice (-1);
 * jepa_amd_gemm_split_of returns the halves of a q8_0 / q4_0 / q4_K GEMM of this shape (1 for f16,
 * whose parts depend on the row count; the other epilogues do not split). */
int jepa_amd_gemm_split(int split);
int jepa_amd_gemm_split_of(int wtype, int64_t n_out, int64_t n_in);

/* ---- GGUF quantizer ---------------------------------------------------------------------------
 * The reference's jepa-quantize (tools/jepa-quantize.cpp) as a library call: in_path (an f32 / f16
 * jepa GGUF, or a quantized one with allow_requant) -> out_path with the 2-D attention / FFN /
 * projection / classifier weights re-typed to `type` ("f32", "f16", "q8_0", "q4_0", "q4_k"; f32
 * widens every tensor), the same keep rule, per-tensor K-quant fallback to q4_0, metadata copied in
 * order with general.file_type updated, GGUF v3 with 32-byte alignment. Tensors whose name contains
 * one of the n_keep strings in `keep` keep their type. The block quantizers run on HIP device
 * `device` (-1: 0) and are bit-exact with ggml's reference quantizers. verbose logs the plan.
 * Returns 0, or -1 with the reason in jepa_error_text(). */
int jepa_amd_quantize_file(const char * in_path, const char * out_path, const char * type, const char * const * keep, int n_keep,
                           bool allow_requant, int device, bool verbose);

/* f32 values on the device -> ggml blocks of gtype (8 q8_0, 2 q4_0, 12 q4_K) or f16 (1), bit-exact
 * with ggml's reference quantizers (test hook of the quantizer kernels). n must be whole blocks. */
int jepa_amd_quantize_rows(int device, int gtype, const float * x_dev, int64_t n, void * out_dev);

/* One v_mfma_f32_32x32x16_f16 on host matrices a [32][16], b [16][32] -> d [32][32] (row-major),
 * written back through the accumulator layout the GEMM epilogues assume. */
int jepa_amd_mfma_probe(int device, const float * a, const float * b, float * d);

/* The 3-D RoPE tables this library uploads for an encoder (host only, no device work): [n_rows][head_dim]
 * cos and sin rows for grid (grid_t, grid_h, grid_w), variant 0 (V-JEPA 2, tiled) or 1 (V-JEPA 2.1,
 * interleaved), with the 2.1 interpolation to (train_h, train_w) when interpolate is set. ids (may
 * be NULL: every token, T-major) selects rows of the grid. signed_sin = 1 gives the sine table with
 * the rotation's sign on the even lanes, as the QKV epilogue reads it; 0 the plain sines. Replaces
 * nothing in the reference: it exposes the tables of reference src/rope3d.cpp:9-134 to the tests
 * that pin them against the reference's golden vectors. Returns 0, or -1 on a bad argument. */
int jepa_amd_rope_tables(int head_dim, int grid_t, int grid_h, int grid_w, int variant, int interpolate, int train_h, int train_w,
                         float theta, const int32_t * ids, int64_t n_rows, int signed_sin, float * cos_out, float * sin_out);

/* Throughput ceiling of the q8_0 GEMM's inner step from registers alone (no memory, no barriers), one
 * workgroup per CU with waves_per_simd (1-4) waves on each SIMD: per 32x32x32 block and MFMA tile one
 * int8 MFMA (the block sum), one f16 MFMA (the scale products) and 32 VALU ops (16 conversions, 16
 * fmas). mode 0: the whole step in each wave (the kernels' form); 1: the two MFMAs alone; 2: the VALU
 * ops alone; 3: even waves the MFMA half, odd waves the VALU half. *ns_per_step: nanoseconds of one SIMD
 * per whole step (65536 int8 ops). No counterpart in the reference: a measurement hook. */
int jepa_amd_gemm_step_probe(int device, int mode, int waves_per_simd, int iters, double * ns_per_step);

/* Copy of n float32 values between device buffers (a plain copy kernel, for counter calibration). */
int jepa_amd_copy(int device, const float * src_dev, float * dst_dev, int64_t n, int reps, double * ms);

/* Force the MFMA GEMM onto workgroup tile `index` for later launches whose n_out it divides; -1
 * restores the automatic choice. Process-wide (tests and tuning). Tiles (weight rows x tokens):
 * 0: 256x128, 1: 192x128, 2: 128x128, 3: 128x128 (other wave shape), 4: 64x128, 5: 128x64, 6: 256x64,
 * 7: 256x64 (other wave shape; only for the q8_K GELU epilogue), 8: 384x64 (4-bit q4_0 only). q4_K
 * weights run tiles 2, 3, 5, 6 and 7, 4-bit q4_0 (rows a multiple of 128) tiles 0, 2, 3, 5, 6, 7 and 8;
 * a tile a launch cannot take leaves that launch on the automatic choice.
 * Returns 0, or -1 for an index past the table. */
int jepa_amd_gemm_tile(int index);

#ifdef __cplusplus
}
#endif
