/*
 * gcq.h - C ABI of libgcq: gfx950 HIP kernels for the quantized mat-mul and KV-cache attention
 * path of ggml-compiler's programs (ggml_mul_mat on GGUF Q8_0 / Q4_0 / Q4_K (and Q5_K / Q6_K) blocks,
 * ggml_flash_attn_ext over an f16 cache, ggml_rms_norm, ggml_rope_ext and the decode step's glue).
 *
 * Plain C: device pointers, sizes and a hipStream_t passed as void* (NULL = the default stream).
 * Every int function returns 0 on success and -1 on failure, with gcq_last_error() describing it
 * (the convention of runtime/include/ggml_compiler_rt.h:9-11, thread-local as
 * runtime/src/ggml_compiler_rt.cpp:43-47). Size queries return 0 for arguments they reject.
 * Arguments are checked on the host before anything is launched.
 *
 * Type ids are GGUF's ggml_type values. Sizes follow ggml's naming: a weight has N rows of K
 * values (ggml ne = [K, N]); an activation has M (or B) rows of K values (ne = [K, M]); results
 * are M rows of N floats (ne = [N, M]).
 *
 * Device layouts: a weight is uploaded in ggml's block bytes and converted once by
 * gcq_pack_weights to the layout the kernels read (same byte count, rounded up to 256-byte
 * sections). Activations are quantized into a workspace by gcq_quantize_act or by gcq_mul_mat
 * itself.
 */
#ifndef GCQ_H
#define GCQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GCQ_API __attribute__((visibility("default")))

enum {
    GCQ_TYPE_F32 = 0,
    GCQ_TYPE_F16 = 1,
    GCQ_TYPE_Q4_0 = 2,
    GCQ_TYPE_Q8_0 = 8,
    GCQ_TYPE_Q4_K = 12,
    GCQ_TYPE_Q5_K = 13,
    GCQ_TYPE_Q6_K = 14,
    GCQ_TYPE_Q8_K = 15,
    GCQ_TYPE_I32 = 26,
};

GCQ_API const char * gcq_version(void);
GCQ_API const char * gcq_last_error(void);
/* Errors recorded by the calling thread so far: lets a caller of a void function (ggml_backend_tensor_set
 * and the like, whose ggml originals abort) see whether it failed. */
GCQ_API uint64_t gcq_error_count(void);
/* Number of gfx950 devices HIP reports (0 when none is present or HIP cannot start). */
GCQ_API int gcq_device_count(void);

/* ---- sizes ---------------------------------------------------------------------------------- */
/* ggml bytes of one row of n values (ggml_compiler_row_size, runtime/include/ggml_compiler_rt.h:88-89). */
GCQ_API size_t gcq_row_size(int type, int64_t n);
/* Bytes of a packed device weight of nrows x n_per_row. */
GCQ_API size_t gcq_weight_size(int type, int64_t nrows, int64_t n_per_row);
/* Bytes of B quantized activation rows of K values for a weight type. */
GCQ_API size_t gcq_act_size(int wtype, int64_t B, int64_t K);
/* Workspace gcq_mul_mat needs for M activation rows. */
GCQ_API size_t gcq_mul_mat_workspace(int wtype, int64_t M, int64_t K);
/* Workspace gcq_flash_attn_ext needs. */
GCQ_API size_t gcq_flash_attn_workspace(int Sq, int H, int Hkv, int Dv, int n_kv);

/* ---- quantization --------------------------------------------------------------------------- */
/* Encode f32 rows (device) in ggml's block bytes (device), exactly as ggml's reference encoders
 * (ggml_quantize_chunk without an importance matrix). Replaces the arithmetic behind
 * ggml_compiler_quantize (runtime/include/ggml_compiler_rt.h:83-87,
 * runtime/src/ggml_compiler_rt.cpp:859-876). Types: Q8_0, Q4_0, Q4_K, Q5_K, Q6_K (the storage types of
 * ggml_compiler/quant/types.py:6-19 this library computes with). */
GCQ_API int gcq_quantize(int type, const float * src, int64_t nrows, int64_t n_per_row, void * dst, void * stream);
/* ggml block rows (device) -> packed device weight. dst must hold gcq_weight_size bytes, 16-byte
 * aligned (src too for Q4_K / Q5_K). Replaces the weight upload of
 * runtime/src/ggml_compiler_rt.cpp:445-479 (:476). */
GCQ_API int gcq_pack_weights(int type, const void * src, int64_t nrows, int64_t n_per_row, void * dst, void * stream);
/* Packed weight -> f32 rows (ggml dequantize_row_*; bit-exact). */
GCQ_API int gcq_dequantize(int type, const void * w, int64_t nrows, int64_t n_per_row, float * dst, void * stream);
/* f32 rows x [B][ldx] -> the weight type's vec_dot_type (Q8_0 for Q4_0/Q8_0, Q8_K for the K-quants): the
 * src1 conversion ggml-cpu's mul_mat performs (canonical Q8_0 variant: x86 AVX2). */
GCQ_API int gcq_quantize_act(int wtype, const float * x, int64_t ldx, int64_t B, int64_t K, void * act, void * stream);
/* A quantized activation in ggml's block bytes (block_q8_0 / block_q8_K), for comparisons. */
GCQ_API int gcq_act_to_ggml(int wtype, const void * act, int64_t B, int64_t K, void * dst, void * stream);

/* ---- mul_mat -------------------------------------------------------------------------------- */
/* y[m][n] (row stride ldy) = sum_k W[n][k] x[m][k], x f32 [M][ldx]: ggml_mul_mat(W, x) with W a
 * packed Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K weight (runtime/src/ops.cpp:107-119 ->
 * runtime/include/ggml_compiler_ops.h:116-122). M <= 8: GEMV; M > 8: int8-MFMA GEMM (Q4_0 / Q8_0
 * per 32-value block, the K-quants per 256-value super-block). ws: gcq_mul_mat_workspace bytes,
 * 256-byte aligned. */
GCQ_API int gcq_mul_mat(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx, int64_t M,
                        float * y, int64_t ldy, void * ws, size_t ws_size, void * stream);
/* gcq_mul_mat without a workspace argument and without any device allocation. No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). The quantized activation lives in a static device
 * array of GCQ_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call whose
 * gcq_mul_mat_workspace(wtype, M, K) exceeds it fails with an error. Runs on the current device
 * (the stream must belong to it). Calls that overlap on one GPU share the array and race.
 * Results equal gcq_mul_mat's bit for bit. */
#define GCQ_NOALLOC_SCRATCH_BYTES (16u << 20)
GCQ_API int gcq_mul_mat_noalloc(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx,
                                int64_t M, float * y, int64_t ldy, void * stream);
/* The same with the activation already quantized (gcq_quantize_act, gcq_rms_norm_q8,
 * gcq_swiglu_q8); with res (M x N at row stride ldy, may be y itself) y = res + W x: the ggml_add of
 * a residual that follows the mul_mat, fused. */
GCQ_API int gcq_mul_mat_q(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y,
                          int64_t ldy, const float * res, void * stream);
/* The GEMV kernels' exact int32 block dot sums: out[b][n][blk] (Q4_0/Q8_0),
 * out[b][n][superblock][10] (Q4_K, Q5_K: 8 sub-block dots, sum sc*dot, sum m*bsums) or
 * out[b][n][superblock][17] (Q6_K: 16 sub-block sums of (q - 32) * x, sum sc * those). B <= 8. */
GCQ_API int gcq_block_isums(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t B,
                            int32_t * out, void * stream);
/* The GEMM's (MFMA) int32 sums of K-block blk: out[m][n] (Q4_0 / Q8_0, blk a 32-value block);
 * K-quants, blk a 256-value super-block: out[m][n][2] = {sum sc * dot, sum m * bsums} (Q4_K, Q5_K)
 * or out[m][n] = sum sc * dot (Q6_K), the same integers as gcq_block_isums' last one or two. */
GCQ_API int gcq_gemm_block_isums(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                                 int blk, int32_t * out, void * stream);

/* ---- attention ------------------------------------------------------------------------------ */
/* ggml_flash_attn_ext(q, k, v, mask, scale, 0, 0) with GGML_PREC_F32 on f16 K/V
 * (runtime/src/ops.cpp:217-243, runtime/include/ggml_compiler_ops.h:133-136).
 * q[h][s][d] f32 at element strides (q_h, q_s); k, v [hk][j][d] f16 at (k_h, k_j), (v_h, v_j);
 * mask [s][j] f16 at row stride m_s or NULL; out [s][h][Dv] f32. D = Dv in {64, 128, 256},
 * H / Hkv <= 8. ws: gcq_flash_attn_workspace bytes. */
GCQ_API int gcq_flash_attn_ext(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                               const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, float * out,
                               int D, int Dv, int Sq, int H, int Hkv, int n_kv, float scale, void * ws, size_t ws_size,
                               void * stream);

/* ---- norms, rope, glue ---------------------------------------------------------------------- */
/* ggml_rms_norm(x, eps) over rows of n (runtime/src/ops.cpp:144-148); w (n floats) or NULL: the
 * ggml_mul by a norm weight that follows it, fused. */
GCQ_API int gcq_rms_norm(const float * x, int64_t ldx, float * y, int64_t ldy, const float * w, int64_t rows,
                         int64_t n, float eps, void * stream);
/* One row x [K]: ggml_rms_norm (eps) -> ggml_mul by the norm weight norm_w [K] -> ggml_mul_mat by
 * the packed Q4_0 / Q8_0 weight w [N][K], the three nodes every decoder layer feeds its QKV and
 * gate/up projections with (ggml_compiler/llm.py:369-373, 421-425), into y [N] (y = res + W x' when
 * res is given). For K <= 16384 one launch: the GEMV workgroups normalize and quantize x
 * themselves (ws unused, may be NULL); otherwise gcq_rms_norm_q8 into ws
 * (gcq_mul_mat_workspace(wtype, 1, K) bytes) then the GEMV. y equals gcq_rms_norm_q8 + gcq_mul_mat_q bit for bit; with norm_w NULL
 * the norm is skipped and y equals gcq_mul_mat's. */
GCQ_API int gcq_rms_norm_mul_mat(int wtype, const void * w, int64_t N, int64_t K, const float * x, const float * norm_w,
                                 float eps, float * y, const float * res, void * ws, size_t ws_size, void * stream);
/* ggml_rms_norm + ggml_mul by w + the Q8_0 conversion a following mul_mat makes of its src1, fused:
 * act (gcq_act_size(GCQ_TYPE_Q4_0, rows, n) bytes) holds what gcq_quantize_act makes of
 * gcq_rms_norm's output, byte for byte. n % 32 == 0. */
GCQ_API int gcq_rms_norm_q8(const float * x, int64_t ldx, const float * w, int64_t rows, int64_t n, float eps,
                            void * act, void * stream);
/* ggml_swiglu_split(g, u) + the Q8_0 conversion of the next mul_mat's src1, fused (rows of n at row
 * stride ld for g and u). Equal byte for byte to gcq_quantize_act of gcq_swiglu's output. */
GCQ_API int gcq_swiglu_q8(const float * g, const float * u, int64_t ld, int64_t rows, int64_t n, void * act,
                          void * stream);
/* ggml_rope_ext(x, pos, ff, n_dims, mode=NEOX, 0, base, freq_scale, 0, attn_factor, 32, 1)
 * (runtime/src/ops.cpp:277-291). x[s][h][d] at (sx_s, sx_h), out[s][h][d] at (so_s, so_h); may
 * be the same memory. ff: n_dims/2 floats or NULL. */
GCQ_API int gcq_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, int64_t so_s, int64_t so_h,
                          const int32_t * pos, int64_t D, int64_t H, int64_t S, int n_dims, float freq_base,
                          float freq_scale, float attn_factor, const float * ff, void * stream);
/* ggml_set_rows into an f16 cache (runtime/src/ops.cpp:260-275):
 * dst[h][idx[j]][d] = f16(src[h][j][d]), j < n, h < Hrows, d < D (D % 8 == 0). dst has dst_rows
 * rows per head; an index outside [0, dst_rows) writes nothing. */
GCQ_API int gcq_set_rows_f16(void * dst, int64_t dst_h, int64_t dst_j, const float * src, int64_t src_h,
                             int64_t src_j, const int32_t * idx, int64_t n, int64_t D, int64_t Hrows, int64_t dst_rows,
                             void * stream);
/* ggml_get_rows (runtime/src/ops.cpp:302-309): out[j][:] = row idx[j] of a table of nrows x D
 * (F32, F16, a packed Q4_0 / Q8_0 / Q6_K weight or Q4_K / Q5_K super-blocks), as f32, each element as
 * ggml's dequantize_row_* gives it; an index outside the table gives NaNs. */
GCQ_API int gcq_get_rows(int type, const void * table, int64_t nrows, int64_t D, const int32_t * idx, int64_t n,
                         float * out, void * stream);
/* ggml_swiglu_split(g, u) = silu(g) * u (runtime/src/ops.cpp:251-258). */
GCQ_API int gcq_swiglu(const float * g, const float * u, float * y, int64_t n, void * stream);
/* ggml_add / ggml_mul: y[i] = a[i] op b[i % nb]. */
GCQ_API int gcq_add(const float * a, const float * b, float * y, int64_t n, int64_t nb, void * stream);
GCQ_API int gcq_mul(const float * a, const float * b, float * y, int64_t n, int64_t nb, void * stream);
/* ggml_argmax of each row (runtime/src/ops.cpp:293-300): the first index of the maximum. */
GCQ_API int gcq_argmax(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, void * stream);

/* ---- synthetic data ------------------------------------------------------------------------- */
/* Deterministic streams (counter-based splitmix64): approximately N(0, stddev^2) floats and
 * uniform token ids, element i from (seed, offset + i). */
GCQ_API int gcq_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev, void * stream);
GCQ_API int gcq_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab, void * stream);

/* ---- measurement ---------------------------------------------------------------------------- */
/* No counterpart in the reference: for benchmarks that set a kernel's time against the fastest
 * one-launch read of the same bytes. Reads `bytes` (a multiple of 16) at src (16-byte aligned) once
 * with waves_per_cu (4, 8, 16 or 32) wavefronts per CU, each reading a contiguous range with
 * `unroll` (1, 2 or 4) 1 KiB loads in flight; computes nothing (sink, a device word, is written
 * only in the unlikely case that the XOR of the words equals a constant). */
GCQ_API int gcq_stream_read(const void * src, size_t bytes, int waves_per_cu, int unroll, uint32_t * sink,
                            void * stream);

/* ---- Llama-style causal LM ------------------------------------------------------------------ */
/* The program ggml-compiler's causal_lm compiles (ggml_compiler/llm.py:361-444) on libgcq's
 * kernels: GQA attention over an f16 KV cache, SwiGLU FFN, RMSNorm, NEOX RoPE, every matmul weight
 * Q4_0 or Q8_0 (q/k/v and gate/up stored row-stacked). Its entry points are prefill, decode and
 * an on-device greedy generate (llm.py:12-14, :421-436); the KV cache is state, zeroed at creation
 * and by gcq_llama_reset (ggml_compiler_reset, runtime/include/ggml_compiler_rt.h:112-113). */
typedef struct {
    int   n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, max_ctx;
    int   wtype; /* GCQ_TYPE_Q4_0 or GCQ_TYPE_Q8_0 */
    float rms_eps, rope_base;
} gcq_llama_config;
typedef struct gcq_llama gcq_llama;

/* Allocates weights (norm weights 1, matmul weights unset), KV cache and buffers for prompt chunks
 * of up to max_prompt tokens. NULL on failure. */
GCQ_API gcq_llama * gcq_llama_create(const gcq_llama_config * cfg, int max_prompt);
GCQ_API void        gcq_llama_free(gcq_llama * m);
/* Every matmul weight and the embedding ~N(0, stddev^2), weight i drawn from gcq_fill_normal's
 * stream with seed + i, encoded on the GPU exactly as ggml's reference encoder. */
GCQ_API int gcq_llama_init_random(gcq_llama * m, uint64_t seed, float stddev);
/* Weights in order: token_embd, per layer blk.L.{attn_norm, attn_qkv, attn_output, ffn_norm,
 * ffn_gate_up, ffn_down}, output_norm, output. type: GCQ_TYPE_F32 (norms) or the weight type. */
GCQ_API int gcq_llama_n_weights(const gcq_llama * m);
GCQ_API int gcq_llama_weight_info(const gcq_llama * m, int i, const char ** name, int * type, int64_t * rows,
                                  int64_t * cols);
/* Load / read one weight as host ggml block bytes (f32 for norms); nbytes must match exactly
 * (the weight upload of runtime/src/ggml_compiler_rt.cpp:445-479). */
GCQ_API int gcq_llama_set_weight(gcq_llama * m, const char * name, const void * data, size_t nbytes);
GCQ_API int gcq_llama_get_weight(const gcq_llama * m, const char * name, void * data, size_t nbytes);
/* Zero the KV cache and return to position 0. */
GCQ_API int gcq_llama_reset(gcq_llama * m);
/* Tokens in the context so far. */
GCQ_API int gcq_llama_position(const gcq_llama * m);
/* Append n tokens (any n; chunks of max_prompt); logits (n_vocab floats, host) of the last one, or NULL. */
GCQ_API int gcq_llama_prefill(gcq_llama * m, const int32_t * tokens, int n, float * logits);
/* Append one token through the captured decode step; its logits and / or greedy next token (host). */
GCQ_API int gcq_llama_decode(gcq_llama * m, int32_t token, float * logits, int32_t * next);
/* Feed `first`, then each greedy token back, n_new steps on the device; out_tokens (host) gets the
 * n_new tokens produced (no end-of-sequence stop). */
GCQ_API int gcq_llama_generate(gcq_llama * m, int32_t first, int n_new, int32_t * out_tokens);
/* Layers [first_layer, first_layer + n_layers) on n given residual-stream rows x (host, n x n_embd
 * f32) at positions pos .. pos + n - 1: the kernels a prompt chunk (n > 1, n <= max_prompt) or the
 * decode step (n == 1) runs, K / V of those layers written into the cache at those positions.
 * x_out (host, n x n_embd) gets the last layer's output; x_mid (host, n_layers x n x n_embd, or
 * NULL) each layer's rows after attention (x + attention, before the FFN). The position that
 * prefill / decode continue from is not changed. For layer-by-layer comparisons of the decoder
 * (the per-layer graph of ggml_compiler/llm.py:361-444) against a reference fed the same rows. */
GCQ_API int gcq_llama_forward_layers(gcq_llama * m, const float * x, int n, int pos, int first_layer, int n_layers,
                                     float * x_out, float * x_mid);

#ifdef __cplusplus
}
#endif

#endif /* GCQ_H */
