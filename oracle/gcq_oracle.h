/*
 * gcq_oracle.h - CPU oracle for the quantized mat-mul / KV-cache attention path.
 *
 * TEST INFRASTRUCTURE. This library is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The product path
 * (libgcq.so, HIP kernels for gfx950) neither links nor calls anything here.
 *
 * It restates, in plain C, the CPU semantics of the ggml calls that ggml-compiler's runtime
 * issues for this path (runtime/src/ops.cpp:107-119 mul_mat, :144-148 rms_norm, :217-243
 * flash_attn, :260-275 set_rows, :277-291 rope, :302-309 get_rows) and of the weight encoder
 * behind ggml_compiler_quantize (runtime/src/ggml_compiler_rt.cpp:859-876). ggml itself
 * (llama.cpp b11223, runtime/CMakeLists.txt:18) is a fetched dependency that is absent here; the
 * algorithms follow ggml's published ggml-quants.c / ggml-cpu semantics as restated per function
 * in gcq_oracle.c.
 *
 * Type ids are GGUF's: F32=0, F16=1, Q4_0=2, Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14, Q8_K=15.
 */
#ifndef GCQ_ORACLE_H
#define GCQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15 };

/* Activation (vec_dot_type) Q8_0 quantizer variants. */
enum { ORC_ACT_Q8_0_AVX2 = 0, ORC_ACT_Q8_0_SCALAR = 1 };

uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_n(const float * x, uint16_t * y, int64_t n);
void     orc_fp16_to_fp32_n(const uint16_t * x, float * y, int64_t n);

/* Deterministic synthetic data (same stream as the product's GPU generator). */
uint64_t orc_rnd64(uint64_t seed, uint64_t i);
void     orc_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev);
void     orc_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab);

size_t orc_block_size(int type);
size_t orc_type_size(int type);
size_t orc_row_size(int type, int64_t n);

/* Weight encoders (ggml reference encoders, no importance matrix). Return bytes written or 0. */
size_t orc_quantize(int type, const float * src, int64_t nrows, int64_t n_per_row, void * dst);
/* The K-quant searches of one sub-block (make_qkx2_quants for Q4_K / Q5_K, make_qx_quants for Q6_K):
 * codes L, the returned scale and (qkx2) the negated min; for tests of the search's choice. */
float orc_make_qkx2(const float * x, const float * w, uint8_t * L, float * the_min, int nmax, float rmin, int nstep,
                    float * trace);
float orc_make_qx16(const float * x, uint8_t * L);
/* Activation quantizers: Q8_0 (variant ORC_ACT_*) or Q8_K, k values. */
void   orc_quantize_act_q8_0(const float * x, void * y, int64_t k, int variant);
void   orc_quantize_act_q8_K(const float * x, void * y, int64_t k);
/* Dequantize whole rows of a weight type (Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, F32) to f32. */
int    orc_dequantize(int type, const void * src, float * dst, int64_t nrows, int64_t n_per_row);

/* Integer block dot sums of one weight row against one quantized activation row.
 * Q4_0, Q8_0 (activation Q8_0): one int32 per 32-block.
 * Q4_K, Q5_K (activation Q8_K): per 256-superblock 10 int32: the 8 sub-block sums sum_l q*q8,
 * then sum_j sc_j*dot_j, then sum_j m_j*(bsums[2j]+bsums[2j+1]).
 * Q6_K (activation Q8_K): per 256-superblock 17 int32: the 16 sub-block sums sum_l (q-32)*q8,
 * then sum_j sc_j*those. Returns the count written. */
int64_t orc_block_isums(int type, const void * w_row, const void * xq_row, int64_t k, int32_t * out);

/* y[m, n] = sum_k w[n, k] * x[m, k]: w is N rows of a weight type in ggml layout, x f32 [M, K]
 * quantized to the weight's vec_dot type first (Q8_0 canonical variant, or Q8_K for the K-quants). */
int orc_mul_mat(int type, const void * w, int64_t N, int64_t K, const float * x, int64_t M, float * y,
                int n_threads);

/* ggml_rms_norm over rows of n: y = x / sqrt(mean(x^2) + eps). */
void orc_rms_norm(const float * x, float * y, int64_t rows, int64_t n, float eps, int n_threads);

/* ggml_rope_ext, NEOX mode (2), ext_factor 0. x[s][h][d] at element strides (sx_s, sx_h, 1);
 * out contiguous [S][H][D]. freq_factors may be NULL. */
void orc_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, const int32_t * pos, int64_t D,
                   int64_t H, int64_t S, int n_dims, float freq_base, float freq_scale, float attn_factor,
                   const float * freq_factors);

/* ggml_flash_attn_ext with f16 K/V, f32 accumulation. q[h][s][d] f32 at strides (q_h, q_s, 1);
 * k[hk][j][d], v[hk][j][d] f16 at strides (k_h, k_j, 1), (v_h, v_j, 1); mask[s][j] f16 at row
 * stride m_s (NULL = none); out [Sq][H][Dv] f32. Query head h reads KV head h / (H / Hkv). */
void orc_flash_attn_ext(const float * q, int64_t q_h, int64_t q_s, const uint16_t * k, int64_t k_h, int64_t k_j,
                        const uint16_t * v, int64_t v_h, int64_t v_j, const uint16_t * mask, int64_t m_s, float * out,
                        int D, int Dv, int Sq, int H, int Hkv, int n_kv, float scale, int n_threads);

/* Glue ops of a decoder step. */
void orc_swiglu(const float * g, const float * u, float * y, int64_t n);  /* silu(g) * u */
int  orc_argmax(const float * x, int64_t n);                              /* first max */

#ifdef __cplusplus
}
#endif

#endif
