/*
 * ggml.h - the part of ggml's graph-building API that ggml-compiler's generated stage builders and
 * runtime dispatcher call on the quantized decode / prefill path, provided by libgcq.
 *
 * The builders (ggml_compiler/emit/cpp.py:63-122) and the runtime's op dispatcher
 * (runtime/src/ops.cpp:107-309) construct ggml graphs node by node; this header keeps ggml's names,
 * argument order, tensor fields (type, ne, nb, op, op_params, src, view_src, view_offs, data, name)
 * and type ids (GGUF's ggml_type values), so that such code compiles against it unchanged.
 * Graphs are executed by the HIP backend of ggml-backend.h (ggml_backend_hip_init), which runs the
 * nodes on libgcq's gfx950 kernels.
 *
 * Differences from ggml, all on failure paths: a constructor given operands it cannot combine
 * returns NULL and records the reason (ggml_last_error(), the same text as gcq_last_error())
 * where ggml would abort; a NULL operand propagates as NULL; ggml_build_forward_expand ignores a
 * NULL tensor and the graph then fails to compute with that reason. Tensor metadata lives on the
 * host heap (mem_size is accepted and not enforced); no_alloc = false gives tensors host memory, as
 * in ggml, which the HIP backend does not compute on.
 */
#ifndef GGML_H
#define GGML_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#define GGML_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS           4
#define GGML_MAX_SRC            10
#define GGML_MAX_OP_PARAMS      64
#define GGML_MAX_NAME           64
#define GGML_DEFAULT_GRAPH_SIZE 2048
#define GGML_ROPE_TYPE_NEOX     2

/* GGUF type ids (the values ggml-compiler's GGUF files store). */
enum ggml_type {
    GGML_TYPE_F32  = 0,
    GGML_TYPE_F16  = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q2_K = 10,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_I8   = 24,
    GGML_TYPE_I16  = 25,
    GGML_TYPE_I32  = 26,
    GGML_TYPE_I64  = 27,
    GGML_TYPE_F64  = 28,
    GGML_TYPE_BF16 = 30,
    GGML_TYPE_COUNT = 40,
};

enum ggml_prec {
    GGML_PREC_DEFAULT = 0,
    GGML_PREC_F32     = 10,
};

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED       = -1,
    GGML_STATUS_SUCCESS      = 0,
    GGML_STATUS_ABORTED      = 1,
};

/* The ops this library builds (ggml's names; the numbering is this library's own). */
enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_ADD,
    GGML_OP_MUL,
    GGML_OP_SCALE,
    GGML_OP_CPY,
    GGML_OP_CONT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_GET_ROWS,
    GGML_OP_SET_ROWS,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_ROPE,
    GGML_OP_FLASH_ATTN_EXT,
    GGML_OP_ARGMAX,
    GGML_OP_GLU,
    GGML_OP_UNARY,
    GGML_OP_SOFT_MAX,
    GGML_OP_IM2COL,
    GGML_OP_CONV_2D_DIRECT,
    GGML_OP_SUB,
    GGML_OP_DIV,
    GGML_OP_NORM,
    GGML_OP_SUM_ROWS,
    GGML_OP_MEAN,
    GGML_OP_REPEAT,
    GGML_OP_CONCAT,
    GGML_OP_COUNT,
};

enum ggml_unary_op {
    GGML_UNARY_OP_ABS      = 0,
    GGML_UNARY_OP_NEG      = 1,
    GGML_UNARY_OP_TANH     = 2,
    GGML_UNARY_OP_RELU     = 3,
    GGML_UNARY_OP_SIGMOID  = 4,
    GGML_UNARY_OP_GELU     = 7,
    GGML_UNARY_OP_SILU     = 10,
    GGML_UNARY_OP_EXP      = 11,
    GGML_UNARY_OP_GELU_ERF = 12,
    GGML_UNARY_OP_SOFTPLUS = 13,
    /* ggml has these as ops of their own; kept under UNARY here */
    GGML_UNARY_OP_SQR  = 100,
    GGML_UNARY_OP_SQRT = 101,
    GGML_UNARY_OP_LOG  = 102,
    GGML_UNARY_OP_SIN  = 103,
    GGML_UNARY_OP_COS  = 104,
    GGML_UNARY_OP_CLAMP = 105, /* ggml's clamp op: op_params[1] min, [2] max */
};

enum ggml_glu_op {
    GGML_GLU_OP_SWIGLU = 2,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT  = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
    GGML_TENSOR_FLAG_PARAM  = 4,
};

struct ggml_backend_buffer;
struct ggml_context;
struct ggml_cgraph;

struct ggml_tensor {
    enum ggml_type               type;
    struct ggml_backend_buffer * buffer;
    int64_t                      ne[GGML_MAX_DIMS]; /* elements, innermost first */
    size_t                       nb[GGML_MAX_DIMS]; /* strides in bytes */
    enum ggml_op                 op;
    int32_t                      op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t                      flags;
    struct ggml_tensor *         src[GGML_MAX_SRC];
    struct ggml_tensor *         view_src; /* the tensor owning the memory of a view */
    size_t                       view_offs;
    void *                       data;
    char                         name[GGML_MAX_NAME];
    void *                       extra; /* backend-private */
};

struct ggml_init_params {
    size_t mem_size;
    void * mem_buffer;
    bool   no_alloc;
};

GGML_API const char * ggml_last_error(void);

/* ---- context, types, shapes ----------------------------------------------------------------- */
GGML_API struct ggml_context * ggml_init(struct ggml_init_params params);
GGML_API void                  ggml_free(struct ggml_context * ctx);
GGML_API size_t                ggml_tensor_overhead(void);
GGML_API size_t                ggml_graph_overhead(void);
GGML_API size_t                ggml_graph_overhead_custom(size_t size, bool grads);

GGML_API size_t       ggml_type_size(enum ggml_type type);
GGML_API int64_t      ggml_blck_size(enum ggml_type type);
GGML_API size_t       ggml_row_size(enum ggml_type type, int64_t ne);
GGML_API const char * ggml_type_name(enum ggml_type type);
GGML_API bool         ggml_is_quantized(enum ggml_type type);
GGML_API const char * ggml_op_name(enum ggml_op op);
GGML_API const char * ggml_op_desc(const struct ggml_tensor * t);

GGML_API int64_t ggml_nelements(const struct ggml_tensor * t);
GGML_API int64_t ggml_nrows(const struct ggml_tensor * t);
GGML_API size_t  ggml_nbytes(const struct ggml_tensor * t);
GGML_API bool    ggml_is_contiguous(const struct ggml_tensor * t);
GGML_API bool    ggml_is_transposed(const struct ggml_tensor * t);
GGML_API bool    ggml_is_permuted(const struct ggml_tensor * t);
GGML_API bool    ggml_is_vector(const struct ggml_tensor * t);
GGML_API bool    ggml_is_matrix(const struct ggml_tensor * t);
GGML_API bool    ggml_are_same_shape(const struct ggml_tensor * a, const struct ggml_tensor * b);
GGML_API bool    ggml_can_repeat(const struct ggml_tensor * a, const struct ggml_tensor * b);

/* ---- tensors -------------------------------------------------------------------------------- */
GGML_API struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims,
                                              const int64_t * ne);
GGML_API struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                 int64_t ne1);
GGML_API struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                 int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                                 int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor * ggml_set_name(struct ggml_tensor * t, const char * name);
GGML_API const char *         ggml_get_name(const struct ggml_tensor * t);
GGML_API struct ggml_tensor * ggml_get_tensor(struct ggml_context * ctx, const char * name);
GGML_API struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx);
GGML_API struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * t);
GGML_API void                 ggml_set_input(struct ggml_tensor * t);
GGML_API void                 ggml_set_output(struct ggml_tensor * t);

/* ---- views (no data of their own) ----------------------------------------------------------- */
GGML_API struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                           size_t offset);
GGML_API struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                           int64_t ne1, size_t nb1, size_t offset);
GGML_API struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                           int64_t ne1, int64_t ne2, size_t nb1, size_t nb2, size_t offset);
GGML_API struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                           int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1, size_t nb2,
                                           size_t nb3, size_t offset);
GGML_API struct ggml_tensor * ggml_view_tensor(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_reshape(struct ggml_context * ctx, struct ggml_tensor * a,
                                           struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0);
GGML_API struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                              int64_t ne1);
GGML_API struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                              int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0,
                                              int64_t ne1, int64_t ne2, int64_t ne3);
/* Source dim i becomes result dim axis_i. */
GGML_API struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1,
                                           int axis2, int axis3);
GGML_API struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a);

/* ---- ops ------------------------------------------------------------------------------------ */
/* Each replaces the ggml call the reference's dispatcher makes for that IR op (runtime/src/ops.cpp,
   lines cited per call) and that its generated builders make (ggml_compiler/emit/cpp.py:63-122). */
/* a contiguous copy of a (its type) / a in b's type and shape (into b's memory) / a in another type
   (ops.cpp:101 cont, :344-348 cast) */
GGML_API struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type);
/* a + b, a - b, a * b, a / b, b repeated over a (ggml_can_repeat; ops.cpp:56-64,76-79) */
GGML_API struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_div(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
/* Elementwise f(a) of a contiguous f32 tensor (ops.cpp:81-100): gelu is the tanh form
   0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), gelu_erf 0.5 x (1 + erf(x / sqrt 2)), silu
   x / (1 + e^-x), softplus log(1 + e^x) (x itself above 20). */
GGML_API struct ggml_tensor * ggml_gelu(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_gelu_erf(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_silu(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_relu(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_tanh(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_sigmoid(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_exp(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_log(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_neg(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_abs(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_sqr(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_sqrt(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_sin(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_cos(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_softplus(struct ggml_context * ctx, struct ggml_tensor * a);
/* min(max(a, min), max) elementwise (ops.cpp clamp) */
GGML_API struct ggml_tensor * ggml_clamp(struct ggml_context * ctx, struct ggml_tensor * a, float min, float max);
/* (x - mean) / sqrt(var + eps) per row of a contiguous f32 tensor, no affine (ops.cpp norm) */
GGML_API struct ggml_tensor * ggml_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
/* sum / mean of each row of a contiguous f32 tensor -> [1, ne1, ne2, ne3] (ops.cpp:81-100's
   mean and sum_rows) */
GGML_API struct ggml_tensor * ggml_sum_rows(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_mean(struct ggml_context * ctx, struct ggml_tensor * a);
/* a tiled to [ne0, ne1, ne2, ne3] (each a multiple of a's; ops.cpp repeat) */
GGML_API struct ggml_tensor * ggml_repeat_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                             int64_t ne2, int64_t ne3);
/* a then b along dim (0-3), the other dims equal, one type (ops.cpp concat) */
GGML_API struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                          int dim);
/* softmax(a * scale + mask) over each row of a contiguous f32 a [n, r1, r2, r3]; mask f32 or
   f16 [n, >= r1, m2, m3] (contiguous, r2 % m2 == 0, r3 % m3 == 0) or NULL; max_bias 0 (no ALiBi)
   (ops.cpp:150-155) */
GGML_API struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a,
                                                struct ggml_tensor * mask, float scale, float max_bias);
/* a * s + b (ops.cpp:121-131, runtime/include/ggml_compiler_ops.h:110-113) */
GGML_API struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s);
GGML_API struct ggml_tensor * ggml_scale_bias(struct ggml_context * ctx, struct ggml_tensor * a, float s, float b);
/* a [K, N] (weight), b [K, M, ...] -> [N, M, ...] f32: out = b a^T per row (ops.cpp:107-119,
   runtime/include/ggml_compiler_ops.h:115-122) */
GGML_API struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
/* Accumulation precision of a mul_mat or flash_attn_ext node (this library accumulates in f32 always). */
GGML_API void ggml_prec_set_acc(struct ggml_tensor * t, enum ggml_prec prec);
GGML_API void ggml_mul_mat_set_prec(struct ggml_tensor * a, enum ggml_prec prec);
GGML_API void ggml_flash_attn_ext_set_prec(struct ggml_tensor * a, enum ggml_prec prec);
/* x / sqrt(mean(x^2) + eps) per row (ops.cpp:144-148) */
GGML_API struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
/* a [D, H, S], b positions i32 [S], c frequency factors [n_dims/2] or NULL (ops.cpp:277-291) */
GGML_API struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                            struct ggml_tensor * c, int n_dims, int mode, int n_ctx_orig,
                                            float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                            float beta_fast, float beta_slow);
/* rows b (i32) of a -> f32 (ops.cpp:302-309) */
GGML_API struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
/* a[:, c[j], ...] = b[:, j, ...] converted to a's type; the result is a view of a (ops.cpp:260-275) */
GGML_API struct ggml_tensor * ggml_set_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                            struct ggml_tensor * c);
/* q [D, Sq, H, 1] f32, k [D, n_kv, Hkv, 1], v [Dv, n_kv, Hkv, 1], mask [n_kv, >= Sq] f16 or NULL
   -> [Dv, H, Sq, 1] f32 (ops.cpp:217-243, runtime/include/ggml_compiler_ops.h:124-148) */
GGML_API struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q,
                                                  struct ggml_tensor * k, struct ggml_tensor * v,
                                                  struct ggml_tensor * mask, float scale, float max_bias,
                                                  float logit_softcap);
/* silu(a) * b (ops.cpp:251-258) */
GGML_API struct ggml_tensor * ggml_swiglu_split(struct ggml_context * ctx, struct ggml_tensor * a,
                                                struct ggml_tensor * b);
/* index of the maximum of each row -> i32 [rows] (ops.cpp:293-300) */
GGML_API struct ggml_tensor * ggml_argmax(struct ggml_context * ctx, struct ggml_tensor * a);

/* Off the path: declared so that code written against ggml (runtime/include/ggml_compiler_ops.h's
   conv_2d) compiles; they build nodes with ggml's result shapes, which ggml_backend_supports_op
   rejects and graph_compute reports as unsupported. */
/* a kernel [KW, KH, IC, OC], b input [W, H, IC, N] -> [IC*KH*KW, OW, OH, N] (is_2D) */
GGML_API struct ggml_tensor * ggml_im2col(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                          int s0, int s1, int p0, int p1, int d0, int d1, bool is_2D,
                                          enum ggml_type dst_type);
/* a kernel [KW, KH, IC, OC], b input [W, H, IC, N] -> [OW, OH, OC, N] */
GGML_API struct ggml_tensor * ggml_conv_2d_direct(struct ggml_context * ctx, struct ggml_tensor * a,
                                                  struct ggml_tensor * b, int s0, int s1, int p0, int p1, int d0,
                                                  int d1);

/* ---- graphs --------------------------------------------------------------------------------- */
GGML_API struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx);
GGML_API struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads);
GGML_API void                 ggml_build_forward_expand(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor);
GGML_API int                  ggml_graph_n_nodes(struct ggml_cgraph * cgraph);
/* i < 0 counts from the end */
GGML_API struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * cgraph, int i);
GGML_API void                 ggml_graph_add_node(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor);
GGML_API void                 ggml_graph_clear(struct ggml_cgraph * cgraph);

#ifdef __cplusplus
}
#endif

#endif /* GGML_H */
