/*
 * ggml-backend.h - the part of ggml's backend API that ggml-compiler's runtime uses to hold
 * weights, state and per-call-site compute buffers on a device and to run a built graph, provided by
 * libgcq for one HIP device (gfx950).
 *
 * The reference runtime allocates a context's tensors in one device buffer
 * (ggml_backend_alloc_ctx_tensors, runtime/src/ggml_compiler_rt.cpp:150-191, 445-479), copies
 * inputs and outputs with ggml_backend_tensor_set / _get (:1079-1094, :1125-1144) and runs each call
 * site's graph with ggml_backend_graph_compute (:356-374), asking ggml_backend_supports_op before
 * choosing flash attention (runtime/src/ops.cpp:228-240). Same names, arguments and status values.
 *
 * Quantized weights: a Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K tensor allocated here holds the layout the kernels read
 * (gcq_pack_weights), which takes a few bytes more than ggml_nbytes. ggml_backend_tensor_set and
 * _get convert whole tensors to and from ggml's block bytes (offset 0, size ggml_nbytes); a partial
 * range of a quantized tensor is an error.
 *
 * Execution: ggml_backend_graph_compute runs the graph's nodes on the backend's stream, fusing
 * rms_norm -> mul -> mul_mat, swiglu -> mul_mat and mul_mat -> add chains where the intermediate
 * has no other use and is not flagged as an output. The launches are captured into a HIP graph and
 * replayed while the nodes, their shapes and their data addresses stay the same. A node outside
 * the supported set fails the compute with GGML_STATUS_FAILED and a message (ggml_last_error()).
 */
#ifndef GGML_BACKEND_H
#define GGML_BACKEND_H

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_backend *             ggml_backend_t;
typedef struct ggml_backend_buffer *      ggml_backend_buffer_t;
typedef struct ggml_backend_buffer_type * ggml_backend_buffer_type_t;

/* A backend on HIP device `device` (must be gfx950), NULL with ggml_last_error() set otherwise.
   Stands where the reference creates its GPU backend (runtime/src/ggml_compiler_rt.cpp:104-125). */
GGML_API ggml_backend_t             ggml_backend_hip_init(int device);
GGML_API bool                       ggml_backend_is_hip(ggml_backend_t backend);
GGML_API void                       ggml_backend_free(ggml_backend_t backend);
GGML_API const char *               ggml_backend_name(ggml_backend_t backend);
GGML_API void                       ggml_backend_synchronize(ggml_backend_t backend);
GGML_API ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend);
GGML_API const char *               ggml_backend_buft_name(ggml_backend_buffer_type_t buft);
/* Whether graph_compute can run this node (its op, types, shapes and layout). */
GGML_API bool                       ggml_backend_supports_op(ggml_backend_t backend, const struct ggml_tensor * op);
/* Runs the graph and waits for it. */
GGML_API enum ggml_status           ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph);
/* HIP graph capture and replay of graph_compute's launches (on by default). */
GGML_API void                       ggml_backend_hip_set_use_graphs(ggml_backend_t backend, bool use);

/* One device buffer holding every tensor of ctx that has no data yet (views get their base's
   memory); NULL if there is none or the allocation fails. */
GGML_API ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx, ggml_backend_t backend);
GGML_API ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context * ctx,
                                                                        ggml_backend_buffer_type_t buft);
GGML_API void                  ggml_backend_buffer_free(ggml_backend_buffer_t buffer);
GGML_API size_t                ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer);
GGML_API void *                ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer);
GGML_API void                  ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value);
GGML_API bool                  ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer);
/* Bytes a tensor takes in this buffer type (the packed size for quantized weights). */
GGML_API size_t                ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft,
                                                                const struct ggml_tensor * tensor);

/* Host <-> device copies into / out of a tensor's bytes [offset, offset + size); synchronous. */
GGML_API void ggml_backend_tensor_set(struct ggml_tensor * tensor, const void * data, size_t offset, size_t size);
GGML_API void ggml_backend_tensor_get(const struct ggml_tensor * tensor, void * data, size_t offset, size_t size);
GGML_API void ggml_backend_tensor_memset(struct ggml_tensor * tensor, uint8_t value, size_t offset, size_t size);
/* dst = src, same type and shape, both contiguous */
GGML_API void ggml_backend_tensor_copy(struct ggml_tensor * src, struct ggml_tensor * dst);
/* Gives a view the memory of its view_src (which must have it). */
GGML_API enum ggml_status ggml_backend_view_init(struct ggml_tensor * tensor);

GGML_API const char * ggml_status_to_string(enum ggml_status status);

#ifdef __cplusplus
}
#endif

#endif /* GGML_BACKEND_H */
