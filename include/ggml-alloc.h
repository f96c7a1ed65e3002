/*
 * ggml-alloc.h - ggml's graph allocator as the reference runtime uses it: one allocator per call
 * site gives every node (and every leaf without memory) of a built graph its place in a device
 * buffer that the allocator owns and grows (runtime/src/ggml_compiler_rt.cpp:150-191, ggml_gallocr_*).
 * Memory of a node is reused once every node that reads it (directly or through a view) has run;
 * inputs (ggml_set_input), outputs (ggml_set_output) and the last node keep theirs.
 */
#ifndef GGML_ALLOC_H
#define GGML_ALLOC_H

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_gallocr * ggml_gallocr_t;

GGML_API ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft);
GGML_API void           ggml_gallocr_free(ggml_gallocr_t galloc);
/* Sizes the buffer for the graph without assigning addresses. */
GGML_API bool           ggml_gallocr_reserve(ggml_gallocr_t galloc, struct ggml_cgraph * graph);
/* Assigns every node and data-less leaf of the graph its memory (growing the buffer if needed). */
GGML_API bool           ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph * graph);
GGML_API size_t         ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id);

#ifdef __cplusplus
}
#endif

#endif /* GGML_ALLOC_H */
