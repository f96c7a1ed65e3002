/*
 * ggml_compiler_rt.h - the part of ggml-compiler's runtime C API that libgcq provides.
 *
 * Same names, types, argument meaning and error convention as the reference's header
 * (runtime/include/ggml_compiler_rt.h): int functions return 0 / -1, size functions return 0 on
 * error, and ggml_compiler_last_error() describes the last failure of the calling thread.
 * Provided here: version, last_error, default_options, has_backend, quantize, row_size
 * (runtime/include/ggml_compiler_rt.h:77-89). The GGUF program loader and its model handle
 * (load, run, entries, symbols, builder hooks, :91-172) are not part of this library.
 *
 * Backends: libgcq runs on HIP devices only. GGML_COMPILER_BACKEND_HIP is added to the reference's
 * enum (CPU = 0, CUDA = 1, AUTO = 2, runtime/include/ggml_compiler_rt.h:45-49); AUTO means the first
 * HIP device, as the reference's AUTO means the first GPU (runtime/src/ggml_compiler_rt.cpp:104-125).
 */
#ifndef GGML_COMPILER_RT_H
#define GGML_COMPILER_RT_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#define GGML_COMPILER_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_COMPILER_MAX_RANK 8

typedef enum {
    GGML_COMPILER_BACKEND_CPU  = 0,
    GGML_COMPILER_BACKEND_CUDA = 1,
    GGML_COMPILER_BACKEND_AUTO = 2,
    GGML_COMPILER_BACKEND_HIP  = 3,
} ggml_compiler_backend;

typedef enum {
    GGML_COMPILER_DTYPE_F32 = 0,
    GGML_COMPILER_DTYPE_F16 = 1,
    GGML_COMPILER_DTYPE_I32 = 2,
} ggml_compiler_dtype;

typedef struct {
    ggml_compiler_backend backend;
    int                   device;
    int                   n_threads;
    bool                  allow_cpu_fallback;
} ggml_compiler_options;

GGML_COMPILER_API const char *          ggml_compiler_version(void);
GGML_COMPILER_API const char *          ggml_compiler_last_error(void);
GGML_COMPILER_API ggml_compiler_options ggml_compiler_default_options(void);
/* True if a HIP device is present (HIP, AUTO); false for CPU and CUDA, which libgcq does not have. */
GGML_COMPILER_API bool                  ggml_compiler_has_backend(ggml_compiler_backend backend);

/* Encode f32 rows (host memory) in a ggml type ("q8_0", "q4_0", "q4_K", "f16", "f32") exactly as
   ggml stores them, into host memory; the encoding runs on the GPU. Returns the bytes written, or
   0 on error (unknown type, n_per_row not a multiple of the block size, dst_size too small, no
   device). (runtime/include/ggml_compiler_rt.h:83-87) */
GGML_COMPILER_API size_t ggml_compiler_quantize(const char * type, const float * src, int64_t nrows,
                                                int64_t n_per_row, void * dst, size_t dst_size);
/* Bytes one row of n elements takes in that type, or 0 if the type is unknown.
   (runtime/include/ggml_compiler_rt.h:88-89) */
GGML_COMPILER_API size_t ggml_compiler_row_size(const char * type, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* GGML_COMPILER_RT_H */
