/*
 * ggml_compiler_rt.h - the part of ggml-compiler's runtime C API that libgcq provides.
 *
 * Same names, types, argument meaning and error convention as the reference's header
 * (runtime/include/ggml_compiler_rt.h): int functions return 0 / -1, size functions return 0 on
 * error, and ggml_compiler_last_error() describes the last failure of the calling thread.
 * Provided here: version, last_error, default_options, has_backend, quantize, row_size
 * (runtime/include/ggml_compiler_rt.h:77-89), and the GGUF program loader with its model handle:
 * load, metadata, entries, inputs / outputs, symbols, run, stats and the compiled-builder hooks
 * (:91-172). A model runs its program's stages as graphs of this library's ggml API on the HIP
 * backend (ggml-backend.h); a stage node the backend cannot run fails the load with its name.
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

typedef struct ggml_compiler_model ggml_compiler_model;

typedef struct {
    const char *        name; /* valid while the model is alive */
    ggml_compiler_dtype dtype;
    int                 ndim;
    int64_t             shape[GGML_COMPILER_MAX_RANK]; /* PyTorch order */
    size_t              nbytes;
} ggml_compiler_tensor_info;

typedef struct {
    double ms_total; /* wall time of the last run */
    int    n_calls;  /* stage calls of the last run */
} ggml_compiler_stats;

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

/* ---- models (runtime/include/ggml_compiler_rt.h:91-151) -------------------------------------
 * A GGUF written by ggml-compiler (general.architecture "ggml_compiler", the program JSON under
 * "ggml_compiler.program", format versions 1-3). opt may be NULL (the defaults); the backend must
 * be HIP or AUTO and allow_cpu_fallback false. NULL on failure. */
GGML_COMPILER_API ggml_compiler_model * ggml_compiler_load(const char * path, const ggml_compiler_options * opt);
/* The GGUF's string value under key, or NULL (absent or not a string). */
GGML_COMPILER_API const char * ggml_compiler_metadata(const ggml_compiler_model * m, const char * key);
GGML_COMPILER_API void         ggml_compiler_free(ggml_compiler_model * m);
GGML_COMPILER_API const char * ggml_compiler_backend_name(const ggml_compiler_model * m);

/* Entry points e in [0, n_entries); the first is the default of n_inputs / input_info / run. */
GGML_COMPILER_API int          ggml_compiler_n_entries(const ggml_compiler_model * m);
GGML_COMPILER_API const char * ggml_compiler_entry_name(const ggml_compiler_model * m, int e);
GGML_COMPILER_API int          ggml_compiler_entry_n_inputs(const ggml_compiler_model * m, int e);
GGML_COMPILER_API int          ggml_compiler_entry_n_outputs(const ggml_compiler_model * m, int e);
GGML_COMPILER_API int          ggml_compiler_entry_input_info(const ggml_compiler_model * m, int e, int i,
                                                              ggml_compiler_tensor_info * info);
GGML_COMPILER_API int          ggml_compiler_entry_output_info(const ggml_compiler_model * m, int e, int i,
                                                               ggml_compiler_tensor_info * info);
/* Run the named entry point; every input it takes must have been set. */
GGML_COMPILER_API int          ggml_compiler_run_entry(ggml_compiler_model * m, const char * entry);
/* Zero the program's state values (a KV cache). Load starts from zeros too. */
GGML_COMPILER_API int          ggml_compiler_reset(ggml_compiler_model * m);

GGML_COMPILER_API int ggml_compiler_n_inputs(const ggml_compiler_model * m);
GGML_COMPILER_API int ggml_compiler_n_outputs(const ggml_compiler_model * m);
GGML_COMPILER_API int ggml_compiler_input_info(const ggml_compiler_model * m, int i, ggml_compiler_tensor_info * info);
GGML_COMPILER_API int ggml_compiler_output_info(const ggml_compiler_model * m, int i, ggml_compiler_tensor_info * info);

/* Symbols i in [0, n_symbols); any out pointer may be NULL. */
GGML_COMPILER_API int ggml_compiler_n_symbols(const ggml_compiler_model * m);
GGML_COMPILER_API int ggml_compiler_symbol_info(const ggml_compiler_model * m, int i, const char ** name,
                                                int64_t * min, int64_t * max, int64_t * value);
GGML_COMPILER_API int ggml_compiler_set_symbol(ggml_compiler_model * m, const char * name, int64_t value);
/* Bind the symbols an input's shape fixes (each dim with one unknown symbol solved by bisection
   over the symbol's range); the shape must be one the program accepts. */
GGML_COMPILER_API int ggml_compiler_set_input_shape(ggml_compiler_model * m, const char * name, int ndim,
                                                    const int64_t * shape);

/* Host -> device; nbytes must equal the input's size for the current binding. */
GGML_COMPILER_API int ggml_compiler_set_input(ggml_compiler_model * m, const char * name, const void * data,
                                              size_t nbytes);
GGML_COMPILER_API int ggml_compiler_run(ggml_compiler_model * m);
/* Device -> host; nbytes must equal the output's size for the binding of the last run. */
GGML_COMPILER_API int ggml_compiler_get_output(ggml_compiler_model * m, const char * name, void * dst, size_t nbytes);

GGML_COMPILER_API int ggml_compiler_last_stats(const ggml_compiler_model * m, ggml_compiler_stats * st);
GGML_COMPILER_API int ggml_compiler_n_stages(const ggml_compiler_model * m);
GGML_COMPILER_API int ggml_compiler_stage_stats(const ggml_compiler_model * m, int i, const char ** name, double * ms,
                                                int * n_calls);

/* ---- compiled stage builders (runtime/include/ggml_compiler_rt.h:153-172) -------------------
 * A builder replaces the loader's graph construction for one stage: it receives the stage's
 * parameters, looks weights up by GGUF name and names the stage's outputs; the loader keeps the
 * weights, driver values, call sites and the C API. */
struct ggml_context;
struct ggml_tensor;
typedef struct ggml_compiler_stage_build ggml_compiler_stage_build;
typedef int (*ggml_compiler_build_fn)(ggml_compiler_stage_build * b); /* 0 on success */

typedef struct {
    const char *           stage;
    ggml_compiler_build_fn build;
} ggml_compiler_builder;

GGML_COMPILER_API struct ggml_context * ggml_compiler_build_ctx(ggml_compiler_stage_build * b);
GGML_COMPILER_API bool                  ggml_compiler_build_gpu(ggml_compiler_stage_build * b);
GGML_COMPILER_API bool                  ggml_compiler_build_supports(ggml_compiler_stage_build * b,
                                                                     const struct ggml_tensor * t);
GGML_COMPILER_API struct ggml_tensor *  ggml_compiler_build_param(ggml_compiler_stage_build * b, int i);
GGML_COMPILER_API struct ggml_tensor *  ggml_compiler_build_weight(ggml_compiler_stage_build * b,
                                                                   const char * gguf_name);
GGML_COMPILER_API int64_t               ggml_compiler_build_symbol(ggml_compiler_stage_build * b, int i);
GGML_COMPILER_API void                  ggml_compiler_build_output(ggml_compiler_stage_build * b, int i,
                                                                   struct ggml_tensor * t);
/* ggml_compiler_load with the listed stages built by compiled builders. */
GGML_COMPILER_API ggml_compiler_model * ggml_compiler_load_with(const char * path, const ggml_compiler_options * opt,
                                                                const ggml_compiler_builder * builders,
                                                                int n_builders);

#ifdef __cplusplus
}
#endif

#endif /* GGML_COMPILER_RT_H */
