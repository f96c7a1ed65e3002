"""ctypes binding of libgcq.so (include/gcq.h and include/ggml_compiler_rt.h).

The library is found through $GCQ_LIB, else in this package's source tree
(ggml-compiler_amd/lib/libgcq.so), as the reference's bindings find libggml_compiler_rt
(ggml_compiler/runtime/session.py:47-63). There is no fallback: every op runs in libgcq's HIP
kernels, and a missing library or device is an error.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIBRARY = _PKG.parent / "lib" / "libgcq.so"
HEADERS = [_PKG.parents[1] / "include" / h for h in ("gcq.h", "ggml_compiler_rt.h", "ggml.h", "ggml-backend.h",
                                                     "ggml-alloc.h")]


class GcqError(RuntimeError):
    """An error reported by libgcq (its gcq_last_error / ggml_compiler_last_error text)."""


class InitParams(ctypes.Structure):
    """struct ggml_init_params (include/ggml.h)."""
    _fields_ = [("mem_size", ctypes.c_size_t), ("mem_buffer", ctypes.c_void_p), ("no_alloc", ctypes.c_bool)]


class _Options(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_int), ("device", ctypes.c_int), ("n_threads", ctypes.c_int),
                ("allow_cpu_fallback", ctypes.c_bool)]


class TensorInfo(ctypes.Structure):
    """ggml_compiler_tensor_info (include/ggml_compiler_rt.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * 8), ("nbytes", ctypes.c_size_t)]


class Stats(ctypes.Structure):
    """ggml_compiler_stats (include/ggml_compiler_rt.h)."""
    _fields_ = [("ms_total", ctypes.c_double), ("n_calls", ctypes.c_int)]


class Builder(ctypes.Structure):
    """ggml_compiler_builder (include/ggml_compiler_rt.h)."""
    _fields_ = [("stage", ctypes.c_char_p), ("build", ctypes.c_void_p)]


def library_path() -> Path:
    env = os.environ.get("GCQ_LIB")
    if env:
        return Path(env)
    if LIBRARY.exists():
        return LIBRARY
    raise GcqError(f"{LIBRARY} not found: build it (make -C ggml-compiler_amd, or __graft_entry__.build())")


_lib: ctypes.CDLL | None = None

p, i32, i64, u64, sz, f32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t,
                             ctypes.c_float)

SIGNATURES = {
    "gcq_version": ([], ctypes.c_char_p),
    "gcq_last_error": ([], ctypes.c_char_p),
    "gcq_error_count": ([], u64),
    "gcq_device_count": ([], i32),
    "gcq_row_size": ([i32, i64], sz),
    "gcq_weight_size": ([i32, i64, i64], sz),
    "gcq_act_size": ([i32, i64, i64], sz),
    "gcq_mul_mat_workspace": ([i32, i64, i64], sz),
    "gcq_flash_attn_workspace": ([i32, i32, i32, i32, i32], sz),
    "gcq_quantize": ([i32, p, i64, i64, p, p], i32),
    "gcq_pack_weights": ([i32, p, i64, i64, p, p], i32),
    "gcq_dequantize": ([i32, p, i64, i64, p, p], i32),
    "gcq_quantize_act": ([i32, p, i64, i64, i64, p, p], i32),
    "gcq_act_to_ggml": ([i32, p, i64, i64, p, p], i32),
    "gcq_mul_mat": ([i32, p, i64, i64, p, i64, i64, p, i64, p, sz, p], i32),
    "gcq_mul_mat_noalloc": ([i32, p, i64, i64, p, i64, i64, p, i64, p], i32),
    "gcq_mul_mat_q": ([i32, p, i64, i64, p, i64, p, i64, p, p], i32),
    "gcq_rms_norm_q8": ([p, i64, p, i64, i64, f32, p, p], i32),
    "gcq_rms_norm_mul_mat": ([i32, p, i64, i64, p, p, f32, p, p, p, sz, p], i32),
    "gcq_swiglu_q8": ([p, p, i64, i64, i64, p, p], i32),
    "gcq_block_isums": ([i32, p, i64, i64, p, i64, p, p], i32),
    "gcq_gemm_block_isums": ([i32, p, i64, i64, p, i64, i32, p, p], i32),
    "gcq_flash_attn_ext": ([p, i64, i64, p, i64, i64, p, i64, i64, p, i64, p, i32, i32, i32, i32, i32, i32, f32, p, sz,
                            p], i32),
    "gcq_rms_norm": ([p, i64, p, i64, p, i64, i64, f32, p], i32),
    "gcq_rope_neox": ([p, i64, i64, p, i64, i64, p, i64, i64, i64, i32, f32, f32, f32, p, p], i32),
    "gcq_set_rows_f16": ([p, i64, i64, p, i64, i64, p, i64, i64, i64, i64, p], i32),
    "gcq_get_rows": ([i32, p, i64, i64, p, i64, p, p], i32),
    "gcq_swiglu": ([p, p, p, i64, p], i32),
    "gcq_add": ([p, p, p, i64, i64, p], i32),
    "gcq_mul": ([p, p, p, i64, i64, p], i32),
    "gcq_argmax": ([p, i64, i64, i64, p, p], i32),
    "gcq_fill_normal": ([p, i64, u64, u64, f32, p], i32),
    "gcq_stream_read": ([p, sz, i32, i32, p, p], i32),
    "gcq_fill_ids": ([p, i64, u64, u64, ctypes.c_int32, p], i32),
    "gcq_llama_create": ([p, i32], p),
    "gcq_llama_free": ([p], None),
    "gcq_llama_init_random": ([p, u64, f32], i32),
    "gcq_llama_n_weights": ([p], i32),
    "gcq_llama_weight_info": ([p, i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int),
                               ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)], i32),
    "gcq_llama_set_weight": ([p, ctypes.c_char_p, p, sz], i32),
    "gcq_llama_get_weight": ([p, ctypes.c_char_p, p, sz], i32),
    "gcq_llama_reset": ([p], i32),
    "gcq_llama_position": ([p], i32),
    "gcq_llama_prefill": ([p, p, i32, p], i32),
    "gcq_llama_decode": ([p, ctypes.c_int32, p, p], i32),
    "gcq_llama_generate": ([p, ctypes.c_int32, i32, p], i32),
    "gcq_llama_forward_layers": ([p, p, i32, i32, i32, i32, p, p], i32),
    "ggml_compiler_version": ([], ctypes.c_char_p),
    "ggml_compiler_last_error": ([], ctypes.c_char_p),
    "ggml_compiler_default_options": ([], _Options),
    "ggml_compiler_has_backend": ([i32], ctypes.c_bool),
    "ggml_compiler_quantize": ([ctypes.c_char_p, p, i64, i64, p, sz], sz),
    "ggml_compiler_row_size": ([ctypes.c_char_p, i64], sz),
    "ggml_compiler_load": ([ctypes.c_char_p, p], p),
    "ggml_compiler_load_with": ([ctypes.c_char_p, p, p, i32], p),
    "ggml_compiler_metadata": ([p, ctypes.c_char_p], ctypes.c_char_p),
    "ggml_compiler_free": ([p], None),
    "ggml_compiler_backend_name": ([p], ctypes.c_char_p),
    "ggml_compiler_n_entries": ([p], i32),
    "ggml_compiler_entry_name": ([p, i32], ctypes.c_char_p),
    "ggml_compiler_entry_n_inputs": ([p, i32], i32),
    "ggml_compiler_entry_n_outputs": ([p, i32], i32),
    "ggml_compiler_entry_input_info": ([p, i32, i32, p], i32),
    "ggml_compiler_entry_output_info": ([p, i32, i32, p], i32),
    "ggml_compiler_run_entry": ([p, ctypes.c_char_p], i32),
    "ggml_compiler_reset": ([p], i32),
    "ggml_compiler_n_inputs": ([p], i32),
    "ggml_compiler_n_outputs": ([p], i32),
    "ggml_compiler_input_info": ([p, i32, p], i32),
    "ggml_compiler_output_info": ([p, i32, p], i32),
    "ggml_compiler_n_symbols": ([p], i32),
    "ggml_compiler_symbol_info": ([p, i32, p, p, p, p], i32),
    "ggml_compiler_set_symbol": ([p, ctypes.c_char_p, i64], i32),
    "ggml_compiler_set_input_shape": ([p, ctypes.c_char_p, i32, p], i32),
    "ggml_compiler_set_input": ([p, ctypes.c_char_p, p, sz], i32),
    "ggml_compiler_run": ([p], i32),
    "ggml_compiler_get_output": ([p, ctypes.c_char_p, p, sz], i32),
    "ggml_compiler_last_stats": ([p, p], i32),
    "ggml_compiler_n_stages": ([p], i32),
    "ggml_compiler_stage_stats": ([p, i32, p, p, p], i32),
    "ggml_compiler_build_ctx": ([p], p),
    "ggml_compiler_build_gpu": ([p], ctypes.c_bool),
    "ggml_compiler_build_supports": ([p, p], ctypes.c_bool),
    "ggml_compiler_build_param": ([p, i32], p),
    "ggml_compiler_build_weight": ([p, ctypes.c_char_p], p),
    "ggml_compiler_build_symbol": ([p, i32], i64),
    "ggml_compiler_build_output": ([p, i32, p], None),
    # ggml.h (contexts, tensors and graphs are opaque pointers here; ggml.py views tensors)
    "ggml_last_error": ([], ctypes.c_char_p),
    "ggml_init": ([InitParams], p),
    "ggml_free": ([p], None),
    "ggml_tensor_overhead": ([], sz),
    "ggml_graph_overhead": ([], sz),
    "ggml_graph_overhead_custom": ([sz, ctypes.c_bool], sz),
    "ggml_type_size": ([i32], sz),
    "ggml_blck_size": ([i32], i64),
    "ggml_row_size": ([i32, i64], sz),
    "ggml_type_name": ([i32], ctypes.c_char_p),
    "ggml_is_quantized": ([i32], ctypes.c_bool),
    "ggml_op_name": ([i32], ctypes.c_char_p),
    "ggml_op_desc": ([p], ctypes.c_char_p),
    "ggml_nelements": ([p], i64),
    "ggml_nrows": ([p], i64),
    "ggml_nbytes": ([p], sz),
    "ggml_is_contiguous": ([p], ctypes.c_bool),
    "ggml_is_transposed": ([p], ctypes.c_bool),
    "ggml_is_permuted": ([p], ctypes.c_bool),
    "ggml_is_vector": ([p], ctypes.c_bool),
    "ggml_is_matrix": ([p], ctypes.c_bool),
    "ggml_are_same_shape": ([p, p], ctypes.c_bool),
    "ggml_can_repeat": ([p, p], ctypes.c_bool),
    "ggml_new_tensor": ([p, i32, i32, ctypes.POINTER(ctypes.c_int64)], p),
    "ggml_new_tensor_1d": ([p, i32, i64], p),
    "ggml_new_tensor_2d": ([p, i32, i64, i64], p),
    "ggml_new_tensor_3d": ([p, i32, i64, i64, i64], p),
    "ggml_new_tensor_4d": ([p, i32, i64, i64, i64, i64], p),
    "ggml_set_name": ([p, ctypes.c_char_p], p),
    "ggml_get_name": ([p], ctypes.c_char_p),
    "ggml_get_tensor": ([p, ctypes.c_char_p], p),
    "ggml_get_first_tensor": ([p], p),
    "ggml_get_next_tensor": ([p, p], p),
    "ggml_set_input": ([p], None),
    "ggml_set_output": ([p], None),
    "ggml_view_1d": ([p, p, i64, sz], p),
    "ggml_view_2d": ([p, p, i64, i64, sz, sz], p),
    "ggml_view_3d": ([p, p, i64, i64, i64, sz, sz, sz], p),
    "ggml_view_4d": ([p, p, i64, i64, i64, i64, sz, sz, sz, sz], p),
    "ggml_view_tensor": ([p, p], p),
    "ggml_reshape": ([p, p, p], p),
    "ggml_reshape_1d": ([p, p, i64], p),
    "ggml_reshape_2d": ([p, p, i64, i64], p),
    "ggml_reshape_3d": ([p, p, i64, i64, i64], p),
    "ggml_reshape_4d": ([p, p, i64, i64, i64, i64], p),
    "ggml_permute": ([p, p, i32, i32, i32, i32], p),
    "ggml_transpose": ([p, p], p),
    "ggml_cont": ([p, p], p),
    "ggml_cpy": ([p, p, p], p),
    "ggml_cast": ([p, p, i32], p),
    "ggml_add": ([p, p, p], p),
    "ggml_mul": ([p, p, p], p),
    "ggml_scale": ([p, p, f32], p),
    "ggml_scale_bias": ([p, p, f32, f32], p),
    "ggml_mul_mat": ([p, p, p], p),
    "ggml_prec_set_acc": ([p, i32], None),
    "ggml_mul_mat_set_prec": ([p, i32], None),
    "ggml_flash_attn_ext_set_prec": ([p, i32], None),
    "ggml_rms_norm": ([p, p, f32], p),
    "ggml_rope_ext": ([p, p, p, p, i32, i32, i32, f32, f32, f32, f32, f32, f32], p),
    "ggml_get_rows": ([p, p, p], p),
    "ggml_set_rows": ([p, p, p, p], p),
    "ggml_flash_attn_ext": ([p, p, p, p, p, f32, f32, f32], p),
    "ggml_swiglu_split": ([p, p, p], p),
    "ggml_argmax": ([p, p], p),
    "ggml_gelu": ([p, p], p),
    "ggml_tanh": ([p, p], p),
    "ggml_sqr": ([p, p], p),
    "ggml_gelu_erf": ([p, p], p),
    "ggml_silu": ([p, p], p),
    "ggml_relu": ([p, p], p),
    "ggml_sigmoid": ([p, p], p),
    "ggml_exp": ([p, p], p),
    "ggml_log": ([p, p], p),
    "ggml_neg": ([p, p], p),
    "ggml_abs": ([p, p], p),
    "ggml_sqrt": ([p, p], p),
    "ggml_sin": ([p, p], p),
    "ggml_cos": ([p, p], p),
    "ggml_softplus": ([p, p], p),
    "ggml_sub": ([p, p, p], p),
    "ggml_clamp": ([p, p, f32, f32], p),
    "ggml_norm": ([p, p, f32], p),
    "ggml_sum_rows": ([p, p], p),
    "ggml_mean": ([p, p], p),
    "ggml_repeat_4d": ([p, p, i64, i64, i64, i64], p),
    "ggml_concat": ([p, p, p, i32], p),
    "ggml_div": ([p, p, p], p),
    "ggml_soft_max_ext": ([p, p, p, f32, f32], p),
    "ggml_im2col": ([p, p, p, i32, i32, i32, i32, i32, i32, ctypes.c_bool, i32], p),
    "ggml_conv_2d_direct": ([p, p, p, i32, i32, i32, i32, i32, i32], p),
    "ggml_new_graph": ([p], p),
    "ggml_new_graph_custom": ([p, sz, ctypes.c_bool], p),
    "ggml_build_forward_expand": ([p, p], None),
    "ggml_graph_n_nodes": ([p], i32),
    "ggml_graph_node": ([p, i32], p),
    "ggml_graph_add_node": ([p, p], None),
    "ggml_graph_clear": ([p], None),
    # ggml-backend.h
    "ggml_backend_hip_init": ([i32], p),
    "ggml_backend_is_hip": ([p], ctypes.c_bool),
    "ggml_backend_free": ([p], None),
    "ggml_backend_name": ([p], ctypes.c_char_p),
    "ggml_backend_synchronize": ([p], None),
    "ggml_backend_get_default_buffer_type": ([p], p),
    "ggml_backend_buft_name": ([p], ctypes.c_char_p),
    "ggml_backend_supports_op": ([p, p], ctypes.c_bool),
    "ggml_backend_graph_compute": ([p, p], i32),
    "ggml_backend_hip_set_use_graphs": ([p, ctypes.c_bool], None),
    "ggml_backend_alloc_ctx_tensors": ([p, p], p),
    "ggml_backend_alloc_ctx_tensors_from_buft": ([p, p], p),
    "ggml_backend_buffer_free": ([p], None),
    "ggml_backend_buffer_get_size": ([p], sz),
    "ggml_backend_buffer_get_base": ([p], p),
    "ggml_backend_buffer_clear": ([p, ctypes.c_uint8], None),
    "ggml_backend_buffer_is_host": ([p], ctypes.c_bool),
    "ggml_backend_buft_get_alloc_size": ([p, p], sz),
    "ggml_backend_tensor_set": ([p, p, sz, sz], None),
    "ggml_backend_tensor_get": ([p, p, sz, sz], None),
    "ggml_backend_tensor_memset": ([p, ctypes.c_uint8, sz, sz], None),
    "ggml_backend_tensor_copy": ([p, p], None),
    "ggml_backend_view_init": ([p], i32),
    "ggml_status_to_string": ([i32], ctypes.c_char_p),
    # ggml-alloc.h
    "ggml_gallocr_new": ([p], p),
    "ggml_gallocr_free": ([p], None),
    "ggml_gallocr_reserve": ([p, p], ctypes.c_bool),
    "ggml_gallocr_alloc_graph": ([p, p], ctypes.c_bool),
    "ggml_gallocr_get_buffer_size": ([p, i32], sz),
}


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    lib = ctypes.CDLL(str(library_path()))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def error() -> GcqError:
    return GcqError(load().gcq_last_error().decode())


def check(rc: int) -> None:
    if rc != 0:
        raise error()
