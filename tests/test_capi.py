"""CPU-side checks of libgcq's C ABI: the library loads, exports every symbol its headers declare,
answers size queries like ggml, and rejects bad arguments on the host before any launch."""

import ctypes
import re

import pytest

from ggml_compiler_amd import _lib


def _declared():
    names = []
    for h in _lib.HEADERS:
        text = h.read_text()
        text = re.sub(r"#\s*define[^\n]*", "", text)
        names += re.findall(r"(?:GCQ_API|GGML_COMPILER_API|GGML_API)[^;(]*?\b(\w+)\s*\(", text)
    return names


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = _declared()
    assert len(names) == 214
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_row_sizes_match_ggml(orc):
    lib = _lib.load()
    for t, name in ((2, b"q4_0"), (8, b"q8_0"), (12, b"q4_K"), (1, b"f16"), (0, b"f32")):
        for n in (256, 4096, 14336):
            assert lib.gcq_row_size(t, n) == orc.row_size(t, n)
            assert lib.ggml_compiler_row_size(name, n) == orc.row_size(t, n)
    assert lib.ggml_compiler_row_size(b"q4_K", 4096) == 2304  # compiler.py:81-82 ratios
    assert lib.ggml_compiler_row_size(b"q8_0", 4096) == 4352
    assert lib.ggml_compiler_row_size(b"q4_0", 14336) == 8064


def test_row_size_errors():
    lib = _lib.load()
    assert lib.ggml_compiler_row_size(b"q9_9", 32) == 0
    assert "unknown" in lib.ggml_compiler_last_error().decode()
    assert lib.ggml_compiler_row_size(b"q4_K", 100) == 0
    assert "block size" in lib.ggml_compiler_last_error().decode()
    assert lib.gcq_row_size(2, 33) == 0


def test_packed_and_workspace_sizes():
    lib = _lib.load()
    # Same bytes as ggml, each section rounded up to 256 B.
    assert lib.gcq_weight_size(2, 4096, 4096) == 4096 * 128 * 16 + 4096 * 128 * 2
    assert lib.gcq_weight_size(12, 4096, 4096) == 4096 * 2304
    assert lib.gcq_act_size(2, 1, 4096) == 4096 + 128 * 8
    # the whole quantized activation: the K-quant GEMM reads every row's codes, block sums and d
    assert lib.gcq_mul_mat_workspace(12, 100, 4096) == lib.gcq_act_size(12, 100, 4096)
    assert lib.gcq_act_size(12, 100, 4096) == 100 * 4096 + 100 * 256 * 2 + 100 * 16 * 4
    assert lib.gcq_weight_size(3, 1, 32) == 0
    assert lib.gcq_flash_attn_workspace(1, 32, 8, 128, 4096) > 0


def test_host_side_argument_checks():
    """Bad arguments fail with a message before anything reaches a device."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    assert lib.gcq_mul_mat(5, p, 8, 64, p, 64, 1, p, 8, p, 1 << 20, None) == -1
    assert "unsupported weight type" in lib.gcq_last_error().decode()
    assert lib.gcq_mul_mat(2, p, 8, 48, p, 48, 1, p, 8, p, 1 << 20, None) == -1
    assert "multiple of the type's block size" in lib.gcq_last_error().decode()
    assert lib.gcq_mul_mat(2, p, 8, 64, p, 64, 1, p, 8, p, 16, None) == -1
    assert "workspace" in lib.gcq_last_error().decode()
    assert lib.gcq_mul_mat(2, None, 8, 64, p, 64, 1, p, 8, p, 1 << 20, None) == -1
    assert "NULL" in lib.gcq_last_error().decode()
    assert lib.gcq_block_isums(2, p, 8, 64, p, 9, p, None) == -1  # B <= 8
    assert lib.gcq_flash_attn_ext(p, 0, 0, p, 0, 7, p, 0, 8, None, 0, p, 128, 128, 1, 32, 8, 16, 0.1, p, 1 << 20,
                                  None) == -1
    assert "multiples of 8" in lib.gcq_last_error().decode()
    assert lib.gcq_rope_neox(p, 0, 0, p, 0, 0, p, 128, 1, 1, 129, 1e4, 1.0, 1.0, None, None) == -1
    assert lib.gcq_set_rows_f16(p, 0, 12, p, 0, 0, p, 1, 128, 1, 64, None) == -1
    assert lib.gcq_stream_read(p, 1 << 20, 12, 1, p, None) == -1
    assert "waves_per_cu" in lib.gcq_last_error().decode()
    assert lib.gcq_stream_read(p, 100, 16, 1, p, None) == -1
    assert "16-byte" in lib.gcq_last_error().decode()


def test_runtime_api_without_a_device():
    lib = _lib.load()
    o = lib.ggml_compiler_default_options()
    assert (o.backend, o.device, o.n_threads, o.allow_cpu_fallback) == (2, 0, 0, False)
    assert not lib.ggml_compiler_has_backend(0)  # no CPU backend in libgcq
    assert "gfx950" in lib.ggml_compiler_version().decode()
    if lib.gcq_device_count() == 0:
        import numpy as np

        src = np.zeros((1, 32), np.float32)
        dst = np.zeros(34, np.uint8)
        assert lib.ggml_compiler_quantize(b"q8_0", src.ctypes.data, 1, 32, dst.ctypes.data, 34) == 0
        assert "no HIP device" in lib.ggml_compiler_last_error().decode()
    src = bytes(4 * 32)
    assert lib.ggml_compiler_quantize(b"q8_0", src, 1, 32, ctypes.create_string_buffer(10), 10) == 0
    assert "too small" in lib.ggml_compiler_last_error().decode()


def test_product_path_has_no_cpu_fallback():
    """libgcq links no oracle code and exports no CPU compute entry points."""
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True, text=True,
                         check=True).stdout
    assert "orc_" not in out
    deps = subprocess.run(["ldd", str(_lib.library_path())], capture_output=True, text=True).stdout
    assert "gcq_oracle" not in deps
