"""Source compatibility of the ggml API subset: a stage builder written as ggml-compiler's C++
emitter writes them (emit/cpp.py:63-122), including the reference's own header-only helpers
(runtime/include/ggml_compiler_ops.h, compiled where the reference tree lies, not copied), builds
and links against include/ggml.h and libgcq and constructs the decode layer's graph. Host only."""

import subprocess
from pathlib import Path

import pytest

from ggml_compiler_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
REF_INCLUDE = Path("/root/reference/runtime/include")


@pytest.mark.skipif(not (REF_INCLUDE / "ggml_compiler_ops.h").exists(), reason="reference tree not present")
def test_emitted_style_builder_compiles_and_builds(tmp_path):
    exe = tmp_path / "builder_compat"
    lib = _lib.library_path()
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{ROOT / 'include'}", f"-I{REF_INCLUDE}",
                    str(ROOT / "tests" / "cpp" / "builder_compat.cpp"), str(lib), f"-Wl,-rpath,{lib.parent}",
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    ops = [o for o in out if o and not o.startswith("nodes")]
    assert out[len(ops)] == f"nodes {len(ops)}"
    assert ops.count("MUL_MAT") == 7 and ops.count("FLASH_ATTN_EXT") == 1 and ops.count("SET_ROWS") == 2
    assert ops.count("ROPE") == 2 and ops.count("GLU") == 1 and ops.count("RMS_NORM") == 2
    assert ops[-1] == "ADD"
