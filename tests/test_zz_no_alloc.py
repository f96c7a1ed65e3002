"""gcq_mul_mat_noalloc (include/gcq.h) through the C ABI: the same results as gcq_mul_mat with a
workspace, bit for bit, on two calls in a row with the second smaller than the first (the static
scratch keeps the first call's contents), for each path (one-row GEMV, multi-row GEMV, MFMA GEMM,
K-quant row groups); a size beyond the scratch is rejected on the host; and a process whose first
call (the scratch lookup, the device queries) is made while capturing a HIP graph replays it
correctly."""

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from ggml_compiler_amd import _lib

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _weight(gops, orc, t, N, K, seed):
    raw = orc.quantize(orc.normal((N, K), seed=seed, std=0.02), t)
    return gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)


def _with_workspace(lib, qw, x):
    M, K = x.shape
    y = torch.full((M, qw.N), float("nan"), dtype=torch.float32, device="cuda")
    nbytes = int(lib.gcq_mul_mat_workspace(qw.type, M, K))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda")
    assert lib.gcq_mul_mat(qw.type, _p(qw.data), qw.N, K, _p(x), K, M, _p(y), qw.N, _p(ws), ws.numel(),
                           _stream()) == 0, lib.gcq_last_error().decode()
    return y


def _noalloc(lib, qw, x):
    M, K = x.shape
    y = torch.full((M, qw.N), float("nan"), dtype=torch.float32, device="cuda")
    assert lib.gcq_mul_mat_noalloc(qw.type, _p(qw.data), qw.N, K, _p(x), K, M, _p(y), qw.N,
                                   _stream()) == 0, lib.gcq_last_error().decode()
    return y


@pytest.mark.parametrize("t,first,second", [
    ("q4_0", (128, 512, 4096), (3, 300, 1024)),   # MFMA GEMM, then the multi-row GEMV
    ("q8_0", (40, 256, 2048), (9, 64, 512)),      # GEMM twice, the second over less scratch
    ("q4_K", (20, 256, 2048), (2, 100, 512)),     # K-quant groups of 8 rows, then one group
    ("q4_0", (8, 1000, 4096), (1, 700, 4096)),    # GEMV, then the one-row path (no scratch)
])
def test_noalloc_equals_workspace_entry(gops, orc, t, first, second):
    lib = _lib.load()
    for seed, (M, N, K) in enumerate((first, second)):
        print(f"noalloc {t} M={M} N={N} K={K}", flush=True)
        qw = _weight(gops, orc, t, N, K, 40 + seed)
        x = torch.from_numpy(orc.normal((M, K), seed=50 + seed)).cuda()
        want = _with_workspace(lib, qw, x)
        got = _noalloc(lib, qw, x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (t, M, N, K)
        assert np.isfinite(got.cpu().numpy()).all()


def test_noalloc_rejects_sizes_beyond_scratch():
    lib = _lib.load()
    before = lib.gcq_error_count()
    # 4096 rows of 4096 values need 20 MiB of Q8_0 codes and scales: more than the 16 MiB scratch.
    rc = lib.gcq_mul_mat_noalloc(2, None, 4096, 4096, None, 4096, 4096, None, 4096, None)
    assert rc == -1 and lib.gcq_error_count() == before + 1
    assert "scratch" in lib.gcq_last_error().decode()


_CAPTURE = r"""
import ctypes, sys
import numpy as np, torch
sys.path[:0] = [sys.argv[1] + "/ggml-compiler_amd", sys.argv[1] + "/oracle"]
import oracle as orc
from ggml_compiler_amd import _lib, ops
lib = _lib.load()
torch.cuda.set_device(0)
p = lambda t: ctypes.c_void_p(t.data_ptr())
checked = 0
for t, M, N, K in (("q4_0", 8, 700, 4096), ("q8_0", 40, 256, 2048)):
    raw = orc.quantize(orc.normal((N, K), seed=60 + M, std=0.02), t)
    qw = ops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    x = torch.from_numpy(orc.normal((M, K), seed=70 + M)).cuda()
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the process's first noalloc call of this shape: under capture
        rc = lib.gcq_mul_mat_noalloc(qw.type, p(qw.data), N, K, p(x), K, M, p(y), N, ctypes.c_void_p(s.cuda_stream))
    assert rc == 0, lib.gcq_last_error().decode()
    nbytes = int(lib.gcq_mul_mat_workspace(qw.type, M, K))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda")
    want = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.gcq_mul_mat(qw.type, p(qw.data), N, K, p(x), K, M, p(want), N, p(ws), ws.numel(), st) == 0
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), (t, M, rep)
        checked += 1
print("replays equal", checked)
"""


def test_noalloc_first_call_under_graph_capture(gops):
    """A fresh process (so that the call is its first on the device) captures gcq_mul_mat_noalloc
    into a HIP graph and replays it three times with other work between the replays; every replay
    equals gcq_mul_mat with a workspace."""
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", _CAPTURE, str(root)], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "replays equal 6" in r.stdout
