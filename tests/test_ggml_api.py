"""CPU-side checks of the ggml API subset (include/ggml.h): type sizes, tensor strides, views,
permutes and reshapes against numpy's reading of the same bytes, op result shapes and the
errors that replace ggml's aborts, and graph expansion order. No device is touched: tensors
here live in host memory (no_alloc = false) or have no memory at all."""

import ctypes

import numpy as np
import pytest

from ggml_compiler_amd import ggml as G


@pytest.fixture
def ctx():
    c = G.init(no_alloc=False)
    yield c
    G.lib().ggml_free(c)


def _view(t) -> np.ndarray:
    """What a tensor's ne / nb / data describe, read with numpy (f32)."""
    tt = G.T(t)
    base = G.T(tt.view_src) if tt.view_src else tt
    n_base = G.lib().ggml_nbytes(ctypes.cast(ctypes.pointer(base), ctypes.c_void_p))
    buf = (ctypes.c_char * n_base).from_address(base.data)
    arr = np.frombuffer(buf, np.uint8)
    shape = tuple(reversed(tt.ne))
    st = tuple(reversed(tt.nb))
    return np.lib.stride_tricks.as_strided(arr[tt.view_offs:].view(np.float32), shape, st)


def _fill(t, a):
    a = np.ascontiguousarray(a, np.float32)
    ctypes.memmove(G.T(t).data, a.ctypes.data, a.nbytes)


def test_type_traits():
    g = G.lib()
    for t, blck, size, name in [(0, 1, 4, b"f32"), (1, 1, 2, b"f16"), (2, 32, 18, b"q4_0"), (8, 32, 34, b"q8_0"),
                                (12, 256, 144, b"q4_K"), (14, 256, 210, b"q6_K"), (15, 256, 292, b"q8_K"),
                                (26, 1, 4, b"i32")]:
        assert (g.ggml_blck_size(t), g.ggml_type_size(t), g.ggml_type_name(t)) == (blck, size, name)
        assert g.ggml_is_quantized(t) == (blck > 1)
    # compiler.py:80-84 row sizes
    assert g.ggml_row_size(2, 4096) == 2304 and g.ggml_row_size(8, 4096) == 4352 and g.ggml_row_size(12, 14336) == 8064


def test_new_tensor_strides(ctx):
    g = G.lib()
    w = g.ggml_new_tensor_2d(ctx, G.Q4_0, 4096, 10)
    assert G.shape(w) == (4096, 10, 1, 1)
    assert G.strides(w) == (18, 2304, 23040, 23040)
    assert g.ggml_nbytes(w) == 23040 and g.ggml_nrows(w) == 10 and g.ggml_is_contiguous(w)
    assert not g.ggml_new_tensor_2d(ctx, G.Q4_0, 100, 2)
    assert "multiple of q4_0's block" in g.ggml_last_error().decode()
    x = g.ggml_new_tensor_3d(ctx, G.F32, 4, 3, 2)
    assert G.strides(x) == (4, 16, 48, 96) and g.ggml_nbytes(x) == 96


def test_views_permutes_reshapes_read_like_numpy(ctx):
    g = G.lib()
    a = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)  # ggml ne = [5, 4, 3, 2]
    t = g.ggml_new_tensor_4d(ctx, G.F32, 5, 4, 3, 2)
    _fill(t, a)
    assert np.array_equal(_view(t), a)
    p = g.ggml_permute(ctx, t, 0, 2, 1, 3)  # ggml dims 1 <-> 2
    assert G.shape(p) == (5, 3, 4, 2)
    assert np.array_equal(_view(p), a.transpose(0, 2, 1, 3))
    assert not g.ggml_is_contiguous(p) and g.ggml_is_permuted(p)
    tr = g.ggml_transpose(ctx, t)
    assert np.array_equal(_view(tr), a.swapaxes(2, 3))
    assert g.ggml_is_transposed(tr)
    v = g.ggml_view_3d(ctx, t, 5, 2, 3, 20, 80, 20)  # rows 1..2 of each [4, 5] matrix, first batch
    assert np.array_equal(_view(v)[0], a[0, :, 1:3, :])
    vv = g.ggml_view_2d(ctx, p, 5, 2, G.T(p).nb[1], G.T(p).nb[2])  # a view of a view resolves to the base
    assert G.T(vv).view_src == t and G.T(vv).view_offs == 20
    assert np.array_equal(_view(vv)[0, 0], a[0, 0:2, 1, :])
    r = g.ggml_reshape_2d(ctx, t, 20, 6)
    assert np.array_equal(_view(r)[0, 0], a.reshape(6, 20))
    assert not g.ggml_reshape_2d(ctx, p, 20, 6)
    assert "not contiguous" in g.ggml_last_error().decode()
    assert not g.ggml_view_1d(ctx, t, 200, 0)
    assert "exceeds" in g.ggml_last_error().decode()
    assert not g.ggml_permute(ctx, t, 0, 0, 1, 2)


def test_op_shapes_and_errors(ctx):
    g = G.lib()
    W = g.ggml_new_tensor_2d(ctx, G.Q4_0, 256, 64)
    x = g.ggml_new_tensor_3d(ctx, G.F32, 256, 5, 2)
    y = g.ggml_mul_mat(ctx, W, x)
    assert G.shape(y) == (64, 5, 2, 1) and G.T(y).type == G.F32 and G.T(y).op == G.OP["MUL_MAT"]
    assert not g.ggml_mul_mat(ctx, W, g.ggml_new_tensor_2d(ctx, G.F32, 128, 1))
    assert "cannot multiply" in g.ggml_last_error().decode()
    assert not g.ggml_mul_mat(ctx, None, x)  # a NULL operand propagates
    q = g.ggml_new_tensor_3d(ctx, G.F32, 128, 1, 32)
    k = g.ggml_new_tensor_3d(ctx, G.F16, 128, 512, 8)
    m = g.ggml_new_tensor_2d(ctx, G.F16, 512, 1)
    o = g.ggml_flash_attn_ext(ctx, q, k, k, m, 0.1, 0.0, 0.0)
    assert G.shape(o) == (128, 32, 1, 1)
    assert not g.ggml_flash_attn_ext(ctx, q, k, k, g.ggml_new_tensor_2d(ctx, G.F16, 256, 1), 0.1, 0.0, 0.0)
    assert "mask" in g.ggml_last_error().decode()
    pos = g.ggml_new_tensor_1d(ctx, G.I32, 1)
    r = g.ggml_rope_ext(ctx, q, g.ggml_new_tensor_1d(ctx, G.I32, 32), None, 128, 2, 0, 1e4, 1, 0, 1, 32, 1)
    assert G.shape(r) == (128, 1, 32, 1)
    assert not g.ggml_rope_ext(ctx, q, pos, None, 128, 2, 0, 1e4, 1, 0, 1, 32, 1)
    cache = g.ggml_new_tensor_3d(ctx, G.F16, 128, 512, 8)
    kr = g.ggml_new_tensor_3d(ctx, G.F32, 128, 1, 8)
    w = g.ggml_set_rows(ctx, cache, kr, pos)
    tw = G.T(w)
    assert tw.view_src == cache and tw.data == G.T(cache).data and tw.src[2] == cache
    assert G.shape(g.ggml_get_rows(ctx, W, g.ggml_new_tensor_1d(ctx, G.I32, 3))) == (256, 3, 1, 1)
    b = g.ggml_new_tensor_1d(ctx, G.F32, 64)
    assert G.shape(g.ggml_add(ctx, y, b)) == (64, 5, 2, 1)
    assert not g.ggml_add(ctx, b, y)
    assert "broadcast" in g.ggml_last_error().decode()
    assert G.shape(g.ggml_argmax(ctx, g.ggml_new_tensor_2d(ctx, G.F32, 100, 4))) == (4, 1, 1, 1)
    c = g.ggml_cast(ctx, kr, G.F16)
    assert G.T(c).type == G.F16 and g.ggml_is_contiguous(c)


def test_graph_order_and_leafs(ctx):
    g = G.lib()
    x = g.ggml_new_tensor_1d(ctx, G.F32, 32)
    w = g.ggml_new_tensor_1d(ctx, G.F32, 32)
    n = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, x, 1e-5), w)
    s = g.ggml_swiglu_split(ctx, n, n)
    gr = g.ggml_new_graph(ctx)
    g.ggml_build_forward_expand(gr, s)
    g.ggml_build_forward_expand(gr, s)  # a second expand adds nothing
    ops = [G.T(g.ggml_graph_node(gr, i)).op for i in range(g.ggml_graph_n_nodes(gr))]
    assert ops == [G.OP["RMS_NORM"], G.OP["MUL"], G.OP["GLU"]]
    assert g.ggml_graph_node(gr, -1) == s
    g.ggml_graph_clear(gr)
    assert g.ggml_graph_n_nodes(gr) == 0


def test_named_lookup_and_status_strings(ctx):
    g = G.lib()
    t = g.ggml_set_name(g.ggml_new_tensor_1d(ctx, G.F32, 4), b"blk.0.attn_norm")
    assert g.ggml_get_tensor(ctx, b"blk.0.attn_norm") == t
    assert g.ggml_get_tensor(ctx, b"nope") is None
    assert g.ggml_get_first_tensor(ctx) == t and g.ggml_get_next_tensor(ctx, t) is None
    assert b"success" in g.ggml_status_to_string(0)
    assert b"failed" in g.ggml_status_to_string(-1)
