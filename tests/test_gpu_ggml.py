"""The ggml API subset on the HIP backend: graphs built with ggml calls, allocated by the graph
allocator and run by ggml_backend_graph_compute, against the oracle (1e-3 by the reference's parity
metric for float results, bit-exact for integer and byte results) and against libgcq's direct
entry points, which run the same kernels (bit-exact). Covers every supported node, each fusion
chain and its unfused twin, HIP-graph replay with changing inputs, the allocator's memory reuse,
the errors for nodes off the path, and a Llama decoder built node by node as the reference's
decode stage builds it (ggml_compiler/llm.py:361-444) against the oracle's run of that model."""

import math

import numpy as np
import pytest
import torch

from conftest import to_np
from ggml_compiler_amd import ggml as G

pytestmark = pytest.mark.gpu
TOL = 1e-3
TOL_LM = 1e-2
NP = {0: np.float32, 1: np.uint16, 26: np.int32}


@pytest.fixture(scope="module")
def be(gops):
    b = G.Backend(0)
    yield b
    b.close()


class Graph:
    """Leaves in one device buffer, nodes built by `build`, allocated and computed."""

    def __init__(self, be, leaves, build, outputs=(), use_graphs=True):
        g = G.lib()
        self.g, self.be = g, be
        self.wctx = G.init()
        self.L = {}
        for name, (typ, ne, data) in leaves.items():
            t = g.ggml_new_tensor(self.wctx, typ, len(ne), (G.ctypes.c_int64 * len(ne))(*ne))
            G.T(t)
            g.ggml_set_name(t, name.encode())
            self.L[name] = t
        self.buf = g.ggml_backend_alloc_ctx_tensors(self.wctx, be.be)
        assert self.buf, g.ggml_last_error()
        for name, (typ, ne, data) in leaves.items():
            if data is not None:
                G.set_data(self.L[name], data)
        self.ctx = G.init()
        built = build(g, self.ctx, self.L)
        built = built if isinstance(built, list) else [built]
        self.built = built
        self.out = built[0]
        for t in outputs:
            g.ggml_set_output(t(self) if callable(t) else t)
        self.graph = g.ggml_new_graph(self.ctx)
        for t in built:
            G.T(t)
            g.ggml_build_forward_expand(self.graph, t)
        self.ga = g.ggml_gallocr_new(g.ggml_backend_get_default_buffer_type(be.be))
        assert g.ggml_gallocr_alloc_graph(self.ga, self.graph), g.ggml_last_error()
        g.ggml_backend_hip_set_use_graphs(be.be, use_graphs)

    def run(self, t=None):
        G.compute(self.be.be, self.graph)
        t = self.out if t is None else t
        return G.get_data(t, NP[G.T(t).type])

    def close(self):
        self.g.ggml_gallocr_free(self.ga)
        self.g.ggml_free(self.ctx)
        self.g.ggml_backend_buffer_free(self.buf)
        self.g.ggml_free(self.wctx)
        self.g.ggml_backend_hip_set_use_graphs(self.be.be, True)


def _weight(orc, t, N, K, seed):
    return orc.quantize(orc.normal((N, K), seed=seed, std=0.02), t)


# ------------------------------------------------------------------------------- mul_mat

@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("M", [1, 3, 16])
def test_mul_mat_node(be, gops, orc, t, M):
    """The mul_mat node against the oracle, and bit-exact against gcq_mul_mat (the same kernels:
    decode-row GEMV, GEMV, MFMA GEMM or K-quant row groups); the weight's ggml bytes read back."""
    N, K = 300, 1024
    tid = orc.TYPES[t]
    raw = _weight(orc, t, N, K, 40 + M)
    x = orc.normal((M, K), seed=41)
    gr = Graph(be, {"w": (tid, [K, N], raw), "x": (G.F32, [K, M], x)},
               lambda g, ctx, L: g.ggml_mul_mat(ctx, L["w"], L["x"]))
    y = gr.run().reshape(M, N)
    back = G.get_data(gr.L["w"], np.uint8)
    gr.close()
    assert np.array_equal(back.reshape(-1), raw.reshape(-1))  # packed on set, unpacked on get
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    assert np.array_equal(y, to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda())))


@pytest.mark.parametrize("t", ["q4_K", "q5_K", "q6_K"])
def test_kquant_row_mul_mat_add(be, gops, orc, t):
    """One row times a K-quant weight, then add(residual): the residual folds into the one-launch
    row kernel's store (read through the scalar unit); bit-equal to the product plus the residual
    added on the host in f32."""
    N, K = 300, 1024
    tid = orc.TYPES[t]
    raw = _weight(orc, t, N, K, 60)
    x = orc.normal((1, K), seed=61)
    r = orc.normal((1, N), seed=62)
    gr = Graph(be, {"w": (tid, [K, N], raw), "x": (G.F32, [K, 1], x), "r": (G.F32, [N, 1], r)},
               lambda g, ctx, L: g.ggml_add(ctx, L["r"], g.ggml_mul_mat(ctx, L["w"], L["x"])))
    y = gr.run().reshape(1, N)
    gr.close()
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    y0 = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda())).reshape(1, N)
    assert np.array_equal(y, (y0 + r).astype(np.float32))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K) + r) < TOL


@pytest.mark.parametrize("M", [1, 4, 12])
@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
def test_norm_mul_mat_add_chain(be, orc, t, M):
    """rms_norm -> mul(w) -> mul_mat -> add(residual) folded into one GEMV / GEMM launch sequence,
    against the oracle and against the same graph with the chain broken (every node launched)."""
    N, K = 512, 2048
    tid = orc.TYPES[t]
    raw = _weight(orc, t, N, K, 50)
    x = orc.normal((M, K), seed=51)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=52)).astype(np.float32)
    r = orc.normal((M, N), seed=53)
    leaves = {"w": (tid, [K, N], raw), "x": (G.F32, [K, M], x), "nw": (G.F32, [K], nw), "r": (G.F32, [N, M], r)}
    keep = {}

    def build(g, ctx, L):
        keep["n"] = g.ggml_rms_norm(ctx, L["x"], 1e-5)
        keep["m"] = g.ggml_mul(ctx, keep["n"], L["nw"])
        keep["mm"] = g.ggml_mul_mat(ctx, L["w"], keep["m"])
        return g.ggml_add(ctx, L["r"], keep["mm"])

    fused = Graph(be, leaves, build)
    yf = fused.run().reshape(M, N)
    fused.close()
    split = Graph(be, leaves, build, outputs=[lambda s: keep["n"], lambda s: keep["mm"]])
    ys = split.run().reshape(M, N)
    split.close()
    ref = orc.mul_mat(raw, t, orc.rms_norm(x, 1e-5) * nw[None, :], K) + r
    assert orc.parity(yf, ref) < TOL
    assert orc.parity(ys, ref) < TOL
    assert orc.parity(yf, ys) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
def test_norm_row_folded_into_several_gemvs(be, orc, t):
    """One normalized row read by three mul_mats (q / k / v of a decode step), one of them followed
    by an add: each GEMV normalizes x in its prologue; against the oracle and the unfolded graph."""
    K = 2048
    tid = orc.TYPES[t]
    Ns = (512, 256, 256)
    raws = [_weight(orc, t, N, K, 130 + i) for i, N in enumerate(Ns)]
    x = orc.normal((1, K), seed=134)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=135)).astype(np.float32)
    r = orc.normal((1, Ns[2]), seed=136)
    leaves = {"x": (G.F32, [K, 1], x), "nw": (G.F32, [K], nw), "r": (G.F32, [Ns[2], 1], r)}
    for i, (N, raw) in enumerate(zip(Ns, raws)):
        leaves[f"w{i}"] = (tid, [K, N], raw)
    keep = {}

    def build(g, ctx, L):
        keep["m"] = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5), L["nw"])
        a = g.ggml_mul_mat(ctx, L["w0"], keep["m"])
        b = g.ggml_mul_mat(ctx, L["w1"], keep["m"])
        c = g.ggml_add(ctx, g.ggml_mul_mat(ctx, L["w2"], keep["m"]), L["r"])
        for u in (a, b, c):
            g.ggml_set_output(u)
        return [a, b, c]

    got = {}
    for name, outs in (("fold", ()), ("split", [lambda s: keep["m"]])):
        gr = Graph(be, leaves, build, outputs=outs)
        gr.run()
        got[name] = [G.get_data(gr.built[i], np.float32) for i in range(3)]
        gr.close()
    xn = orc.rms_norm(x, 1e-5) * nw[None, :]
    refs = [orc.mul_mat(raws[0], t, xn, K)[0], orc.mul_mat(raws[1], t, xn, K)[0],
            orc.mul_mat(raws[2], t, xn, K)[0] + r[0]]
    for i in range(3):
        assert orc.parity(got["fold"][i], refs[i]) < TOL, i
        assert orc.parity(got["split"][i], refs[i]) < TOL, i


@pytest.mark.parametrize("t", ["q4_0", "q8_0"])
@pytest.mark.parametrize("Ns,K", [((512, 128, 128), 4096), ((1024, 1024), 2048), ((640, 64, 192), 14336)])
def test_sibling_gemvs_in_one_launch(be, gops, orc, t, Ns, K):
    """Two or three mul_mats of one normalized row with no add (q / k / v, gate / up) run as one
    decode-row launch over the weights' rows; each result equals gcq_rms_norm_mul_mat on its weight
    alone bit for bit, and the oracle within 1e-3."""
    tid = orc.TYPES[t]
    raws = [_weight(orc, t, N, K, 140 + i) for i, N in enumerate(Ns)]
    x = orc.normal((1, K), seed=144)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=145)).astype(np.float32)
    leaves = {"x": (G.F32, [K, 1], x), "nw": (G.F32, [K], nw)}
    for i, (N, raw) in enumerate(zip(Ns, raws)):
        leaves[f"w{i}"] = (tid, [K, N], raw)

    def build(g, ctx, L):
        m = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5), L["nw"])
        outs = [g.ggml_mul_mat(ctx, L[f"w{i}"], m) for i in range(len(Ns))]
        for u in outs:
            g.ggml_set_output(u)
        return outs

    gr = Graph(be, leaves, build)
    gr.run()
    got = [G.get_data(gr.built[i], np.float32) for i in range(len(Ns))]
    gr.close()
    xd, nwd = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    xn = orc.rms_norm(x, 1e-5) * nw[None, :]
    for i, raw in enumerate(raws):
        qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
        assert np.array_equal(got[i], to_np(gops.rms_norm_mul_mat(qw, xd, nwd, 1e-5)).reshape(-1)), i
        assert orc.parity(got[i], orc.mul_mat(raw, t, xn, K)[0]) < TOL, i


@pytest.mark.parametrize("t", ["q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("Ns,K", [((512, 128, 128), 4096), ((1024, 1024), 2048), ((640, 64, 192), 8192)])
def test_kquant_sibling_gemvs_in_one_launch(be, orc, t, Ns, K):
    """Two or three mul_mats of one normalized row by Q4_K / Q5_K weights run as one K-quant row
    launch over the weights' rows (the row normalized and quantized to Q8_K in it); each result
    equals the graph of that weight alone (rms_norm -> mul -> mul_mat, one launch with the same
    prologue) bit for bit, and the oracle within 1e-3."""
    tid = orc.TYPES[t]
    raws = [_weight(orc, t, N, K, 160 + i) for i, N in enumerate(Ns)]
    x = orc.normal((1, K), seed=164)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=165)).astype(np.float32)
    leaves = {"x": (G.F32, [K, 1], x), "nw": (G.F32, [K], nw)}
    for i, (N, raw) in enumerate(zip(Ns, raws)):
        leaves[f"w{i}"] = (tid, [K, N], raw)

    def build(g, ctx, L):
        m = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5), L["nw"])
        outs = [g.ggml_mul_mat(ctx, L[f"w{i}"], m) for i in range(len(Ns))]
        for u in outs:
            g.ggml_set_output(u)
        return outs

    gr = Graph(be, leaves, build)
    gr.run()
    got = [G.get_data(gr.built[i], np.float32) for i in range(len(Ns))]
    gr.close()
    xn = orc.rms_norm(x, 1e-5) * nw[None, :]
    for i, (N, raw) in enumerate(zip(Ns, raws)):
        one = Graph(be, {"x": leaves["x"], "nw": leaves["nw"], "w": (tid, [K, N], raw)},
                    lambda g, ctx, L: g.ggml_mul_mat(ctx, L["w"], g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5),
                                                                             L["nw"])))
        want = one.run().reshape(-1)
        one.close()
        assert np.array_equal(got[i], want), i
        assert orc.parity(got[i], orc.mul_mat(raw, t, xn, K)[0]) < TOL, i


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K", "q4_K/q6_K"])
def test_qkv_rope_cache_writes_in_one_launch(be, orc, t):
    """The decode step's q / k / v GEMVs of one normalized row, the q and k ropes and the k / v
    set_rows into f16 caches (built as the reference builds them) run as one launch whose epilogue
    ropes and writes the caches (q4_K/q6_K: v in Q6_K, as Q4_K_M files store it in some layers:
    the q / k launch, then the v launch writing its cache); the roped q and both caches equal the
    unfused graph's (each intermediate marked as an output, which keeps them apart) to 1e-6. The
    row is an embedding row (get_rows), whose launch also builds the epilogue's rotation table."""
    K, H, Hkv, D, ctx, p = 2048, 8, 2, 128, 64, 13
    ts = t.split("/") if "/" in t else [t, t]
    wts = [ts[0], ts[0], ts[1]]
    raws = [_weight(orc, wt, N, K, 150 + i) for i, (wt, N) in enumerate(zip(wts, (H * D, Hkv * D, Hkv * D)))]
    x = orc.normal((1, K), seed=154)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=155)).astype(np.float32)
    emb = np.concatenate([orc.normal((2, K), seed=156), x])  # x: row 2 of an embedding table
    leaves = {"emb": (G.F32, [K, 3], emb), "tok": (G.I32, [1], np.array([2], np.int32)), "nw": (G.F32, [K], nw),
              "pos": (G.I32, [1], np.array([p], np.int32)), "ck": (G.F16, [D, ctx, Hkv], None),
              "cv": (G.F16, [D, ctx, Hkv], None)}
    for i, raw in enumerate(raws):
        leaves[f"w{i}"] = (orc.TYPES[wts[i]], [K, raw.shape[0]], raw)
    res = {}
    for split in (False, True):
        keep = {}

        def build(g, ctx_, L):
            xr = g.ggml_get_rows(ctx_, L["emb"], L["tok"])  # with the fused launch: one of the rotation table
            n = g.ggml_mul(ctx_, g.ggml_rms_norm(ctx_, xr, 1e-5), L["nw"])
            q, k, v = (g.ggml_mul_mat(ctx_, L[f"w{i}"], n) for i in range(3))
            rp = (D, 2, 0, 500000.0, 1.0, 0.0, 1.0, 32.0, 1.0)
            q = g.ggml_rope_ext(ctx_, g.ggml_reshape_3d(ctx_, q, D, H, 1), L["pos"], None, *rp)
            k = g.ggml_rope_ext(ctx_, g.ggml_reshape_3d(ctx_, k, D, Hkv, 1), L["pos"], None, *rp)
            v = g.ggml_reshape_3d(ctx_, v, D, Hkv, 1)
            kw = g.ggml_set_rows(ctx_, L["ck"], g.ggml_permute(ctx_, k, 0, 2, 1, 3), L["pos"])
            vw = g.ggml_set_rows(ctx_, L["cv"], g.ggml_permute(ctx_, v, 0, 2, 1, 3), L["pos"])
            keep["k"] = k
            out = g.ggml_cont(ctx_, g.ggml_permute(ctx_, q, 0, 2, 1, 3))
            return [out, kw, vw]

        gr = Graph(be, leaves, build, outputs=[lambda s: keep["k"]] if split else ())
        for name in ("ck", "cv"):
            G.checked(G.lib().ggml_backend_tensor_memset, gr.L[name], 0, 0, G.nbytes(gr.L[name]))
        gr.run()
        res[split] = [G.get_data(gr.built[0], np.float32), G.get_data(gr.L["ck"], np.uint16),
                      G.get_data(gr.L["cv"], np.uint16)]
        gr.close()
    assert orc.parity(res[False][0], res[True][0]) < 1e-6
    for i in (1, 2):
        a = res[False][i].view(np.float16).astype(np.float32).reshape(Hkv, ctx, D)
        b = res[True][i].view(np.float16).astype(np.float32).reshape(Hkv, ctx, D)
        assert not a[:, np.arange(ctx) != p].any() and not b[:, np.arange(ctx) != p].any()
        assert orc.parity(a[:, p], b[:, p]) < 1e-3  # f16 rows: one f16 ulp where a last f32 bit differs


@pytest.mark.parametrize("M", [1, 9])
def test_swiglu_mul_mat_add_chain(be, orc, M):
    N, F = 256, 1024
    raw = _weight(orc, "q4_0", N, F, 60)
    gt = orc.normal((M, F), seed=61)
    up = orc.normal((M, F), seed=62)
    r = orc.normal((M, N), seed=63)
    gr = Graph(be, {"w": (G.Q4_0, [F, N], raw), "g": (G.F32, [F, M], gt), "u": (G.F32, [F, M], up),
                    "r": (G.F32, [N, M], r)},
               lambda g, ctx, L: g.ggml_add(ctx, L["r"], g.ggml_mul_mat(ctx, L["w"],
                                                                        g.ggml_swiglu_split(ctx, L["g"], L["u"]))))
    y = gr.run().reshape(M, N)
    gr.close()
    assert orc.parity(y, orc.mul_mat(raw, "q4_0", orc.swiglu(gt, up), F) + r) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q8_0"])
@pytest.mark.parametrize("F", [1024, 14336])
def test_swiglu_prologue_equals_separate_launches(be, gops, orc, t, F):
    """One token: swiglu -> mul_mat -> add runs as one decode-row GEMV whose prologue computes
    silu(g) * u and its Q8_0 codes; equal bit for bit to gcq_swiglu_q8 + gcq_mul_mat_q (+ add)."""
    N = 512
    raw = _weight(orc, t, N, F, 64)
    gt, up, r = orc.normal((1, F), seed=65), orc.normal((1, F), seed=66), orc.normal((1, N), seed=67)
    tid = orc.TYPES[t]
    gr = Graph(be, {"w": (tid, [F, N], raw), "g": (G.F32, [F, 1], gt), "u": (G.F32, [F, 1], up),
                    "r": (G.F32, [N, 1], r)},
               lambda g, ctx, L: g.ggml_add(ctx, L["r"], g.ggml_mul_mat(ctx, L["w"],
                                                                        g.ggml_swiglu_split(ctx, L["g"], L["u"]))))
    y = gr.run().reshape(1, N)
    gr.close()
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, F)
    act = gops.swiglu_q8(torch.from_numpy(gt).cuda(), torch.from_numpy(up).cuda())
    want = to_np(gops.mul_mat_q(qw, act, 1, res=torch.from_numpy(r).cuda()))
    assert np.array_equal(y, want)
    assert orc.parity(y, orc.mul_mat(raw, t, orc.swiglu(gt, up), F) + r) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("F,K", [(512, 2048), (14336, 4096)])
def test_gate_up_swiglu_in_one_launch(be, orc, t, F, K):
    """The FFN of one token as the reference builds it: rms_norm -> mul -> gate and up mul_mats ->
    swiglu_split -> down mul_mat -> add. The gate / up GEMVs run as one launch writing silu(gate) *
    up (the row pairs read from the two weights); equal bit for bit to the graph with the
    normalized row kept as an output (gate and up then launched as a pair with separate results,
    the swiglu in the down GEMV's prologue), and the oracle within 1e-3."""
    tid = orc.TYPES[t]
    N = 256
    wg, wu, wd = _weight(orc, t, F, K, 150), _weight(orc, t, F, K, 151), _weight(orc, t, N, F, 152)
    x = orc.normal((1, K), seed=153)
    nw = (1.0 + 0.1 * orc.normal((K,), seed=154)).astype(np.float32)
    r = orc.normal((1, N), seed=155)
    leaves = {"x": (G.F32, [K, 1], x), "nw": (G.F32, [K], nw), "wg": (tid, [K, F], wg), "wu": (tid, [K, F], wu),
              "wd": (tid, [F, N], wd), "r": (G.F32, [N, 1], r)}
    keep = {}

    def build(g, ctx, L):
        keep["m"] = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5), L["nw"])
        h = g.ggml_swiglu_split(ctx, g.ggml_mul_mat(ctx, L["wg"], keep["m"]), g.ggml_mul_mat(ctx, L["wu"], keep["m"]))
        return g.ggml_add(ctx, g.ggml_mul_mat(ctx, L["wd"], h), L["r"])

    got = {}
    for name, outs in (("fused", ()), ("split", [lambda s: keep["m"]])):
        gr = Graph(be, leaves, build, outputs=outs)
        got[name] = gr.run().reshape(1, N)
        gr.close()
    if t in ("q4_K", "q5_K", "q6_K") and F > 8192:
        # the split graph's K-quant GEMVs of more than 8192 rows run batched after a separate
        # quantization: the same int32 dots, summed in another order
        assert orc.parity(got["fused"], got["split"]) < 1e-4
    else:
        assert np.array_equal(got["fused"], got["split"])
    xn = orc.rms_norm(x, 1e-5) * nw[None, :]
    h = orc.swiglu(orc.mul_mat(wg, t, xn, K), orc.mul_mat(wu, t, xn, K))
    assert orc.parity(got["fused"], orc.mul_mat(wd, t, h, F) + r) < TOL


# ----------------------------------------------------------------------------- attention

@pytest.mark.parametrize("Sq,n_kv,H,Hkv,D", [(1, 300, 8, 2, 128), (5, 130, 4, 4, 64), (1, 1, 32, 8, 128),
                                             (3, 513, 16, 2, 256)])
def test_flash_attn_over_cache_views(be, orc, Sq, n_kv, H, Hkv, D):
    """q as a permuted view [D, Sq, H] of [D, H, Sq]; K and V the first n_kv rows of f16 caches
    [D, ctx, Hkv]; a causal f16 mask with -inf (every query row sees at least one key)."""
    ctx_rows = n_kv + 64
    q = orc.normal((Sq, H, D), seed=70)
    kc = orc.fp32_to_fp16(orc.normal((Hkv, ctx_rows, D), seed=71))
    vc = orc.fp32_to_fp16(orc.normal((Hkv, ctx_rows, D), seed=72))
    pos0 = n_kv - Sq
    mask = np.where(np.arange(n_kv)[None, :] <= pos0 + np.arange(Sq)[:, None], 0.0, -np.inf).astype(np.float32)
    m16 = orc.fp32_to_fp16(mask)
    scale = 1.0 / math.sqrt(D)

    def build(g, ctx, L):
        qp = g.ggml_permute(ctx, L["q"], 0, 2, 1, 3)
        kv = g.ggml_view_3d(ctx, L["k"], D, n_kv, Hkv, 2 * D, 2 * D * ctx_rows, 0)
        vv = g.ggml_view_3d(ctx, L["v"], D, n_kv, Hkv, 2 * D, 2 * D * ctx_rows, 0)
        o = g.ggml_flash_attn_ext(ctx, qp, kv, vv, L["m"], scale, 0.0, 0.0)
        g.ggml_prec_set_acc(o, G.PREC_F32)
        return o

    gr = Graph(be, {"q": (G.F32, [D, H, Sq], q), "k": (G.F16, [D, ctx_rows, Hkv], kc),
                    "v": (G.F16, [D, ctx_rows, Hkv], vc), "m": (G.F16, [n_kv, Sq], m16)}, build)
    assert G.lib().ggml_backend_supports_op(be.be, gr.out)
    y = gr.run().reshape(Sq, H, D)
    gr.close()
    ref = orc.flash_attn_ext(q.transpose(1, 0, 2), kc[:, :n_kv], vc[:, :n_kv], m16, scale)
    assert orc.parity(y, ref) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("n_kv,H,Hkv,D", [(40, 32, 8, 128), (3000, 32, 8, 128), (700, 8, 8, 64), (5, 8, 2, 128)])
def test_attention_merged_into_output_projection(be, orc, n_kv, H, Hkv, D, t):
    """flash_attn_ext of one query row -> reshape -> mul_mat -> add: the decode kernel's split
    partials merged in the GEMV prologue (one split: its row; Q4_K / Q5_K: merged and quantized to
    Q8_K by every wavefront, a super-block each), against the oracle and the unfused graph (the
    attention output flagged as an output)."""
    ctx_rows, E = n_kv + 16, 512
    q = orc.normal((1, H, D), seed=140)
    kc = orc.fp32_to_fp16(orc.normal((Hkv, ctx_rows, D), seed=141))
    vc = orc.fp32_to_fp16(orc.normal((Hkv, ctx_rows, D), seed=142))
    m16 = orc.fp32_to_fp16(np.where(np.arange(n_kv) < n_kv - 3, 0.0, -np.inf).astype(np.float32)[None, :])
    wo = _weight(orc, t, E, H * D, 143)
    r = orc.normal((1, E), seed=144)
    scale = 1.0 / math.sqrt(D)
    keep = {}

    def build(g, ctx, L):
        kv = g.ggml_view_3d(ctx, L["k"], D, n_kv, Hkv, 2 * D, 2 * D * ctx_rows, 0)
        vv = g.ggml_view_3d(ctx, L["v"], D, n_kv, Hkv, 2 * D, 2 * D * ctx_rows, 0)
        keep["a"] = g.ggml_flash_attn_ext(ctx, g.ggml_permute(ctx, L["q"], 0, 2, 1, 3), kv, vv, L["m"], scale, 0.0, 0.0)
        return g.ggml_add(ctx, g.ggml_mul_mat(ctx, L["w"], g.ggml_reshape_2d(ctx, keep["a"], D * H, 1)), L["r"])

    leaves = {"q": (G.F32, [D, H, 1], q), "k": (G.F16, [D, ctx_rows, Hkv], kc), "v": (G.F16, [D, ctx_rows, Hkv], vc),
              "m": (G.F16, [n_kv, 1], m16), "w": (orc.TYPES[t], [H * D, E], wo), "r": (G.F32, [E, 1], r)}
    got = {}
    for name, outs in (("fused", ()), ("split", [lambda s: keep["a"]])):
        gr = Graph(be, leaves, build, outputs=outs)
        got[name] = gr.run().copy()
        gr.close()
    att = orc.flash_attn_ext(q.transpose(1, 0, 2), kc[:, :n_kv], vc[:, :n_kv], m16, scale).reshape(1, H * D)
    ref = orc.mul_mat(wo, t, att, H * D) + r
    assert orc.parity(got["fused"].reshape(1, E), ref) < TOL
    assert orc.parity(got["split"].reshape(1, E), ref) < TOL


def test_supports_op_and_off_path_errors(be, orc):
    g = G.lib()
    ctx = G.init()
    q = g.ggml_new_tensor_3d(ctx, G.F32, 96, 1, 4)
    k = g.ggml_new_tensor_3d(ctx, G.F16, 96, 64, 4)
    assert not g.ggml_backend_supports_op(be.be, g.ggml_flash_attn_ext(ctx, q, k, k, None, 0.1, 0.0, 0.0))
    w = g.ggml_new_tensor_2d(ctx, G.F32, 64, 8)
    x = g.ggml_new_tensor_2d(ctx, G.F32, 64, 1)
    assert g.ggml_backend_supports_op(be.be, g.ggml_mul_mat(ctx, w, x))  # activation x activation
    xh = g.ggml_new_tensor_2d(ctx, G.F16, 64, 1)
    assert not g.ggml_backend_supports_op(be.be, g.ggml_mul_mat(ctx, w, xh))  # f16 rows as the second operand
    assert "needs f32 rows" in g.ggml_last_error().decode()
    rope = g.ggml_rope_ext(ctx, g.ggml_new_tensor_3d(ctx, G.F32, 64, 2, 1), g.ggml_new_tensor_1d(ctx, G.I32, 1),
                           None, 64, 0, 0, 1e4, 1, 0, 1, 32, 1)
    assert not g.ggml_backend_supports_op(be.be, rope)
    assert "NEOX" in g.ggml_last_error().decode()
    # a graph whose tensors have no device memory fails to compute, with the reason
    gr = g.ggml_new_graph(ctx)
    g.ggml_build_forward_expand(gr, g.ggml_scale(ctx, x, 2.0))
    assert g.ggml_backend_graph_compute(be.be, gr) == -1
    assert "no memory" in g.ggml_last_error().decode()
    g.ggml_free(ctx)


# ------------------------------------------------------------ activation x activation mul_mat

def _mul_mat_ref(a, b, a_f16):
    """ggml_mul_mat's closed form (ggml_compiler/ir/ops.py:201-211) in float64 over numpy arrays in
    PyTorch order: a [..., N, K], b [..., M, K] -> [..., M, N], a's batch dims repeat-interleaved
    over b's. With an f16 a, b is rounded to f16 first (ggml-cpu's vec_dot_type conversion)."""
    rank = max(a.ndim, b.ndim)
    a = a.reshape((1,) * (rank - a.ndim) + a.shape).astype(np.float64)
    b = b.reshape((1,) * (rank - b.ndim) + b.shape)
    if a_f16:
        b = b.astype(np.float16)
    b = b.astype(np.float64)
    for d in range(rank - 2):
        if a.shape[d] != b.shape[d]:
            a = np.repeat(a, b.shape[d] // a.shape[d], axis=d)
    return b @ np.swapaxes(a, -1, -2)


@pytest.mark.parametrize("ashape,bshape", [
    ((8, 16), (5, 16)),              # the reference's cases (tests/unit/test_runtime_ops.py:86-95)
    ((8, 16), (3, 5, 16)),
    ((3, 8, 16), (3, 5, 16)),
    ((2, 8, 16), (4, 5, 16)),        # grouped-query: a's batch repeat-interleaved
    ((2, 3, 8, 16), (2, 3, 5, 16)),
    ((8, 100, 128), (32, 1, 128)),   # decode Q·Kᵀ: 8 KV heads, 32 query heads, one query row
    ((2, 70, 33), (6, 130, 33)),     # ragged tiles in every direction
])
@pytest.mark.parametrize("a_type", [G.F32, G.F16])
def test_mul_mat_activations(be, orc, ashape, bshape, a_type):
    """mul_mat of an f32 / f16 first operand (an activation, a KV-cache view) by f32 rows against
    the float64 closed form: 1e-5 by the parity metric (the reference's f32 bar)."""
    a = orc.normal(ashape, seed=160)
    b = orc.normal(bshape, seed=161)
    a_dev = a.astype(np.float16).view(np.uint16) if a_type == G.F16 else a
    gr = Graph(be, {"a": (a_type, list(reversed(ashape)), a_dev), "b": (G.F32, list(reversed(bshape)), b)},
               lambda g, ctx, L: g.ggml_mul_mat(ctx, L["a"], L["b"]))
    got = gr.run()
    gr.close()
    a_used = a.astype(np.float16).astype(np.float32) if a_type == G.F16 else a
    want = _mul_mat_ref(a_used, b, a_type == G.F16)
    assert orc.parity(got.reshape(want.shape), want) < 1e-5


def test_mul_mat_strided_operands(be, orc):
    """Both operands as permuted views (q stored [Sq, H, D] read as [H, Sq, D]; k stored [n, Hkv, D]
    read as [Hkv, n, D]): no copy, same result as the contiguous product."""
    Sq, H, Hkv, n, D = 5, 8, 2, 37, 64
    q = orc.normal((Sq, H, D), seed=162)
    k = orc.normal((n, Hkv, D), seed=163)

    def build(g, ctx, L):
        qv = g.ggml_permute(ctx, L["q"], 0, 2, 1, 3)   # ggml [D, Sq, H]
        kv = g.ggml_permute(ctx, L["k"], 0, 2, 1, 3)   # ggml [D, n, Hkv]
        return g.ggml_mul_mat(ctx, kv, qv)             # [n, Sq, H]

    gr = Graph(be, {"q": (G.F32, [D, H, Sq], q), "k": (G.F32, [D, Hkv, n], k)}, build)
    got = gr.run()
    gr.close()
    want = _mul_mat_ref(k.transpose(1, 0, 2), q.transpose(1, 0, 2), False)
    assert orc.parity(got.reshape(want.shape), want) < 1e-5


@pytest.mark.parametrize("Sq,n_kv", [(1, 300), (6, 64)])
def test_eager_attention_matches_flash(be, orc, Sq, n_kv):
    """The flash-attention fallback of runtime/include/ggml_compiler_ops.h:140-148 (the attention an
    unfused program computes): mul_mat(k, q) -> soft_max_ext(mask, scale) -> mul_mat(cont(vᵀ), kq) ->
    cont(permute), with f16 K/V and grouped-query heads, against the oracle's flash_attn_ext at 1e-3."""
    D, H, Hkv = 128, 8, 2
    scale = D ** -0.5
    q = orc.normal((H, Sq, D), seed=164)
    k16 = orc.fp32_to_fp16(orc.normal((Hkv, n_kv, D), seed=165))
    v16 = orc.fp32_to_fp16(orc.normal((Hkv, n_kv, D), seed=166))
    mask = np.zeros((Sq, n_kv), np.float32)
    for s_ in range(Sq):
        mask[s_, n_kv - Sq + s_ + 1:] = -np.inf
    m16 = orc.fp32_to_fp16(mask)

    def build(g, ctx, L):
        kq = g.ggml_mul_mat(ctx, L["k"], L["q"])                       # [n_kv, Sq, H]
        g.ggml_mul_mat_set_prec(kq, 10)
        kq = g.ggml_soft_max_ext(ctx, kq, L["m"], scale, 0.0)
        vt = g.ggml_cont(ctx, g.ggml_transpose(ctx, L["v"]))          # [n_kv, D, Hkv]
        kqv = g.ggml_mul_mat(ctx, vt, kq)                              # [D, Sq, H]
        g.ggml_mul_mat_set_prec(kqv, 10)
        return g.ggml_cont(ctx, g.ggml_permute(ctx, kqv, 0, 2, 1, 3))  # [D, H, Sq]

    gr = Graph(be, {"q": (G.F32, [D, Sq, H], q), "k": (G.F16, [D, n_kv, Hkv], k16),
                    "v": (G.F16, [D, n_kv, Hkv], v16), "m": (G.F16, [n_kv, Sq], m16)}, build)
    got = gr.run().reshape(Sq, H, D)
    gr.close()
    want = orc.flash_attn_ext(q, k16, v16, m16, scale)
    assert orc.parity(got, want.reshape(Sq, H, D)) < TOL


# --------------------------------------------------------------------- rope, rows, copies

def test_rope_node_on_a_strided_view(be, orc):
    """rope of q taken as a view of a fused projection row block ([D, H, S] with a wider head
    stride), positions per token."""
    D, H, S, Hx = 128, 6, 4, 8
    big = orc.normal((S, Hx, D), seed=80)
    pos = np.array([3, 700, 1, 4095], np.int32)

    def build(g, ctx, L):
        v = g.ggml_view_3d(ctx, L["x"], D, H, S, 4 * D, 4 * D * Hx, 4 * D)  # heads 1..6
        return g.ggml_rope_ext(ctx, v, L["p"], None, D, G.ROPE_NEOX, 0, 500000.0, 1.0, 0.0, 1.0, 32.0, 1.0)

    gr = Graph(be, {"x": (G.F32, [D, Hx, S], big), "p": (G.I32, [S], pos)}, build)
    y = gr.run().reshape(S, H, D)
    gr.close()
    assert orc.parity(y, orc.rope_neox(big[:, 1:7], pos, D, 500000.0)) < TOL


def test_set_rows_then_get_rows(be, orc):
    """set_rows of a permuted f32 block into an f16 cache (exact f16 rounding, other rows untouched);
    get_rows of a Q4_0 table (bit-exact dequantized rows)."""
    D, Hkv, rows, n = 64, 2, 32, 3
    k = orc.normal((n, Hkv, D), seed=90)
    idx = np.array([5, 0, 31], np.int32)
    init = orc.fp32_to_fp16(orc.normal((Hkv, rows, D), seed=91))

    def build(g, ctx, L):
        return g.ggml_set_rows(ctx, L["c"], g.ggml_permute(ctx, L["k"], 0, 2, 1, 3), L["i"])

    gr = Graph(be, {"c": (G.F16, [D, rows, Hkv], init), "k": (G.F32, [D, Hkv, n], k), "i": (G.I32, [n], idx)},
               build)
    gr.run()
    got = G.get_data(gr.L["c"], np.uint16).reshape(Hkv, rows, D)
    gr.close()
    want = init.copy()
    want[:, idx] = orc.fp32_to_fp16(k.transpose(1, 0, 2))
    assert np.array_equal(got, want)

    V, E = 100, 256
    tab = _weight(orc, "q4_0", V, E, 92)
    ids = np.array([7, 99, 0, 7], np.int32)
    gr = Graph(be, {"t": (G.Q4_0, [E, V], tab), "i": (G.I32, [4], ids)},
               lambda g, ctx, L: g.ggml_get_rows(ctx, L["t"], L["i"]))
    y = gr.run().reshape(4, E)
    back = G.get_data(gr.L["t"], np.uint8)  # the packed weight read back as ggml bytes
    gr.close()
    assert np.array_equal(y, orc.dequantize(tab[ids], "q4_0", E))
    assert np.array_equal(back.reshape(V, -1), tab)


def test_small_steps_in_one_launch(be, orc):
    """A decode graph's first steps, the embedding row (get_rows of a Q8_0 table), the mask's f16
    cast (0 and -inf) and a strided f32 -> f16 copy, read nothing another writes and run as one
    launch of three jobs: each result bit-exact (dequantized rows, f16 rounding); then the same
    graph replayed with new indices and mask values."""
    V, E, n_kv = 50, 4096, 768
    tab = _weight(orc, "q8_0", V, E, 93)
    a = orc.normal((3, 5, 8), seed=94)
    outs = {}

    def build(g, ctx, L):
        outs["rows"] = g.ggml_get_rows(ctx, L["t"], L["i"])
        outs["mask"] = g.ggml_cast(ctx, L["m"], G.F16)
        outs["perm"] = g.ggml_cast(ctx, g.ggml_permute(ctx, L["a"], 0, 2, 1, 3), G.F16)
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    ids = np.array([49, 3], np.int32)
    mask = np.where(np.arange(n_kv) <= 517, 0.0, -np.inf).astype(np.float32)
    gr = Graph(be, {"t": (G.Q8_0, [E, V], tab), "i": (G.I32, [2], ids), "m": (G.F32, [n_kv, 1], mask),
                    "a": (G.F32, [8, 5, 3], a)}, build)
    for step in range(2):
        gr.run()
        got = {k: G.get_data(t, NP[G.T(t).type]) for k, t in outs.items()}
        assert np.array_equal(got["rows"].reshape(2, E), orc.dequantize(tab[ids], "q8_0", E)), step
        assert np.array_equal(got["mask"], orc.fp32_to_fp16(mask)), step
        assert np.array_equal(got["perm"], orc.fp32_to_fp16(a.transpose(1, 0, 2)).reshape(-1)), step
        ids = np.array([0, 17], np.int32)
        mask = np.where(np.arange(n_kv) % 3 == 0, -np.inf, 0.25 * np.arange(n_kv)).astype(np.float32)
        G.set_data(gr.L["i"], ids)
        G.set_data(gr.L["m"], mask)
    gr.close()


def test_cont_cast_scale_binary_argmax(be, orc):
    a = orc.normal((3, 5, 8), seed=100)  # ggml [8, 5, 3]
    b = orc.normal((8,), seed=101)
    outs = {}

    def build(g, ctx, L):
        p = g.ggml_permute(ctx, L["a"], 0, 2, 1, 3)  # [8, 3, 5]
        outs["cont"] = g.ggml_cont(ctx, p)
        outs["f16"] = g.ggml_cast(ctx, p, G.F16)
        outs["back"] = g.ggml_cast(ctx, outs["f16"], G.F32)
        outs["scale"] = g.ggml_scale_bias(ctx, L["a"], 0.5, 2.0)
        outs["add"] = g.ggml_add(ctx, L["a"], L["b"])
        outs["mul"] = g.ggml_mul(ctx, outs["add"], L["b"])
        outs["amax"] = g.ggml_argmax(ctx, g.ggml_reshape_2d(ctx, outs["mul"], 8, 15))
        outs["glu"] = g.ggml_swiglu_split(ctx, L["a"], outs["scale"])
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    gr = Graph(be, {"a": (G.F32, [8, 5, 3], a), "b": (G.F32, [8], b)}, build)
    gr.run()
    got = {k: G.get_data(t, NP[G.T(t).type]) for k, t in outs.items()}
    gr.close()
    pa = a.transpose(1, 0, 2)
    assert np.array_equal(got["cont"], pa.reshape(-1))
    assert np.array_equal(got["f16"], orc.fp32_to_fp16(pa).reshape(-1))
    assert np.array_equal(got["back"], orc.fp16_to_fp32(orc.fp32_to_fp16(pa)).reshape(-1))
    assert np.allclose(got["scale"], (a * 0.5 + 2.0).reshape(-1), rtol=0, atol=1e-6)
    s = a + b
    assert np.array_equal(got["add"], s.reshape(-1))
    assert np.array_equal(got["mul"], (s * b).reshape(-1))
    assert np.array_equal(got["amax"], np.argmax((s * b).reshape(15, 8), axis=1).astype(np.int32))
    assert orc.parity(got["glu"], orc.swiglu(a, a * 0.5 + 2.0).reshape(-1)) < 1e-6


def _argmax_rows(x):
    """ggml-cpu's forward_argmax per row: the first index of the maximum, NaN never winning, 0 for
    a row with no value above -inf."""
    v = np.where(np.isnan(x), -np.inf, x)
    return np.where(np.isneginf(v).all(axis=1), 0, np.argmax(v, axis=1)).astype(np.int32)


@pytest.mark.parametrize("rows,n", [(1, 128256), (3, 8192), (2, 50001), (65, 8192), (4, 1000)])
def test_argmax_long_rows(be, rows, n):
    """Up to 64 rows of 8192 values or more take the sliced argmax (each workgroup a 2048-value
    slice, the last of a row's to finish picks among their results); others the one-workgroup
    kernel. Ties at the maximum (lower index wins, across slices), NaN, a row of -inf; the graph
    replayed three times (the sliced kernel's row counters must be left at zero)."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[0, sorted({n // 3, n - 1, min(2049, n - 2)})] = 50.0  # ties (in different slices for long rows)
    x[0, 5] = np.nan
    x[-1, :] = -np.inf
    x[-1, 3] = np.nan
    if rows > 2:
        x[1, ::7] = np.nan
        x[1, 2047:2049] = 60.0  # a tie across a slice boundary
    want = _argmax_rows(x)

    def build(g, ctx, L):
        return g.ggml_argmax(ctx, L["x"])

    gr = Graph(be, {"x": (G.F32, [n, rows], x)}, build)
    for _ in range(3):
        got = gr.run()
        assert np.array_equal(got, want), (got[:8], want[:8])
    gr.close()


@pytest.mark.parametrize("kind", ["mul_mat", "argmax"])
def test_result_copied_into_its_own_tensor(be, orc, kind):
    """cpy(result, y) into a tensor y that no other node reads or writes (a program stage's result
    reaching its value): the producing launch writes y itself and the copy is dropped. y equals the
    graph where the result is also kept as an output (so it is written and copied) bit for bit,
    and the oracle."""
    N, K = 2048, 4096
    w = _weight(orc, "q4_0", N, K, 160)
    x = orc.normal((1, K), seed=161)
    res = {}

    def build(g, ctx, L):
        m = g.ggml_mul_mat(ctx, L["w"], L["x"])
        res["m"] = g.ggml_argmax(ctx, m) if kind == "argmax" else m
        return g.ggml_cpy(ctx, res["m"], L["y"])

    ytype = G.I32 if kind == "argmax" else G.F32
    leaves = {"w": (orc.TYPES["q4_0"], [K, N], w), "x": (G.F32, [K, 1], x),
              "y": (ytype, [1] if kind == "argmax" else [N, 1], None)}
    got = {}
    for name, outs in (("folded", ()), ("copied", [lambda s: res["m"]])):
        gr = Graph(be, leaves, build, outputs=outs)
        gr.run()
        gr.run()
        got[name] = G.get_data(gr.L["y"], NP[G.T(gr.L["y"]).type])
        gr.close()
    assert np.array_equal(got["folded"], got["copied"])
    ref = orc.mul_mat(w, "q4_0", x, K).reshape(-1)
    if kind == "argmax":  # the oracle's value at the chosen index is its maximum, to the tolerance
        assert abs(ref[got["folded"][0]] - ref.max()) <= TOL * np.abs(ref).max()
    else:
        assert orc.parity(got["folded"], ref) < TOL


UNARY_REF = {  # torch's fp32 functions on the CPU (softplus: ggml's threshold of 20)
    "relu": torch.relu, "gelu": lambda x: torch.nn.functional.gelu(x, approximate="tanh"),
    "gelu_erf": torch.nn.functional.gelu, "silu": torch.nn.functional.silu, "tanh": torch.tanh,
    "sigmoid": torch.sigmoid, "exp": torch.exp, "log": torch.log, "neg": torch.neg, "abs": torch.abs,
    "sqr": torch.square, "sqrt": torch.sqrt, "sin": torch.sin, "cos": torch.cos,
    "softplus": lambda x: torch.nn.functional.softplus(x, threshold=20.0)}


def test_unary_sub_div(be, orc):
    """Each elementwise function against torch's, on values that cover both signs (log and sqrt
    on |x| + 0.1); sub and div with a broadcast row, bit-exact."""
    a = orc.normal((3, 7, 40), seed=110) * 3.0
    pos = np.abs(a) + 0.1
    b = orc.normal((40,), seed=111) + 2.0
    outs = {}

    def build(g, ctx, L):
        for name in UNARY_REF:
            src = L["p"] if name in ("log", "sqrt") else L["a"]
            outs[name] = getattr(g, "ggml_" + name)(ctx, src)
        outs["sub"] = g.ggml_sub(ctx, L["a"], L["b"])
        outs["div"] = g.ggml_div(ctx, L["a"], L["b"])
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    gr = Graph(be, {"a": (G.F32, [40, 7, 3], a), "p": (G.F32, [40, 7, 3], pos), "b": (G.F32, [40], b)}, build)
    gr.run()
    got = {k: G.get_data(t, np.float32) for k, t in outs.items()}
    gr.close()
    for name, f in UNARY_REF.items():
        x = torch.from_numpy(pos if name in ("log", "sqrt") else a)
        want = f(x).numpy().reshape(-1)
        assert np.allclose(got[name], want, rtol=2e-6, atol=2e-6), name
    assert np.array_equal(got["sub"], (a - b).reshape(-1))
    assert np.array_equal(got["div"], (a / b).reshape(-1))


@pytest.mark.parametrize("n", [1, 96, 5000])
def test_norm_clamp_row_sums(be, orc, n):
    """norm (layer norm without affine) against torch's layer_norm, clamp against torch's, sum_rows
    and mean against float64 sums, over rows [n, 3, 2]."""
    a = orc.normal((2, 3, n), seed=130 + n) * 2.0 + 0.5
    outs = {}

    def build(g, ctx, L):
        outs["norm"] = g.ggml_norm(ctx, L["a"], 1e-5)
        outs["clamp"] = g.ggml_clamp(ctx, L["a"], -1.0, 0.75)
        outs["sum"] = g.ggml_sum_rows(ctx, L["a"])
        outs["mean"] = g.ggml_mean(ctx, L["a"])
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    gr = Graph(be, {"a": (G.F32, [n, 3, 2], a)}, build)
    gr.run()
    got = {k: G.get_data(t, np.float32) for k, t in outs.items()}
    gr.close()
    x = torch.from_numpy(a)
    want = torch.nn.functional.layer_norm(x, (n,), eps=1e-5).numpy().reshape(-1)
    assert np.allclose(got["norm"], want, rtol=1e-5, atol=2e-5)
    assert np.array_equal(got["clamp"], np.clip(a, -1.0, 0.75).reshape(-1))
    s64 = a.astype(np.float64).sum(-1).reshape(-1)
    assert np.allclose(got["sum"], s64, rtol=1e-6, atol=1e-5)
    # ggml's forward_mean: the row sum rounded to f32, then one f32 division by (float) n
    assert np.array_equal(got["mean"], s64.astype(np.float32) / np.float32(n))


@pytest.mark.parametrize("bshape", [[40, 1, 3], [1, 7, 3], [1, 1, 3], [1, 7, 1], [40, 7, 1], [1, 1, 1]])
def test_binary_broadcast_every_dim(be, orc, bshape):
    """add / sub / mul / div with the second operand repeated along any dims (ggml_can_repeat), as
    lowered programs emit them: x - mean over a leading dim, x * rsqrt(var + eps), rope's cos / sin
    products broadcast over heads. Bit-exact against numpy's broadcasting of the same f32 values."""
    a = orc.normal((3, 7, 40), seed=150)                  # ggml ne [40, 7, 3]
    b = orc.normal(tuple(reversed(bshape)), seed=151) + 3.0
    outs = {}

    def build(g, ctx, L):
        for name in ("add", "sub", "mul", "div"):
            outs[name] = getattr(g, "ggml_" + name)(ctx, L["a"], L["b"])
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    gr = Graph(be, {"a": (G.F32, [40, 7, 3], a), "b": (G.F32, bshape, b)}, build)
    gr.run()
    got = {k: G.get_data(t, np.float32) for k, t in outs.items()}
    gr.close()
    for name, f in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)):
        assert np.array_equal(got[name], f(a, b).reshape(-1)), name


def test_repeat_and_concat(be, orc):
    """repeat_4d tiles a [5, 2, 1] tensor to [10, 6, 3]; concat along each dim, one operand a
    permuted (strided) view; both bit-exact against numpy."""
    a = orc.normal((1, 2, 5), seed=140)
    x = orc.normal((3, 4, 6), seed=141)   # ggml [6, 4, 3]
    y = orc.normal((3, 4, 6), seed=142)
    outs = {}

    def build(g, ctx, L):
        outs["rep"] = g.ggml_repeat_4d(ctx, L["a"], 10, 6, 3, 1)
        for dim in range(3):
            outs[f"cat{dim}"] = g.ggml_concat(ctx, L["x"], L["y"], dim)
        yp = g.ggml_permute(ctx, L["y"], 1, 0, 2, 3)  # [4, 6, 3], strided
        outs["catp"] = g.ggml_concat(ctx, g.ggml_cont(ctx, g.ggml_permute(ctx, L["x"], 1, 0, 2, 3)), yp, 2)
        for t in outs.values():
            g.ggml_set_output(t)
        return list(outs.values())

    gr = Graph(be, {"a": (G.F32, [5, 2, 1], a), "x": (G.F32, [6, 4, 3], x), "y": (G.F32, [6, 4, 3], y)}, build)
    gr.run()
    got = {k: G.get_data(t, np.float32) for k, t in outs.items()}
    gr.close()
    assert np.array_equal(got["rep"], np.tile(a, (3, 3, 2)).reshape(-1))
    for dim in range(3):  # ggml dim d is numpy axis 2 - d
        assert np.array_equal(got[f"cat{dim}"], np.concatenate([x, y], axis=2 - dim).reshape(-1)), dim
    xt, yt = x.transpose(0, 2, 1), y.transpose(0, 2, 1)
    assert np.array_equal(got["catp"], np.concatenate([xt, yt], axis=0).reshape(-1))


@pytest.mark.parametrize("mask_type", [None, G.F16, G.F32])
@pytest.mark.parametrize("n", [7, 300, 4097])
def test_soft_max(be, orc, n, mask_type):
    """softmax(x * scale + mask) over rows [n, 5, 4, 2], the mask [n, 6, 2, 1] broadcast over the
    batch dims (rows 0..4 of it), against torch's; rows sum to 1."""
    x = orc.normal((2, 4, 5, n), seed=120 + n) * 4.0
    m = orc.normal((1, 2, 6, n), seed=121 + n) * 2.0
    m[..., : n // 3] = -np.inf
    mdata = orc.fp32_to_fp16(m) if mask_type == G.F16 else m
    mval = orc.fp16_to_fp32(mdata) if mask_type == G.F16 else m
    out = {}

    def build(g, ctx, L):
        out["y"] = g.ggml_soft_max_ext(ctx, L["x"], L["m"] if mask_type is not None else None, 0.7, 0.0)
        g.ggml_set_output(out["y"])
        return [out["y"]]

    leaves = {"x": (G.F32, [n, 5, 4, 2], x)}
    if mask_type is not None:
        leaves["m"] = (mask_type, [n, 6, 2, 1], mdata)
    gr = Graph(be, leaves, build)
    y = gr.run().reshape(2, 4, 5, n)
    gr.close()
    logits = torch.from_numpy(x) * 0.7
    if mask_type is not None:
        mb = np.broadcast_to(mval[:, :, :5], (1, 2, 5, n))
        logits = logits + torch.from_numpy(np.concatenate([mb, mb], axis=1).repeat(2, axis=0))
    want = torch.softmax(logits, dim=-1).numpy()
    assert np.allclose(y, want, rtol=1e-5, atol=1e-7)
    assert np.allclose(y.sum(-1), 1.0, atol=1e-5)


# -------------------------------------------------------------------- replay, allocation

def test_graph_replay_with_new_inputs(be, orc):
    """The captured HIP graph is replayed for each compute; inputs set in between are read; every
    replay equals the launches run one by one (graphs off)."""
    N, K = 512, 1024
    raw = _weight(orc, "q4_0", N, K, 110)
    nw = np.ones(K, np.float32)

    def build(g, ctx, L):
        return g.ggml_mul_mat(ctx, L["w"], g.ggml_mul(ctx, g.ggml_rms_norm(ctx, L["x"], 1e-5), L["nw"]))

    leaves = {"w": (G.Q4_0, [K, N], raw), "x": (G.F32, [K, 1], None), "nw": (G.F32, [K], nw)}
    results = {}
    for use in (True, False):
        gr = Graph(be, leaves, build, use_graphs=use)
        outs = []
        for seed in (111, 112, 111, 113):
            G.set_data(gr.L["x"], orc.normal((1, K), seed=seed))
            outs.append(gr.run().copy())
        gr.close()
        results[use] = outs
    for a, b in zip(results[True], results[False]):
        assert np.array_equal(a, b)
    assert np.array_equal(results[True][0], results[True][2])
    assert not np.array_equal(results[True][0], results[True][1])
    ref = orc.mul_mat(raw, "q4_0", orc.rms_norm(orc.normal((1, K), seed=113), 1e-5), K)
    assert orc.parity(results[True][3].reshape(1, N), ref) < TOL


def test_allocator_reuses_memory(be, orc):
    """A chain of 12 elementwise nodes over 1 MiB each needs a few live buffers, not 12."""
    n = 1 << 18
    x = orc.normal((n,), seed=120)

    def build(g, ctx, L):
        t = L["x"]
        for i in range(12):
            t = g.ggml_scale_bias(ctx, t, 1.0, 1.0)
        return t

    gr = Graph(be, {"x": (G.F32, [n], x)}, build)
    size = G.lib().ggml_gallocr_get_buffer_size(gr.ga, 0)
    y = gr.run()
    gr.close()
    assert size <= 3 * 4 * n
    assert np.allclose(y, x + 12.0, rtol=0, atol=1e-4)


# ------------------------------------------------------------------------ decoder graph

@pytest.mark.parametrize("wtype", [2, 8])
def test_decode_graph_matches_oracle_and_fused_model(be, orc, wtype):
    """The decode step built with ggml calls (separate q / k / v and gate / up weights, f16 cache
    written by set_rows, flash attention over cache views with an f16 mask) for 8 tokens: logits
    against the oracle's run of the same model and against the hand-fused decoder."""
    from ggml_compiler_amd.llm import LlamaConfig, Model
    from llama_ref import OracleLlama

    cfg = LlamaConfig(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000,
                      max_ctx=256, wtype=wtype, rms_eps=1e-5, rope_base=10000.0)
    m = Model(cfg, max_prompt=16)
    m.init_random(seed=11)
    w = {name: m.get_weight(name) for name, *_ in m.weights()}
    o = OracleLlama(cfg, w)
    dg = G.DecodeGraph(be, cfg, w, n_kv=256)
    tok = 17
    for p in range(8):
        lg = dg.step(tok, p)
        lo = o.forward([tok])
        lm, _ = m.decode(tok)
        assert orc.parity(lg, lo) < TOL_LM, p
        assert orc.parity(lg, lm) < TOL_LM, p
        tok = int(np.argmax(lo))
    dg.reset()
    assert orc.parity(dg.step(17, 0), OracleLlama(cfg, w).forward([17])) < TOL_LM
    dg.close()
