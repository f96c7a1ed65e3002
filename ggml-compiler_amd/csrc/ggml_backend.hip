// ggml_backend.hip - the HIP backend of the ggml API subset (include/ggml-backend.h,
// include/ggml-alloc.h): device buffers, the graph allocator, and graph execution on libgcq's
// kernels.
//
// Execution plans a graph into launch steps (one per node, or one per fusion chain), then runs the
// steps on the backend's stream. Chains (find_chains) fold the nodes the reference's decoder graph
// emits around each projection (runtime/src/ops.cpp:107-148, ggml_compiler/llm.py:361-444) into the
// launches libgcq has for them:
//   rms_norm -> mul(w)                     one rms_norm launch with the weight
//   rms_norm -> mul(w) -> mul_mat [-> add]  one decode-row GEMV normalizing x itself (one row), or
//                                          rms_norm + Q8_0 conversion, then the GEMV / GEMM
//   rms_norm -> mul -> {gate, up} mul_mats -> swiglu   one decode-row GEMV over the two weights'
//                                          row pairs, silu(gate) * up in its epilogue
//   swiglu -> mul_mat [-> add]             swiglu + Q8_0 conversion, then the GEMV / GEMM
//   mul_mat -> add                         the residual added in the GEMV / GEMM epilogue
// A chain is formed only where each intermediate has exactly one reader and is not flagged as an
// output, so no node outside the chain sees the difference. The allocator uses the same chains:
// a chain's inputs stay live until the chain's last node, where its work runs.
//
// The steps' launches are captured into a HIP graph per ggml_cgraph and replayed while the plan
// (every kernel argument) is unchanged; device inputs set with ggml_backend_tensor_set between
// computes are read by the replay.
#include "gcq_common.h"
#include "ggml_impl.h"

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <unordered_map>

namespace gcq {

void launch_pack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_unpack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_act_quant(int wtype, const float * x, int64_t ldx, int64_t B, int64_t k, void * act, hipStream_t s);
bool row_gemv_kq_fits(int type, int64_t N, int64_t K);
bool row_gemv_kq_norm_fits(int type, int64_t N, int64_t K);
void launch_row_gemv_kq(int type, const void * w, int64_t N, int64_t K, const float * x, const float * norm_w, float eps,
                        float * y, const float * res, hipStream_t s);
void launch_gemv(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t B, float * y, int64_t ldy,
                 hipStream_t s, const float * res);
void launch_gemm(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                 hipStream_t s, const float * res);
void launch_gemm_kq(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                    hipStream_t s, const float * res);
size_t attn_workspace(int Sq, int H, int Hkv, int Dv, int n_kv);
void launch_flash_attn(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                       const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, float * out, int D,
                       int Dv, int Sq, int H, int Hkv, int n_kv, float scale, void * ws, size_t ws_size, hipStream_t s);
void launch_rms_norm(const float * x, int64_t ldx, float * y, int64_t ldy, const float * w, int64_t rows, int64_t n,
                     float eps, hipStream_t s);
void launch_rmsnorm_q8(const float * x, int64_t ldx, const float * w, float eps, int64_t rows, int64_t n, void * act,
                       hipStream_t s);
void launch_swiglu_q8(const float * g, const float * u, int64_t ld, int64_t n, int64_t rows, void * act,
                      hipStream_t s);
void launch_get_rows(int type, const void * tab, int64_t nrows_tab, int64_t D, const int32_t * idx, int64_t n,
                     float * out, hipStream_t s);
void launch_swiglu(const float * g, const float * u, float * y, int64_t n, hipStream_t s);
void launch_binary(int op, const float * a, const float * b, float * y, int64_t n, int64_t nb, hipStream_t s);
void launch_mul_mat_f(bool a_f16, const void * a, const int64_t * ane, const int64_t * anb_el, const float * b,
                      const int64_t * bne, const int64_t * bnb_el, float * out, hipStream_t s);
void launch_binary_bcast(int op, const float * a, const float * b, float * y, const int64_t * ane, const int64_t * bne,
                         hipStream_t s);
void launch_argmax(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, hipStream_t s);
size_t argmax_split_scratch();
bool argmax_split_fits(int64_t rows, int64_t n);
void launch_argmax_split(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, void * scratch,
                         hipStream_t s);
int decode_group(int GT, int max_kv);
int decode_splits(int D, int H, int G, int n_kv, int max_split, bool wide);
bool attn_decode_fits(int D, int G);
void launch_attn_decode(const float * q, int64_t q_h, const void * k, int64_t k_h, int64_t k_j, const void * v,
                        int64_t v_h, int64_t v_j, int D, int H, int Hkv, int n_kv, const int * n_kv_dev, float scale,
                        int nsplit, int chunk, int kv_rows, int GS, float * out, float * part_o, float2 * part_ml,
                        hipStream_t s, const Prefetch * pf, const void * mask, int nw_lanes);

namespace {

// ------------------------------------------------------------------------ tensor predicates

std::string tname(const ggml_tensor * t) {
    std::string s = std::string(ggml_op_name(t->op));
    if (t->name[0]) s += " '" + std::string(t->name) + "'";
    s += " [";
    for (int i = 0; i < 4; i++) s += std::to_string(t->ne[i]) + (i < 3 ? ", " : "]");
    return s;
}

bool is_output(const ggml_tensor * t) { return (t->flags & GGML_TENSOR_FLAG_OUTPUT) != 0; }

// Rows of ne[0] elements at one byte stride (dims 1..3 collapse into rows), elements packed.
bool uniform_rows(const ggml_tensor * t, int64_t & rows, size_t & stride) {
    if (t->nb[0] != ggml_tsize(t->type) || ggml_blck(t->type) != 1) return false;
    rows = ggml_nrows(t);
    stride = t->nb[0] * (size_t) t->ne[0];
    bool first = true;
    size_t expect = 0;
    for (int k = 1; k < 4; k++) {
        if (t->ne[k] == 1) continue;
        if (first) {
            stride = t->nb[k];
            first = false;
        } else if (t->nb[k] != expect) {
            return false;
        }
        expect = t->nb[k] * (size_t) t->ne[k];
    }
    return stride >= t->nb[0] * (size_t) t->ne[0];
}

// The tensor starts 16-byte aligned in its buffer (buffers are 256-byte aligned).
bool aligned16(const ggml_tensor * t) { return t->view_offs % 16 == 0; }

// f32 rows usable as a GEMV / GEMM activation: uniform, 16-byte aligned rows.
bool act_rows(const ggml_tensor * t, int64_t & rows, int64_t & ld) {
    size_t stride;
    if (t->type != GGML_TYPE_F32 || !uniform_rows(t, rows, stride) || !aligned16(t) || stride % 16) return false;
    ld = (int64_t) (stride / 4);
    return true;
}

// A packed weight used whole: the tensor owning the memory (or a full reshape / view of it at
// offset 0 with the same row length).
bool whole_packed(const ggml_tensor * a) {
    if (!is_packed_type(a->type)) return false;
    const ggml_tensor * b = base_of(a);
    return a->view_offs == 0 && b->type == a->type && b->ne[0] == a->ne[0] && ggml_nelements(b) == ggml_nelements(a) &&
           ggml_is_contiguous(a) && ggml_is_contiguous(b);
}

static_assert((int) UN_ABS == (int) GGML_UNARY_OP_ABS &&
                  (int) UN_NEG == (int) GGML_UNARY_OP_NEG &&
                  (int) UN_TANH == (int) GGML_UNARY_OP_TANH &&
                  (int) UN_RELU == (int) GGML_UNARY_OP_RELU &&
                  (int) UN_SIGMOID == (int) GGML_UNARY_OP_SIGMOID &&
                  (int) UN_GELU == (int) GGML_UNARY_OP_GELU &&
                  (int) UN_SILU == (int) GGML_UNARY_OP_SILU &&
                  (int) UN_EXP == (int) GGML_UNARY_OP_EXP &&
                  (int) UN_GELU_ERF == (int) GGML_UNARY_OP_GELU_ERF &&
                  (int) UN_SOFTPLUS == (int) GGML_UNARY_OP_SOFTPLUS &&
                  (int) UN_SQR == (int) GGML_UNARY_OP_SQR &&
                  (int) UN_SQRT == (int) GGML_UNARY_OP_SQRT &&
                  (int) UN_LOG == (int) GGML_UNARY_OP_LOG &&
                  (int) UN_SIN == (int) GGML_UNARY_OP_SIN &&
                  (int) UN_COS == (int) GGML_UNARY_OP_COS &&
                  (int) UN_CLAMP == (int) GGML_UNARY_OP_CLAMP,
              "k_unary's numbering is ggml_unary_op's");

bool f32_contig(const ggml_tensor * t) { return t->type == GGML_TYPE_F32 && ggml_is_contiguous(t); }

// b repeats over a as y[i] = a[i] op b[i % nelements(b)]: b's shape is a prefix of a's.
bool prefix_broadcast(const ggml_tensor * b, const ggml_tensor * a) {
    int j = 0;
    while (j < 4 && b->ne[j] == a->ne[j]) j++;
    for (int k = j; k < 4; k++)
        if (b->ne[k] != 1) return false;
    return true;
}

// mul_mat whose weight is a whole packed Q4_0 / Q8_0 (fused activation conversions make Q8_0 codes).
bool q8_mul_mat(const ggml_tensor * mm) {
    const ggml_tensor * a = mm->src[0];
    return (a->type == GGML_TYPE_Q4_0 || a->type == GGML_TYPE_Q8_0) && whole_packed(a) && a->ne[2] == 1 &&
           a->ne[3] == 1;
}

// A mul_mat of one row by a Q4_K / Q5_K / Q6_K weight that the K-quant row GEMV runs with the
// rms_norm prologue.
bool kq_norm_mul_mat(const ggml_tensor * mm) {
    const ggml_tensor * a = mm->src[0];
    return is_kquant(a->type) && whole_packed(a) && a->ne[2] == 1 &&
           a->ne[3] == 1 && ggml_nrows(mm->src[1]) == 1 && row_gemv_kq_norm_fits(a->type, a->ne[1], a->ne[0]);
}

// Up to 3 weights of one type and row length that one decode-row launch reads (Q4_0 / Q8_0 by
// the row GEMV's ranges, Q4_K / Q5_K by the K-quant row GEMV's): spans under 2 GB.
bool weights_fit_one_launch(int type, int n, const uint8_t * const * w, const int64_t * N, int64_t K) {
    if (is_kquant(type)) {
        RowKqArgs a{};
        return row_gemv_kq_ranges(type, n, w, N, K, a);
    }
    RowArgs a{};
    return row_gemv_ranges(type, n, w, N, K, a);
}

// A mul_mat of one row by a Q4_K / Q5_K / Q6_K weight of rows up to 4096 values that the K-quant
// row GEMV runs with the attention-merge prologue.
bool kq_merge_mul_mat(const ggml_tensor * mm) {
    const ggml_tensor * a = mm->src[0];
    return is_kquant(a->type) && whole_packed(a) && a->ne[2] == 1 &&
           a->ne[3] == 1 && ggml_nrows(mm->src[1]) == 1 && a->ne[0] <= 4096 && row_gemv_kq_fits(a->type, a->ne[1], a->ne[0]);
}

// flash_attn_ext of one query row that the one-pass decode kernel runs (f16 K/V with 16-byte rows,
// f16 mask or none, no ALiBi / softcap) and whose output the decode-row GEMV can merge from
// split partials (H * D <= 4096).
bool decode_attn_node(const ggml_tensor * t) {
    if (t->op != GGML_OP_FLASH_ATTN_EXT) return false;
    const ggml_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2], *m = t->src[3];
    float fp[3];
    std::memcpy(fp, &t->op_params[0], sizeof(fp));
    const int64_t D = q->ne[0], H = q->ne[2], Hkv = k->ne[2];
    return fp[1] == 0.0f && fp[2] == 0.0f && q->type == GGML_TYPE_F32 && q->nb[0] == 4 && q->nb[1] % 4 == 0 &&
           q->nb[2] % 4 == 0 && q->ne[1] == 1 && q->ne[3] == 1 && aligned16(q) && (q->nb[2] / 4) % 4 == 0 &&
           k->type == GGML_TYPE_F16 && v->type == GGML_TYPE_F16 &&
           k->nb[0] == 2 && v->nb[0] == 2 && k->nb[1] % 16 == 0 && k->nb[2] % 16 == 0 && v->nb[1] % 16 == 0 &&
           v->nb[2] % 16 == 0 && aligned16(k) && aligned16(v) && v->ne[0] == D && H % Hkv == 0 &&
           attn_decode_fits((int) D, (int) (H / Hkv)) && H * D <= 4096 &&
           (!m || (m->type == GGML_TYPE_F16 && m->nb[0] == 2));
}

bool add_takes(const ggml_tensor * add, const ggml_tensor * mm) {
    if (add->op != GGML_OP_ADD || add->type != GGML_TYPE_F32) return false;
    const ggml_tensor * r = add->src[0] == mm ? add->src[1] : add->src[1] == mm ? add->src[0] : nullptr;
    return r && r != mm && f32_contig(r) && ggml_are_same_shape(r, mm) && aligned16(r);
}

}  // namespace

// --------------------------------------------------------------------------------- chains

// The decode step's attention inputs built the reference's way from three GEMVs of one row
// (llm.py:361-444): q -> reshape [D, H, 1] -> rope; k -> reshape -> rope (same positions and
// parameters) -> permute [D, 1, Hkv] -> set_rows into an f16 cache [D, ctx, Hkv]; v -> reshape ->
// permute -> set_rows (same positions) into another. Each intermediate read by the next node only,
// one position, NEOX over all D, no frequency factors, and nothing between the first GEMV and the
// last set_rows reading either cache. Returns {mm_q, mm_k, mm_v, rope_q, members...} or {}.
std::vector<int> qkv_rope_group(const ggml_cgraph * g, const std::vector<int> & mms,
                                const std::unordered_map<const ggml_tensor *, int> & uses,
                                const std::unordered_map<const ggml_tensor *, int> & reader) {
    const int n = (int) g->nodes.size();
    auto next = [&](const ggml_tensor * t) -> int {  // the node reading t, if t has exactly one
        if (is_output(t) || t == g->nodes[n - 1]) return -1;
        auto u = uses.find(t);
        if (u == uses.end() || u->second != 1) return -1;
        return reader.at(t);
    };
    auto is = [&](int i, ggml_op op) { return i >= 0 && g->nodes[i]->op == op; };
    int q = -1, k = -1, v = -1, rq = -1, rk = -1;
    std::vector<int> mem;
    const ggml_tensor *pos = nullptr, *ck = nullptr, *cv = nullptr;
    for (int m : mms) {
        const ggml_tensor * mm = g->nodes[m];
        const int rs = next(mm);
        if (!is(rs, GGML_OP_RESHAPE)) return {};
        const int nx = next(g->nodes[rs]);
        if (is(nx, GGML_OP_ROPE)) {
            const int pm = next(g->nodes[nx]);
            const int sr = is(pm, GGML_OP_PERMUTE) ? next(g->nodes[pm]) : -1;
            if (is(sr, GGML_OP_SET_ROWS) && g->nodes[sr]->src[0] == g->nodes[pm]) {
                if (k >= 0) return {};
                k = m;
                rk = nx;
                ck = base_of(g->nodes[sr]->src[2]);
                mem.insert(mem.end(), {rs, nx, pm, sr});
            } else {
                if (q >= 0) return {};
                q = m;
                rq = nx;
                mem.push_back(rs);
            }
        } else if (is(nx, GGML_OP_PERMUTE)) {
            const int sr = next(g->nodes[nx]);
            if (!is(sr, GGML_OP_SET_ROWS) || g->nodes[sr]->src[0] != g->nodes[nx] || v >= 0) return {};
            v = m;
            cv = base_of(g->nodes[sr]->src[2]);
            pos = g->nodes[sr]->src[1];
            mem.insert(mem.end(), {rs, nx, sr});
        } else {
            return {};
        }
    }
    if (q < 0 || k < 0 || v < 0) return {};
    const ggml_tensor *ropq = g->nodes[rq], *ropk = g->nodes[rk];
    const ggml_tensor * xq = ropq->src[0];
    const int64_t D = xq->ne[0], H = xq->ne[1], Hkv = ropk->src[0]->ne[1];
    float fp[6];
    std::memcpy(fp, &ropq->op_params[5], sizeof(fp));
    const bool ok =
        ropq->src[1] == pos && ropk->src[1] == pos && !ropq->src[2] && !ropk->src[2] &&
        std::memcmp(ropq->op_params, ropk->op_params, sizeof(ropq->op_params)) == 0 &&
        ropq->op_params[1] == D && ropq->op_params[2] == GGML_ROPE_TYPE_NEOX && fp[2] == 0.0f && D % 2 == 0 &&
        D <= 256 && xq->ne[2] == 1 && xq->ne[3] == 1 && ropk->src[0]->ne[0] == D && ropk->src[0]->ne[2] == 1 &&
        pos->type == GGML_TYPE_I32 && ggml_nelements(pos) == 1 && ropq->type == GGML_TYPE_F32 &&
        ggml_is_contiguous(ropq) && ck != cv && ck->type == GGML_TYPE_F16 && cv->type == GGML_TYPE_F16 &&
        ggml_is_contiguous(ck) && ggml_is_contiguous(cv) && ck->ne[0] == D && cv->ne[0] == D &&
        ck->ne[2] == Hkv && cv->ne[2] == Hkv && ck->ne[1] == cv->ne[1] && ck->ne[3] == 1 && cv->ne[3] == 1 &&
        g->nodes[q]->ne[0] == H * D && g->nodes[k]->ne[0] == Hkv * D && g->nodes[v]->ne[0] == Hkv * D;
    if (!ok) return {};
    std::vector<int> grp = {q, k, v, rq};
    grp.insert(grp.end(), mem.begin(), mem.end());
    const int lo = *std::min_element(grp.begin(), grp.end()), hi = *std::max_element(grp.begin(), grp.end());
    for (int i = lo + 1; i < hi; i++) {  // the caches are written at lo: nothing else may read them before hi
        if (std::find(grp.begin(), grp.end(), i) != grp.end()) continue;
        const ggml_op op = g->nodes[i]->op;  // views read nothing (their readers are checked in turn)
        if (op == GGML_OP_VIEW || op == GGML_OP_RESHAPE || op == GGML_OP_PERMUTE || op == GGML_OP_TRANSPOSE) continue;
        for (const ggml_tensor * src : g->nodes[i]->src)
            if (src && (base_of(src) == ck || base_of(src) == cv)) return {};
    }
    return grp;
}

// The gate and up GEMVs of one folded row whose results only a swiglu reads (ggml_swiglu_split of
// the two, llm.py's FFN): one launch writing silu(gate) * up, the row pairs (gate row j, up row j)
// read from the two weights (kind 4: {mm_gate, mm_up, glu}; only the glu's result has memory of
// its own). Same weight type and shape, one row. Returns the group or {}.
std::vector<int> gate_up_group(const ggml_cgraph * g, const std::vector<int> & mms,
                               const std::unordered_map<const ggml_tensor *, int> & uses,
                               const std::unordered_map<const ggml_tensor *, int> & reader) {
    if (mms.size() != 2) return {};
    const int n = (int) g->nodes.size();
    auto next = [&](const ggml_tensor * t) -> int {
        if (is_output(t) || t == g->nodes[n - 1]) return -1;
        auto u = uses.find(t);
        if (u == uses.end() || u->second != 1) return -1;
        return reader.at(t);
    };
    const ggml_tensor *a = g->nodes[mms[0]], *b = g->nodes[mms[1]];
    const int r = next(a);
    if (r < 0 || next(b) != r) return {};
    const ggml_tensor * glu = g->nodes[r];
    if (glu->op != GGML_OP_GLU || glu->op_params[0] != GGML_GLU_OP_SWIGLU || glu->op_params[1] != 0) return {};
    const ggml_tensor *gate = glu->src[0], *up = glu->src[1];
    if (!((gate == a && up == b) || (gate == b && up == a))) return {};
    const ggml_tensor *wg = gate->src[0], *wu = up->src[0];
    if (wg->type != wu->type || wg->ne[0] != wu->ne[0] || wg->ne[1] != wu->ne[1] || glu->type != GGML_TYPE_F32 ||
        !ggml_is_contiguous(glu) || ggml_nrows(glu) != 1 || glu->ne[0] != wg->ne[1] || glu->view_src)
        return {};
    return {gate == a ? mms[0] : mms[1], gate == a ? mms[1] : mms[0], r};
}

Chains find_chains(const ggml_cgraph * g, bool fuse) {
    const int n = (int) g->nodes.size();
    Chains c;
    c.end.resize(n);
    c.member.assign(n, false);
    c.in_fold.assign(n, false);
    for (int i = 0; i < n; i++) c.end[i] = i;
    c.sib.assign(n, -1);
    if (!fuse) return c;  // every node its own launch and its own memory
    std::unordered_map<const ggml_tensor *, int> uses, reader;
    std::unordered_map<const ggml_tensor *, std::vector<int>> readers;
    for (int i = 0; i < n; i++) {
        for (const ggml_tensor * s : g->nodes[i]->src) {
            if (!s) continue;
            uses[s]++;
            reader[s] = i;
            readers[s].push_back(i);
        }
    }
    // The one node reading t, if t may be folded into it.
    auto sole = [&](const ggml_tensor * t) -> int {
        if (is_output(t) || t == g->nodes[n - 1] || t->view_src) return -1;
        auto u = uses.find(t);
        if (u == uses.end() || u->second != 1) return -1;
        return reader[t];
    };
    auto link = [&](std::initializer_list<int> idx) {
        const int last = *(idx.end() - 1);
        for (int i : idx) {
            c.end[i] = last;
            if (i != last) c.member[i] = true;
        }
    };
    // mul_mat at k, optionally followed by the add of a residual.
    auto with_add = [&](int k) -> int {
        const int a = sole(g->nodes[k]);
        return a >= 0 && add_takes(g->nodes[a], g->nodes[k]) ? a : -1;
    };
    for (int i = 0; i < n; i++) {
        const ggml_tensor * t = g->nodes[i];
        if (c.member[i] || c.end[i] != i) continue;
        int64_t rows, ld;
        if (t->op == GGML_OP_RMS_NORM && t->type == GGML_TYPE_F32 && act_rows(t->src[0], rows, ld)) {
            const int j = sole(t);
            if (j < 0) continue;
            const ggml_tensor * m = g->nodes[j];
            const ggml_tensor * w = m->src[1];
            if (m->op != GGML_OP_MUL || m->src[0] != t || !f32_contig(w) || w->ne[0] != t->ne[0] || !ggml_is_vector(w))
                continue;
            const int k = sole(m);
            if (k >= 0 && g->nodes[k]->op == GGML_OP_MUL_MAT && g->nodes[k]->src[1] == m &&
                (q8_mul_mat(g->nodes[k]) || kq_norm_mul_mat(g->nodes[k]))) {
                const int a = with_add(k);
                if (a >= 0) link({i, j, k, a});
                else link({i, j, k});
                continue;
            }
            // One row read by several GEMVs (q / k / v, gate / up): each normalizes x itself in its
            // prologue and the normalized row is never written.
            const std::vector<int> & rd = readers[m];
            bool rows1 = ggml_nrows(m) == 1 && !is_output(m) && m != g->nodes[n - 1] && rd.size() >= 2;
            bool allq8 = true, allkq = true;
            for (int r : rd) {
                const ggml_tensor * mm = g->nodes[r];
                const bool q8 = mm->op == GGML_OP_MUL_MAT && q8_mul_mat(mm) && row_gemv_fits(mm->src[0]->type, m->ne[0]);
                const bool kq = mm->op == GGML_OP_MUL_MAT && kq_norm_mul_mat(mm);
                rows1 = rows1 && mm->op == GGML_OP_MUL_MAT && mm->src[1] == m && mm->src[0] != m && (q8 || kq);
                allq8 = allq8 && q8;
                allkq = allkq && kq;
            }
            if (!rows1) {
                link({i, j});
                continue;
            }
            c.member[i] = c.member[j] = true;
            c.in_fold[i] = c.in_fold[j] = true;
            c.folded.push_back(m);
            int last = j;
            bool adds = false, same = true;
            for (int r : rd) {
                const int a = with_add(r);
                if (a >= 0) link({r, a});
                adds = adds || a >= 0;
                same = same && g->nodes[r]->src[0]->type == g->nodes[rd[0]]->src[0]->type;
                last = std::max(last, c.end[r]);
            }
            c.end[i] = c.end[j] = last;  // x and w are read until the last reader's work runs
            // K-quant q / k / v whose v has a type of its own (Q4_K_M files): the q / k rope launch
            // and the v launch writing its cache, one group
            const bool mixed = !adds && !same && allkq && rd.size() == 3;
            if ((!adds && same && (allq8 || allkq) && rd.size() <= 3) || mixed) {  // the multi-weight launches
                std::vector<int> grp(rd.begin(), rd.end());
                std::sort(grp.begin(), grp.end());
                // the row-pair epilogues: any Q4_0 / Q8_0 row, K-quant rows of at most 4096 values
                bool pairs = allq8 || row_gemv_kq_epi_fits(g->nodes[grp[0]]->src[0]->type, EPI_ROPE_KV, m->ne[0]);
                for (int r : grp) pairs = pairs && (allq8 || row_gemv_kq_epi_fits(g->nodes[r]->src[0]->type, EPI_ROPE_KV, m->ne[0]));
                std::vector<int> qkv = grp.size() == 3 && pairs ? qkv_rope_group(g, grp, uses, reader) : std::vector<int>{};
                // mixed: q and k of one type (qkv_rope_group's order: q, k, v)
                if (mixed && (qkv.empty() || g->nodes[qkv[0]]->src[0]->type != g->nodes[qkv[1]]->src[0]->type)) continue;
                std::vector<int> gu = grp.size() == 2 && pairs ? gate_up_group(g, grp, uses, reader) : std::vector<int>{};
                const int kind = !qkv.empty() ? 3 : !gu.empty() ? 4 : 0;
                if (kind == 3) grp = qkv;
                if (kind == 4) grp = gu;
                int lo = n;
                for (int r : grp) {
                    c.sib[r] = (int) c.groups.size();
                    lo = std::min(lo, r);
                }
                c.groups.push_back(std::move(grp));
                c.kind.push_back(kind);
                c.first.push_back(lo);
            }
        } else if (t->op == GGML_OP_GLU && c.sib[i] < 0 && f32_contig(t->src[0]) && f32_contig(t->src[1]) && aligned16(t->src[0]) &&
                   aligned16(t->src[1]) && t->ne[0] % 32 == 0) {
            const int k = sole(t);
            if (k < 0 || g->nodes[k]->op != GGML_OP_MUL_MAT || g->nodes[k]->src[1] != t || !q8_mul_mat(g->nodes[k]))
                continue;
            const int a = with_add(k);
            if (a >= 0) link({i, k, a});
            else link({i, k});
        } else if (decode_attn_node(t)) {
            // attention row -> reshape to [H*D, 1] -> output projection: the GEMV merges the
            // attention's split partials in its prologue; the row is never written.
            const int j = sole(t);
            if (j < 0) continue;
            const ggml_tensor * rs = g->nodes[j];
            if (rs->op != GGML_OP_RESHAPE || rs->src[0] != t || is_output(rs) || rs == g->nodes[n - 1]) continue;
            auto u = uses.find(rs);
            if (u == uses.end() || u->second != 1) continue;
            const int k = reader[rs];
            const ggml_tensor * mm = g->nodes[k];
            if (mm->op != GGML_OP_MUL_MAT || mm->src[1] != rs || ggml_nrows(rs) != 1 ||
                !((q8_mul_mat(mm) && row_gemv_fits(mm->src[0]->type, rs->ne[0])) || kq_merge_mul_mat(mm)))
                continue;
            const int a = with_add(k);
            if (a >= 0) link({i, j, k, a});
            else link({i, j, k});
        } else if (t->op == GGML_OP_MUL_MAT && whole_packed(t->src[0])) {
            const int a = with_add(i);
            if (a >= 0) link({i, a});
        }
    }
    // Pairs of ropes / set_rows (kinds 1, 2). at(t): the node whose launch computes t's memory
    // (a chain's end, a group's first), -1 for what exists before the graph.
    std::unordered_map<const ggml_tensor *, int> prod;
    for (int i = 0; i < n; i++) prod[g->nodes[i]] = i;
    auto at = [&](const ggml_tensor * t) -> int {
        while (t->view_src) t = t->view_src;
        auto it = prod.find(t);
        if (it == prod.end()) return -1;
        int k = it->second;
        if (c.member[k]) k = c.end[k];
        if (c.sib[k] >= 0) k = c.first[(size_t) c.sib[k]];
        return k;
    };
    auto free_node = [&](int i) { return !c.member[i] && c.sib[i] < 0 && c.end[i] == i; };
    for (int i = 0; i < n; i++) {
        const ggml_tensor * a = g->nodes[i];
        if ((a->op != GGML_OP_ROPE && a->op != GGML_OP_SET_ROWS) || !free_node(i)) continue;
        for (int j = i + 1; j < n; j++) {
            const ggml_tensor * b = g->nodes[j];
            if (b->op != a->op || !free_node(j) || b->src[1] != a->src[1] || at(b->src[0]) >= i) continue;
            if (a->op == GGML_OP_ROPE) {
                if (b->src[2] != a->src[2] || std::memcmp(a->op_params, b->op_params, sizeof(a->op_params)) != 0 ||
                    a->src[0]->ne[0] != b->src[0]->ne[0] || a->src[0]->ne[2] != b->src[0]->ne[2])
                    continue;
            } else {
                const ggml_tensor * dst = base_of(b->src[2]);
                bool read = false;  // nothing between the two may read the second's destination
                for (int k = i + 1; k < j && !read; k++)
                    for (const ggml_tensor * q : g->nodes[k]->src) read = read || (q && base_of(q) == dst);
                if (read || base_of(a->src[2]) == dst) continue;
            }
            c.sib[i] = c.sib[j] = (int) c.groups.size();
            c.groups.push_back({i, j});
            c.kind.push_back(a->op == GGML_OP_ROPE ? 1 : 2);
            c.first.push_back(i);
            break;
        }
    }
    return c;
}

}  // namespace gcq

using namespace gcq;

// ------------------------------------------------------------------------------ structures

struct ggml_backend_buffer_type {
    ggml_backend * be;
};

struct ggml_backend_buffer {
    ggml_backend * be = nullptr;
    void * base = nullptr;
    size_t size = 0;
};

namespace {

enum StepKind {
    S_MULMAT,         // [rms_norm ->] mul_mat [-> add] (x rows f32)
    S_SWIGLU_MULMAT,  // swiglu -> mul_mat [-> add]
    S_RMSNORM,
    S_BINARY,
    S_SCALE,
    S_CPY,
    S_GETROWS,
    S_SETROWS,
    S_ROPE,
    S_FATTN,
    S_SWIGLU,
    S_UNARY,
    S_SOFTMAX,
    S_NORM,
    S_ROWSUM,
    S_REPEAT,
    S_ARGMAX,
    S_ATTN_MULMAT,  // decode attention (split partials) -> mul_mat merging them [-> add]
    S_MULMAT3,      // rms_norm -> mul -> 2 or 3 mul_mats of the one row: one decode-row GEMV
    S_ROPE2,        // two ropes of the same positions
    S_SETROWS2,     // two set_rows of the same indices
    S_ROPE_TABLE,   // the (cos, sin) table of one position for S_QKV_ROPE
    S_QKV_ROPE,     // q / k / v GEMVs with q / k rope and k / v cache writes in the epilogue
    S_GATE_UP,      // gate / up GEMVs of one normalized row with swiglu in the epilogue
    S_MULMAT_F,     // mul_mat of an f32 / f16 first operand (activations, KV-cache views)
    S_JOBS,         // the next n[0] steps (get_rows / cpy / rope table, independent) as one launch
};

// One launch sequence with every argument it takes; compared byte for byte to decide whether a
// captured graph can be replayed, so it is always zero-initialized.
struct Step {
    int kind, type, op, pad;
    const void * in[6];
    void * out;
    void * out2[2];  // S_MULMAT3: the second and third results; S_ROPE2 / S_SETROWS2: the second's
    int64_t m[8];    // S_ROPE2 / S_SETROWS2: the second tensor's strides and sizes
    int64_t n[12];
    float f[6];
    Cpy4 g;
};

Step new_step(int kind) {
    Step s;
    std::memset(&s, 0, sizeof(s));
    s.kind = kind;
    return s;
}

struct Cached {
    std::vector<uintptr_t> fp;  // the nodes it was planned from
    std::vector<uint8_t> sig;   // the steps it holds
    hipGraphExec_t exec = nullptr;
};

// Everything about g's nodes that planning reads: ops, types, flags, shapes, strides, parameters,
// sources and every data address. Equal fingerprints plan to equal steps.
std::vector<uintptr_t> fingerprint(const ggml_cgraph * g) {
    std::vector<uintptr_t> f;
    f.reserve(g->nodes.size() * 40);
    for (const ggml_tensor * t : g->nodes) {
        f.push_back((uintptr_t) t);
        f.push_back(((uintptr_t) t->op << 32) | ((uintptr_t) t->type << 16) | (uintptr_t) (t->flags & 0xffff));
        f.push_back((uintptr_t) t->data);
        f.push_back((uintptr_t) t->view_offs);
        for (int i = 0; i < 4; i++) {
            f.push_back((uintptr_t) t->ne[i]);
            f.push_back((uintptr_t) t->nb[i]);
        }
        for (int i = 0; i < GGML_MAX_OP_PARAMS / 4; i += 2)
            f.push_back(((uintptr_t) (uint32_t) t->op_params[i] << 32) | (uint32_t) t->op_params[i + 1]);
        for (const ggml_tensor * s : t->src) {
            f.push_back((uintptr_t) s);
            if (s) f.push_back((uintptr_t) s->data);
        }
    }
    return f;
}

}  // namespace

struct ggml_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    ggml_backend_buffer_type buft{};
    std::string name;
    void * ws = nullptr;  // workspace of the mul_mat activations and flash-attention partials
    size_t ws_size = 0;
    uint64_t epoch = 0;  // bumped whenever the workspace moves (graphs captured before point at the old one)
    float2 * rope_cs = nullptr;  // (cos, sin) table of the fused q / k / v rope step (<= 128 pairs)
    void * argmax_scratch = nullptr;  // the sliced argmax's row counters (left zero) and partials
    bool use_graphs = true;
    bool fuse = true;  // fusion chains and launch groups (off: every node alone, materialized)
    std::unordered_map<const ggml_cgraph *, Cached> graphs;
    std::vector<Step> steps;

    ~ggml_backend() {
        if (stream) (void) hipStreamSynchronize(stream);
        for (auto & kv : graphs)
            if (kv.second.exec) (void) hipGraphExecDestroy(kv.second.exec);
        if (ws) (void) hipFree(ws);
        if (rope_cs) (void) hipFree(rope_cs);
        if (argmax_scratch) (void) hipFree(argmax_scratch);
        if (stream) (void) hipStreamDestroy(stream);
    }
};

struct ggml_gallocr {
    ggml_backend * be = nullptr;
    ggml_backend_buffer buf;  // a tensor placed here has buffer == &buf
};

namespace {

// --------------------------------------------------------------------------------- helpers

size_t alloc_size(const ggml_tensor * t) {
    if (is_packed_type(t->type) && ggml_is_contiguous(t)) {
        const WeightLayout L = weight_layout(t->type, ggml_nrows(t), t->ne[0]);
        return L.total;
    }
    return ggml_nbytes(t);
}

// The packed weight t (whole, contiguous): rows and row length.
void packed_dims(const ggml_tensor * t, int64_t & rows, int64_t & k) {
    rows = ggml_nrows(t);
    k = t->ne[0];
}

void set_device(const ggml_backend * be) { check_hip(hipSetDevice(be->device), "hipSetDevice"); }

const char * data_of(const ggml_tensor * t) {
    require(t->data != nullptr, "tensor " + tname(t) + " has no memory (allocate its context or graph)");
    require(base_of(t)->buffer != nullptr, "tensor " + tname(t) + " is in host memory, not in a HIP buffer");
    return (const char *) t->data;
}
void * mut_data(const ggml_tensor * t) { return (void *) data_of(t); }

void ensure_ws(ggml_backend * be, size_t need) {
    if (need <= be->ws_size) return;
    check_hip(hipStreamSynchronize(be->stream), "workspace");
    if (be->ws) check_hip(hipFree(be->ws), "hipFree");
    be->ws = nullptr;
    be->ws_size = 0;
    const size_t n = (need + (1 << 20) - 1) & ~size_t((1 << 20) - 1);
    check_hip(hipMalloc(&be->ws, n), "hipMalloc workspace");
    be->ws_size = n;
    be->epoch++;
    for (auto & kv : be->graphs) {  // every captured graph points at the old workspace
        if (kv.second.exec) (void) hipGraphExecDestroy(kv.second.exec);
    }
    be->graphs.clear();
}

// ------------------------------------------------------------------------------- planning

struct Planner {
    ggml_backend * be;
    std::vector<Step> & steps;
    size_t ws_need = 0;
    bool dry = false;  // supports_op: shapes and types only, no data

    const char * d(const ggml_tensor * t) const { return dry ? nullptr : data_of(t); }
    void * o(const ggml_tensor * t) const { return dry ? nullptr : mut_data(t); }

    const std::vector<const ggml_tensor *> * folded = nullptr;  // mul(rms_norm(x), w) rows read by GEMVs

    void mulmat(const ggml_tensor * mm, const ggml_tensor * x, const ggml_tensor * norm_w, float eps,
                const ggml_tensor * res, const ggml_tensor * y) {
        const ggml_tensor * w = mm->src[0];
        if (folded && std::find(folded->begin(), folded->end(), x) != folded->end()) {
            const ggml_tensor * nrm = x->src[0];
            norm_w = x->src[1];
            std::memcpy(&eps, &nrm->op_params[0], 4);
            x = nrm->src[0];
        }
        require(whole_packed(w), "mul_mat " + tname(mm) + ": the weight must be a whole Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K tensor in "
                                                          "a HIP buffer (other weight types are not on this path)");
        require(w->ne[2] == 1 && w->ne[3] == 1, "mul_mat " + tname(mm) + ": batched weights are not supported");
        int64_t M = 0, ldx = 0;
        require(act_rows(x, M, ldx), "mul_mat " + tname(mm) + ": the activation must be f32 rows at one stride, "
                                                              "16-byte aligned (add a cont)");
        int64_t N, K;
        packed_dims(w, N, K);
        Step s = new_step(S_MULMAT);
        s.type = w->type;
        s.in[0] = d(w);
        s.in[1] = d(x);
        s.in[2] = norm_w ? d(norm_w) : nullptr;
        s.in[3] = res ? d(res) : nullptr;
        s.out = o(y);
        s.n[0] = N;
        s.n[1] = K;
        s.n[2] = M;
        s.n[3] = ldx;
        s.n[4] = N;  // ldy: results are contiguous
        s.f[0] = eps;
        const bool row = M == 1 && (w->type == GGML_TYPE_Q4_0 || w->type == GGML_TYPE_Q8_0) && row_gemv_fits(w->type, K);
        if (!row) ws_need = std::max(ws_need, act_layout(w->type, M, K).total);
        steps.push_back(s);
    }

    // mul_mat(a, b) with a f32 / f16 (any strides, innermost contiguous) and b f32 rows (any
    // strides, innermost contiguous): a's batch repeat-interleaved over b's (grouped-query heads).
    void mulmat_float(const ggml_tensor * mm) {
        const ggml_tensor *a = mm->src[0], *b = mm->src[1];
        const size_t ea = ggml_type_size(a->type);
        require(b->type == GGML_TYPE_F32, "mul_mat " + tname(mm) + ": an f32 / f16 first operand needs f32 rows as the second");
        require(a->nb[0] == ea && b->nb[0] == 4, "mul_mat " + tname(mm) + ": both operands need contiguous rows (add a cont)");
        for (int k = 1; k < 4; k++)
            require(a->nb[k] % ea == 0 && b->nb[k] % 4 == 0, "mul_mat " + tname(mm) + ": strides are not whole elements");
        require(a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0,
                "mul_mat " + tname(mm) + ": cannot multiply " + tname(a) + " by " + tname(b));
        require(ggml_is_contiguous(mm), "mul_mat " + tname(mm) + ": the result must be contiguous");
        Step s = new_step(S_MULMAT_F);
        s.type = a->type;
        s.in[0] = d(a);
        s.in[1] = d(b);
        s.out = o(mm);
        for (int k = 0; k < 4; k++) {
            s.m[k] = a->ne[k];
            s.n[k] = b->ne[k];
        }
        for (int k = 1; k < 4; k++) {
            s.m[3 + k] = (int64_t) (a->nb[k] / ea);
            s.n[3 + k] = (int64_t) (b->nb[k] / 4);
        }
        steps.push_back(s);
    }

    const ggml_tensor * table_pos = nullptr;  // the position and parameters of the last table step
    int32_t table_params[16] = {};

    // Group kind 3 (qkv_rope_group's order): the rotation table of the step's position (once for
    // every layer that shares it), then one decode-row launch over the three weights whose
    // epilogue ropes q into rope_q's result and writes roped k and v into the caches at pos.
    void qkv_rope(const ggml_cgraph * g, const std::vector<int> & grp) {
        const ggml_tensor *mq = g->nodes[grp[0]], *mk = g->nodes[grp[1]], *mv = g->nodes[grp[2]];
        const ggml_tensor * rq = g->nodes[grp[3]];
        const ggml_tensor * x = mq->src[1];
        const ggml_tensor * nrm = x->src[0];
        const ggml_tensor * srk = nullptr;
        const ggml_tensor * srv = nullptr;
        for (size_t q = 4; q < grp.size(); q++) {
            const ggml_tensor * t = g->nodes[grp[q]];
            if (t->op != GGML_OP_SET_ROWS) continue;
            if (t->src[0]->src[0] && t->src[0]->src[0]->op == GGML_OP_ROPE) srk = t;
            else srv = t;
        }
        require(srk && srv, "q / k / v rope group: set_rows nodes not found");
        const int type = mq->src[0]->type;
        const uint8_t * w[3] = {(const uint8_t *) d(mq->src[0]), (const uint8_t *) d(mk->src[0]),
                                (const uint8_t *) d(mv->src[0])};
        int64_t N[3], K = 0;
        packed_dims(mq->src[0], N[0], K);
        packed_dims(mk->src[0], N[1], K);
        packed_dims(mv->src[0], N[2], K);
        const ggml_tensor * pos = srv->src[1];
        const ggml_tensor * ck = base_of(srk->src[2]);
        const ggml_tensor * cv = base_of(srv->src[2]);
        if (table_pos != pos || std::memcmp(table_params, rq->op_params, sizeof(table_params)) != 0) {
            if (!be->rope_cs) check_hip(hipMalloc((void **) &be->rope_cs, 128 * sizeof(float2)), "hipMalloc rope table");
            float fp[6];
            std::memcpy(fp, &rq->op_params[5], sizeof(fp));
            Step t = new_step(S_ROPE_TABLE);
            t.in[0] = d(pos);
            t.n[0] = rq->op_params[1];
            t.f[0] = fp[0];
            t.f[1] = fp[1];
            t.f[2] = fp[3];
            steps.push_back(t);
            table_pos = pos;
            std::memcpy(table_params, rq->op_params, sizeof(table_params));
        }
        Step s = new_step(S_QKV_ROPE);
        s.type = type;
        s.in[0] = w[0];
        s.in[1] = d(nrm->src[0]);
        s.in[2] = d(x->src[1]);
        s.in[3] = w[1];
        s.in[4] = w[2];
        s.in[5] = d(pos);
        s.out = o(rq);
        s.out2[0] = o(ck);
        s.out2[1] = o(cv);
        s.n[0] = N[0];
        s.n[1] = N[1];
        s.n[2] = N[2];
        s.n[3] = K;
        s.n[4] = rq->ne[1];   // H
        s.n[5] = ck->ne[2];   // Hkv
        s.n[6] = rq->ne[0];   // D
        s.n[7] = ck->ne[1];   // ctx
        std::memcpy(&s.f[0], &nrm->op_params[0], 4);
        // v's type: another K-quant type puts the v rows in a launch of their own (EPI_V_CACHE)
        const int vtype = mv->src[0]->type;
        s.m[0] = vtype;
        require(vtype == type ? weights_fit_one_launch(type, 3, w, N, K)
                              : weights_fit_one_launch(type, 2, w, N, K) && weights_fit_one_launch(vtype, 1, w + 2, N + 2, K),
                "q / k / v rope group: the weights do not fit one launch");
        steps.push_back(s);
    }

    // Two ropes / set_rows planned as one step when each plans to one step of that kind with the
    // same positions; else their two steps, here.
    void pair(const ggml_tensor * a, const ggml_tensor * b) {
        const size_t n0 = steps.size();
        node(a);
        const size_t n1 = steps.size();
        node(b);
        if (n1 != n0 + 1 || steps.size() != n0 + 2) return;
        Step & s = steps[n0];
        const Step & t = steps[n0 + 1];
        if (s.kind == S_ROPE && t.kind == S_ROPE && s.in[1] == t.in[1] && s.in[2] == t.in[2] && s.n[4] == t.n[4] &&
            s.n[6] == t.n[6] && s.n[7] == t.n[7] && s.f[0] == t.f[0] && s.f[1] == t.f[1] && s.f[2] == t.f[2]) {
            s.kind = S_ROPE2;
            s.in[3] = t.in[0];
            s.out2[0] = t.out;
            s.m[0] = t.n[0];
            s.m[1] = t.n[1];
            s.m[2] = t.n[2];
            s.m[3] = t.n[3];
            s.m[4] = t.n[5];
            steps.pop_back();
        } else if (s.kind == S_SETROWS && t.kind == S_SETROWS && s.in[1] == t.in[1] && s.n[4] == t.n[4]) {
            s.kind = S_SETROWS2;
            s.in[3] = t.in[0];
            s.out2[0] = t.out;
            s.m[0] = t.n[0];
            s.m[1] = t.n[1];
            s.m[2] = t.n[2];
            s.m[3] = t.n[3];
            s.m[4] = t.n[5];
            s.m[5] = t.n[6];
            s.m[6] = t.n[7];
            steps.pop_back();
        }
    }

    // GEMVs of one folded row (nodes grp of g): one decode-row launch over the weights' rows when
    // they fit one (same type, spans under 2 GB), else one step each, all at this place.
    void mulmat_group(const ggml_cgraph * g, const std::vector<int> & grp) {
        const ggml_tensor * m0 = g->nodes[grp[0]];
        const ggml_tensor * x = m0->src[1];
        const ggml_tensor * nrm = x->src[0];
        const int type = m0->src[0]->type;
        const uint8_t * w[3];
        int64_t N[3], K = 0;
        bool ok = grp.size() >= 2 && grp.size() <= 3 &&
                  (type == GGML_TYPE_Q4_0 || type == GGML_TYPE_Q8_0 || is_kquant(type));
        for (size_t k = 0; ok && k < grp.size(); k++) {
            const ggml_tensor * mm = g->nodes[grp[k]];
            const ggml_tensor * wt = mm->src[0];
            ok = whole_packed(wt) && wt->type == type && wt->ne[2] == 1 && wt->ne[3] == 1 && ggml_is_contiguous(mm) &&
                 !dry;
            if (!ok) break;
            packed_dims(wt, N[k], K);
            w[k] = (const uint8_t *) d(wt);
        }
        if (ok) ok = weights_fit_one_launch(type, (int) grp.size(), w, N, K);
        if (!ok) {
            for (int r : grp) mulmat(g->nodes[r], g->nodes[r]->src[1], nullptr, 0.0f, nullptr, g->nodes[r]);
            return;
        }
        Step s = new_step(S_MULMAT3);
        s.type = type;
        s.in[0] = w[0];
        s.in[1] = d(nrm->src[0]);
        s.in[2] = d(x->src[1]);
        s.in[3] = w[1];
        s.in[4] = grp.size() > 2 ? w[2] : nullptr;
        s.out = o(m0);
        s.out2[0] = o(g->nodes[grp[1]]);
        s.out2[1] = grp.size() > 2 ? o(g->nodes[grp[2]]) : nullptr;
        s.n[0] = N[0];
        s.n[1] = N[1];
        s.n[2] = grp.size() > 2 ? N[2] : 0;
        s.n[3] = K;
        std::memcpy(&s.f[0], &nrm->op_params[0], 4);
        steps.push_back(s);
    }

    // Group kind 4: rms_norm -> mul -> {mul_mat gate, mul_mat up} -> swiglu, one decode-row launch.
    void gate_up(const ggml_cgraph * g, const std::vector<int> & grp) {
        const ggml_tensor *mg = g->nodes[grp[0]], *mu = g->nodes[grp[1]], *glu = g->nodes[grp[2]];
        const ggml_tensor * x = mg->src[1];
        const ggml_tensor * nrm = x->src[0];
        int64_t N[2], K = 0;
        packed_dims(mg->src[0], N[0], K);
        packed_dims(mu->src[0], N[1], K);
        Step s = new_step(S_GATE_UP);
        s.type = mg->src[0]->type;
        s.in[0] = d(mg->src[0]);
        s.in[1] = d(nrm->src[0]);
        s.in[2] = d(x->src[1]);
        s.in[3] = d(mu->src[0]);
        s.out = o(glu);
        s.n[0] = N[0];
        s.n[1] = N[1];
        s.n[3] = K;
        std::memcpy(&s.f[0], &nrm->op_params[0], 4);
        steps.push_back(s);
    }

    void swiglu_mulmat(const ggml_tensor * glu, const ggml_tensor * mm, const ggml_tensor * res, const ggml_tensor * y) {
        const ggml_tensor * w = mm->src[0];
        int64_t N, K;
        packed_dims(w, N, K);
        Step s = new_step(S_SWIGLU_MULMAT);
        s.type = w->type;
        s.in[0] = d(w);
        s.in[1] = d(glu->src[0]);
        s.in[2] = d(glu->src[1]);
        s.in[3] = res ? d(res) : nullptr;
        s.out = o(y);
        s.n[0] = N;
        s.n[1] = K;
        s.n[2] = ggml_nrows(glu);
        s.n[3] = glu->ne[0];
        ws_need = std::max(ws_need, act_layout(w->type, s.n[2], K).total);
        steps.push_back(s);
    }

    void rmsnorm(const ggml_tensor * nrm, const ggml_tensor * w, const ggml_tensor * y) {
        const ggml_tensor * x = nrm->src[0];
        int64_t rows = 0;
        size_t stride = 0;
        require(x->type == GGML_TYPE_F32 && uniform_rows(x, rows, stride),
                "rms_norm " + tname(nrm) + ": needs f32 rows at one stride");
        Step s = new_step(S_RMSNORM);
        s.in[0] = d(x);
        s.in[1] = w ? d(w) : nullptr;
        s.out = o(y);
        s.n[0] = (int64_t) (stride / 4);
        s.n[1] = rows;
        s.n[2] = x->ne[0];
        float eps;
        std::memcpy(&eps, &nrm->op_params[0], 4);
        s.f[0] = eps;
        steps.push_back(s);
    }

    void node(const ggml_tensor * t) {
        switch (t->op) {
            case GGML_OP_NONE:
            case GGML_OP_VIEW:
            case GGML_OP_RESHAPE:
            case GGML_OP_PERMUTE:
            case GGML_OP_TRANSPOSE:
                return;
            case GGML_OP_MUL_MAT:
                require(t->src[1]->ne[2] % std::max<int64_t>(1, t->src[0]->ne[2]) == 0, "mul_mat: batch mismatch");
                if (t->src[0]->type == GGML_TYPE_F32 || t->src[0]->type == GGML_TYPE_F16) return mulmat_float(t);
                return mulmat(t, t->src[1], nullptr, 0.0f, nullptr, t);
            case GGML_OP_RMS_NORM:
                return rmsnorm(t, nullptr, t);
            case GGML_OP_ADD:
            case GGML_OP_SUB:
            case GGML_OP_DIV:
            case GGML_OP_MUL: {
                const ggml_tensor *a = t->src[0], *b = t->src[1];
                require(f32_contig(a) && f32_contig(b) && ggml_can_repeat(b, a),
                        std::string(ggml_op_name(t->op)) + " " + tname(t) +
                            ": needs contiguous f32 operands, the second repeating over the first");
                Step s = new_step(S_BINARY);
                s.op = t->op == GGML_OP_ADD ? 0 : t->op == GGML_OP_MUL ? 1 : t->op == GGML_OP_SUB ? 2 : 3;
                s.in[0] = d(a);
                s.in[1] = d(b);
                s.out = o(t);
                s.n[0] = ggml_nelements(a);
                s.n[1] = ggml_nelements(b);
                s.n[2] = prefix_broadcast(b, a) ? 0 : 1;  // 1: per-dim broadcast
                for (int k = 0; k < 4; k++) {
                    s.m[k] = a->ne[k];
                    s.m[4 + k] = b->ne[k];
                }
                steps.push_back(s);
                return;
            }
            case GGML_OP_SCALE: {
                require(f32_contig(t->src[0]), "scale " + tname(t) + ": needs a contiguous f32 input");
                Step s = new_step(S_SCALE);
                s.in[0] = d(t->src[0]);
                s.out = o(t);
                s.n[0] = ggml_nelements(t);
                std::memcpy(&s.f[0], &t->op_params[0], 4);
                std::memcpy(&s.f[1], &t->op_params[1], 4);
                steps.push_back(s);
                return;
            }
            case GGML_OP_CPY:
            case GGML_OP_CONT: {
                const ggml_tensor * a = t->src[0];
                auto ok = [](const ggml_tensor * x) {
                    return (x->type == GGML_TYPE_F32 || x->type == GGML_TYPE_F16) && x->nb[0] % ggml_tsize(x->type) == 0;
                };
                const bool ints = a->type == GGML_TYPE_I32 && t->type == GGML_TYPE_I32 && a->nb[0] % 4 == 0 &&
                                  t->nb[0] % 4 == 0;
                require(ints || (ok(a) && ok(t)), "cpy " + tname(t) + ": f32 / f16, or i32 to i32");
                Step s = new_step(S_CPY);
                s.type = a->type;
                s.op = t->type;
                s.in[0] = d(a);
                s.out = o(t);
                for (int k = 0; k < 4; k++) {
                    s.g.sne[k] = a->ne[k];
                    s.g.snb[k] = (int64_t) a->nb[k];
                    s.g.dne[k] = t->ne[k];
                    s.g.dnb[k] = (int64_t) t->nb[k];
                }
                s.n[0] = ggml_nelements(t);
                steps.push_back(s);
                return;
            }
            case GGML_OP_GET_ROWS: {
                const ggml_tensor *a = t->src[0], *b = t->src[1];
                const bool table = ((a->type == GGML_TYPE_F32 || a->type == GGML_TYPE_F16) && ggml_is_contiguous(a)) ||
                                   ((a->type == GGML_TYPE_Q4_0 || a->type == GGML_TYPE_Q8_0 || a->type == GGML_TYPE_Q4_K ||
                                     a->type == GGML_TYPE_Q5_K || a->type == GGML_TYPE_Q6_K) &&
                                    whole_packed(a));
                require(table && a->ne[2] == 1 && a->ne[3] == 1,
                        "get_rows " + tname(t) + ": the table must be a contiguous F32 / F16 matrix or a whole Q4_0 / "
                                                 "Q8_0 / Q4_K / Q5_K / Q6_K tensor");
                require(ggml_is_contiguous(b) && ggml_is_vector(b), "get_rows " + tname(t) + ": one i32 index vector");
                Step s = new_step(S_GETROWS);
                s.type = a->type;
                s.in[0] = d(a);
                s.in[1] = d(b);
                s.out = o(t);
                s.n[0] = a->ne[1];
                s.n[1] = a->ne[0];
                s.n[2] = b->ne[0];
                steps.push_back(s);
                return;
            }
            case GGML_OP_SET_ROWS: {
                const ggml_tensor *b = t->src[0], *c = t->src[1], *a = t->src[2];
                require(a->type == GGML_TYPE_F16 && a->nb[0] == 2 && a->ne[0] % 8 == 0 && a->nb[1] % 16 == 0 &&
                            a->nb[2] % 16 == 0 && a->ne[3] == 1 && aligned16(a),
                        "set_rows " + tname(t) + ": the destination must be an f16 cache with 16-byte rows");
                require(b->type == GGML_TYPE_F32 && b->nb[0] == 4 && b->nb[1] % 4 == 0 && b->nb[2] % 4 == 0,
                        "set_rows " + tname(t) + ": the rows must be f32");
                require(c->type == GGML_TYPE_I32 && ggml_is_contiguous(c) && ggml_is_vector(c),
                        "set_rows " + tname(t) + ": one i32 index vector");
                Step s = new_step(S_SETROWS);
                s.out = o(a);
                s.in[0] = d(b);
                s.in[1] = d(c);
                s.n[0] = (int64_t) a->nb[2] / 2;
                s.n[1] = (int64_t) a->nb[1] / 2;
                s.n[2] = (int64_t) b->nb[2] / 4;
                s.n[3] = (int64_t) b->nb[1] / 4;
                s.n[4] = b->ne[1];
                s.n[5] = b->ne[0];
                s.n[6] = b->ne[2];
                s.n[7] = a->ne[1];
                steps.push_back(s);
                return;
            }
            case GGML_OP_ROPE: {
                const ggml_tensor *x = t->src[0], *pos = t->src[1], *ff = t->src[2];
                float fp[6];
                std::memcpy(fp, &t->op_params[5], sizeof(fp));
                const int n_dims = t->op_params[1], mode = t->op_params[2];
                require(mode == GGML_ROPE_TYPE_NEOX, "rope " + tname(t) + ": NEOX mode (2) only");
                require(fp[2] == 0.0f, "rope " + tname(t) + ": ext_factor must be 0 (no YaRN)");
                require(x->type == GGML_TYPE_F32 && x->nb[0] == 4 && x->nb[1] % 4 == 0 && x->nb[2] % 4 == 0 &&
                            x->ne[3] == 1 && t->type == GGML_TYPE_F32,
                        "rope " + tname(t) + ": f32 [D, H, S] input");
                require(n_dims > 0 && n_dims % 2 == 0 && n_dims <= x->ne[0], "rope: n_dims must be even and <= D");
                require(ggml_is_contiguous(pos), "rope: positions must be contiguous");
                Step s = new_step(S_ROPE);
                s.in[0] = d(x);
                s.in[1] = d(pos);
                s.in[2] = ff ? d(ff) : nullptr;
                s.out = o(t);
                s.n[0] = (int64_t) x->nb[2] / 4;
                s.n[1] = (int64_t) x->nb[1] / 4;
                s.n[2] = x->ne[0] * x->ne[1];
                s.n[3] = x->ne[0];
                s.n[4] = x->ne[0];
                s.n[5] = x->ne[1];
                s.n[6] = x->ne[2];
                s.n[7] = n_dims;
                s.f[0] = fp[0];
                s.f[1] = fp[1];
                s.f[2] = fp[3];
                steps.push_back(s);
                return;
            }
            case GGML_OP_FLASH_ATTN_EXT: {
                const ggml_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2], *m = t->src[3];
                float fp[3];
                std::memcpy(fp, &t->op_params[0], sizeof(fp));
                require(fp[1] == 0.0f && fp[2] == 0.0f, "flash_attn_ext " + tname(t) + ": no ALiBi or softcap");
                require(q->type == GGML_TYPE_F32 && q->nb[0] == 4 && q->nb[1] % 4 == 0 && q->nb[2] % 4 == 0 &&
                            q->ne[3] == 1,
                        "flash_attn_ext " + tname(t) + ": q must be f32 [D, Sq, H, 1]");
                require(k->type == GGML_TYPE_F16 && v->type == GGML_TYPE_F16 && k->nb[0] == 2 && v->nb[0] == 2 &&
                            k->nb[1] % 16 == 0 && k->nb[2] % 16 == 0 && v->nb[1] % 16 == 0 && v->nb[2] % 16 == 0 &&
                            aligned16(k) && aligned16(v),
                        "flash_attn_ext " + tname(t) + ": K and V must be f16 with 16-byte rows");
                const int64_t D = q->ne[0], H = q->ne[2], Hkv = k->ne[2];
                require(v->ne[0] == D && (D == 64 || D == 128 || D == 256), "flash_attn_ext: head size 64, 128 or 256");
                require(H % Hkv == 0 && H / Hkv <= 8, "flash_attn_ext: 1 to 8 query heads per KV head");
                if (m) require(m->type == GGML_TYPE_F16 && m->nb[0] == 2 && m->nb[1] % 2 == 0 && m->ne[2] == 1,
                               "flash_attn_ext: the mask must be f16 [n_kv, Sq]");
                Step s = new_step(S_FATTN);
                s.in[0] = d(q);
                s.in[1] = d(k);
                s.in[2] = d(v);
                s.in[3] = m ? d(m) : nullptr;
                s.out = o(t);
                s.n[0] = (int64_t) q->nb[2] / 4;
                s.n[1] = (int64_t) q->nb[1] / 4;
                s.n[2] = (int64_t) k->nb[2] / 2;
                s.n[3] = (int64_t) k->nb[1] / 2;
                s.n[4] = (int64_t) v->nb[2] / 2;
                s.n[5] = (int64_t) v->nb[1] / 2;
                s.n[6] = m ? (int64_t) m->nb[1] / 2 : 0;
                s.n[7] = D;
                s.n[8] = q->ne[1];
                s.n[9] = H;
                s.n[10] = Hkv;
                s.n[11] = k->ne[1];
                s.f[0] = fp[0];
                require(s.n[11] >= 1 && s.n[8] >= 1, "flash_attn_ext: empty attention");
                ws_need = std::max(ws_need, attn_workspace((int) s.n[8], (int) H, (int) Hkv, (int) D, (int) s.n[11]));
                steps.push_back(s);
                return;
            }
            case GGML_OP_GLU: {
                require(t->op_params[0] == GGML_GLU_OP_SWIGLU && f32_contig(t->src[0]) && f32_contig(t->src[1]),
                        "glu " + tname(t) + ": swiglu of contiguous f32 operands only");
                Step s = new_step(S_SWIGLU);
                s.in[0] = d(t->src[0]);
                s.in[1] = d(t->src[1]);
                s.out = o(t);
                s.n[0] = ggml_nelements(t);
                steps.push_back(s);
                return;
            }
            case GGML_OP_UNARY: {
                require(f32_contig(t->src[0]) && unary_known(t->op_params[0]),
                        "unary " + tname(t) + ": a known function of a contiguous f32 tensor");
                Step s = new_step(S_UNARY);
                s.op = t->op_params[0];
                s.in[0] = d(t->src[0]);
                s.out = o(t);
                s.n[0] = ggml_nelements(t);
                std::memcpy(&s.f[0], &t->op_params[1], 4);
                std::memcpy(&s.f[1], &t->op_params[2], 4);
                steps.push_back(s);
                return;
            }
            case GGML_OP_REPEAT: {
                const ggml_tensor * a = t->src[0];
                require(a->type == GGML_TYPE_F32 && a->nb[0] == 4 && f32_contig(t),
                        "repeat " + tname(t) + ": an f32 source with unit element stride");
                Step s = new_step(S_REPEAT);
                s.in[0] = d(a);
                s.out = o(t);
                for (int k = 0; k < 4; k++) {
                    s.g.sne[k] = a->ne[k];
                    s.g.snb[k] = (int64_t) a->nb[k];
                    s.g.dne[k] = t->ne[k];
                    s.g.dnb[k] = (int64_t) t->nb[k];
                }
                s.n[0] = ggml_nelements(t);
                steps.push_back(s);
                return;
            }
            case GGML_OP_CONCAT: {
                // Two copies into the halves of the result: a at offset 0, b after a along dim.
                const int dim = t->op_params[0];
                const ggml_tensor * src[2] = {t->src[0], t->src[1]};
                require((t->type == GGML_TYPE_F32 || t->type == GGML_TYPE_F16) && ggml_is_contiguous(t) &&
                            src[0]->nb[0] % ggml_tsize(t->type) == 0 && src[1]->nb[0] % ggml_tsize(t->type) == 0,
                        "concat " + tname(t) + ": f32 / f16 operands");
                for (int h = 0; h < 2; h++) {
                    const ggml_tensor * a = src[h];
                    Step s = new_step(S_CPY);
                    s.type = a->type;
                    s.op = t->type;
                    s.in[0] = d(a);
                    char * base = static_cast<char *>(o(t));
                    s.out = base && h == 1 ? base + src[0]->ne[dim] * t->nb[dim] : base;
                    for (int k = 0; k < 4; k++) {
                        s.g.sne[k] = a->ne[k];
                        s.g.snb[k] = (int64_t) a->nb[k];
                        s.g.dne[k] = a->ne[k];
                        s.g.dnb[k] = (int64_t) t->nb[k];
                    }
                    s.n[0] = ggml_nelements(a);
                    steps.push_back(s);
                }
                return;
            }
            case GGML_OP_NORM:
            case GGML_OP_SUM_ROWS:
            case GGML_OP_MEAN: {
                const ggml_tensor * a = t->src[0];
                require(f32_contig(a), std::string(ggml_op_name(t->op)) + " " + tname(t) + ": needs a contiguous f32 input");
                Step s = new_step(t->op == GGML_OP_NORM ? S_NORM : S_ROWSUM);
                s.in[0] = d(a);
                s.out = o(t);
                s.n[0] = ggml_nrows(a);
                s.n[1] = a->ne[0];
                if (t->op == GGML_OP_NORM) std::memcpy(&s.f[0], &t->op_params[0], 4);
                else s.op = t->op == GGML_OP_MEAN;
                steps.push_back(s);
                return;
            }
            case GGML_OP_SOFT_MAX: {
                const ggml_tensor *a = t->src[0], *m = t->src[1];
                float fp[2];
                std::memcpy(fp, &t->op_params[0], sizeof(fp));
                require(f32_contig(a) && fp[1] == 0.0f,
                        "soft_max " + tname(t) + ": a contiguous f32 input and no ALiBi (max_bias 0)");
                Step s = new_step(S_SOFTMAX);
                s.in[0] = d(a);
                s.out = o(t);
                for (int k = 0; k < 4; k++) s.n[k] = a->ne[k];
                s.n[7] = s.n[8] = 1;
                if (m) {
                    const size_t es = ggml_tsize(m->type);
                    require((m->type == GGML_TYPE_F32 || m->type == GGML_TYPE_F16) && m->nb[0] == es &&
                                m->nb[1] % es == 0 && m->nb[2] % es == 0 && m->nb[3] % es == 0 &&
                                m->ne[0] == a->ne[0] && m->ne[1] >= a->ne[1] && a->ne[2] % m->ne[2] == 0 &&
                                a->ne[3] % m->ne[3] == 0,
                            "soft_max " + tname(t) + ": the mask must be f32 / f16 [n, >= rows, a divisor of each batch dim]");
                    s.in[1] = d(m);
                    s.type = m->type;
                    s.n[4] = (int64_t) (m->nb[1] / es);
                    s.n[5] = (int64_t) (m->nb[2] / es);
                    s.n[6] = (int64_t) (m->nb[3] / es);
                    s.n[7] = m->ne[2];
                    s.n[8] = m->ne[3];
                }
                s.f[0] = fp[0];
                steps.push_back(s);
                return;
            }
            case GGML_OP_ARGMAX: {
                int64_t rows = 0;
                size_t stride = 0;
                require(t->src[0]->type == GGML_TYPE_F32 && uniform_rows(t->src[0], rows, stride),
                        "argmax " + tname(t) + ": needs f32 rows");
                Step s = new_step(S_ARGMAX);
                s.in[0] = d(t->src[0]);
                s.out = o(t);
                s.n[0] = (int64_t) stride / 4;
                s.n[1] = rows;
                s.n[2] = t->src[0]->ne[0];
                if (!dry && argmax_split_fits(rows, s.n[2])) {  // long rows: the sliced kernel
                    if (!be->argmax_scratch) {
                        check_hip(hipMalloc(&be->argmax_scratch, argmax_split_scratch()), "hipMalloc argmax scratch");
                        check_hip(hipMemset(be->argmax_scratch, 0, argmax_split_scratch()), "hipMemset argmax scratch");
                    }
                    s.in[1] = be->argmax_scratch;
                }
                steps.push_back(s);
                return;
            }
            default:
                fail(std::string("op ") + ggml_op_name(t->op) + " (" + tname(t) + ") is not on this library's path");
        }
    }

    void attn_mulmat(const ggml_tensor * fa, const ggml_tensor * mm, const ggml_tensor * res, const ggml_tensor * y) {
        const ggml_tensor *q = fa->src[0], *k = fa->src[1], *v = fa->src[2], *m = fa->src[3];
        const ggml_tensor * w = mm->src[0];
        const int64_t D = q->ne[0], H = q->ne[2], Hkv = k->ne[2], n_kv = k->ne[1];
        require(n_kv >= 1, "flash_attn_ext: empty attention");
        Step s = new_step(S_ATTN_MULMAT);
        s.type = w->type;
        s.in[0] = d(q);
        s.in[1] = d(k);
        s.in[2] = d(v);
        s.in[3] = m ? d(m) : nullptr;
        s.in[4] = d(w);
        s.in[5] = res ? d(res) : nullptr;
        s.out = o(y);
        s.n[0] = (int64_t) q->nb[2] / 4;
        s.n[1] = (int64_t) k->nb[2] / 2;
        s.n[2] = (int64_t) k->nb[1] / 2;
        s.n[3] = (int64_t) v->nb[2] / 2;
        s.n[4] = (int64_t) v->nb[1] / 2;
        s.n[5] = D;
        s.n[6] = H;
        s.n[7] = Hkv;
        s.n[8] = n_kv;
        s.n[9] = w->ne[1];  // N
        s.n[10] = w->ne[0];  // K = H * D
        std::memcpy(&s.f[0], &fa->op_params[0], 4);
        // split plan: as many splits as the merge prologue holds at most
        const int GS = decode_group((int) (H / Hkv), (int) n_kv);
        const int nsplit = decode_splits((int) D, (int) H, GS, (int) n_kv, row_gemv_merge_max(), true);
        s.g.sne[0] = GS;
        s.g.sne[1] = nsplit;
        s.g.sne[2] = (n_kv + nsplit - 1) / nsplit;
        ws_need = std::max(ws_need, align256((size_t) H * nsplit * D * 4) + align256((size_t) H * nsplit * 8) +
                                        align256((size_t) H * D * 4));
        steps.push_back(s);
    }

    // cpy(a, b) where a is one step's whole result, read by nothing else, and b is memory that no
    // other node of g reads or writes (a stage result copied into its value, ...): the step writes
    // b itself and the copy is dropped. Same values, one launch and one pass over a fewer.
    void fold_result_copies(const ggml_cgraph * g) {
        if (dry) return;
        auto range = [](const ggml_tensor * t) {
            const uintptr_t p = (uintptr_t) t->data;
            return std::make_pair(p, p + ggml_nbytes(t));
        };
        auto overlap = [](std::pair<uintptr_t, uintptr_t> x, std::pair<uintptr_t, uintptr_t> y) {
            return x.first < y.second && y.first < x.second;
        };
        for (const ggml_tensor * t : g->nodes) {
            if (t->op != GGML_OP_CPY) continue;
            const ggml_tensor *a = t->src[0], *b = t->src[1];
            if (!a || !b || !a->data || !b->data || a->type != b->type || is_output(a) || a->view_src ||
                !ggml_is_contiguous(a) || !ggml_is_contiguous(b) || !ggml_is_contiguous(t) ||
                ggml_nelements(a) != ggml_nelements(b) || t->data != b->data)
                continue;
            int readers = 0;
            bool shared = false;
            const auto rb = range(b);
            for (const ggml_tensor * n : g->nodes) {
                if (n->view_src == a) readers++;
                for (const ggml_tensor * s : n->src) {
                    if (s == a) readers++;
                    if (n != t && s && s->data && overlap(range(s), rb)) shared = true;
                }
                if (n != t && n->data && overlap(range(n), rb)) shared = true;
            }
            if (readers != 1 || shared) continue;
            // a's producer: the last step before the copy that writes a's memory (steps before it
            // may have written other tensors the allocator placed there earlier)
            int prod = -1, cpy = -1;
            for (int i = 0; i < (int) steps.size(); i++) {
                const Step & s = steps[i];
                if (s.kind == S_CPY && s.in[0] == a->data && s.out == t->data) {
                    cpy = i;
                    break;
                }
                if (s.out == a->data || s.out2[0] == a->data || s.out2[1] == a->data) prod = i;
            }
            if (cpy < 0 || prod < 0) continue;
            Step & p = steps[(size_t) prod];
            const bool whole = p.out == a->data && (p.kind == S_MULMAT || p.kind == S_ARGMAX ||
                                                    p.kind == S_ATTN_MULMAT || p.kind == S_GATE_UP);
            if (!whole) continue;
            p.out = mut_data(b);
            steps.erase(steps.begin() + cpy);
        }
    }

    // Runs of 2 or 3 consecutive small get_rows / cpy / rope-table steps, none reading or writing
    // what another of the run writes, become one launch: an S_JOBS marker in front of them (a
    // decode graph's embedding row, mask cast and rotation table are such a run).
    void group_small_steps() {
        if (dry || !be->fuse) return;
        struct Span {
            uintptr_t lo, hi;
        };
        auto extent = [](const int64_t * ne, const int64_t * nb, int64_t es) {
            int64_t e = es;
            for (int k = 0; k < 4; k++) e += (ne[k] - 1) * nb[k];
            return e;
        };
        // the bytes a step reads (up to two spans) and writes; false: not a small job
        auto spans = [&](const Step & s, Span (&rd)[2], Span & wr) {
            auto sp = [](const void * p, int64_t n) { return Span{(uintptr_t) p, (uintptr_t) p + (uintptr_t) n}; };
            if (s.kind == S_GETROWS) {
                if (s.n[1] * s.n[2] > (1 << 20)) return false;
                rd[0] = sp(s.in[0], s.n[0] * (int64_t) row_bytes(s.type, s.n[1]));
                rd[1] = sp(s.in[1], s.n[2] * 4);
                wr = sp(s.out, s.n[1] * s.n[2] * 4);
                return true;
            }
            if (s.kind == S_CPY) {
                if (s.n[0] > (1 << 20)) return false;
                const int64_t ss = s.type == T_F16 ? 2 : 4, ds = s.op == T_F16 ? 2 : 4;
                rd[0] = sp(s.in[0], extent(s.g.sne, s.g.snb, ss));
                rd[1] = sp(s.in[0], 0);
                wr = sp(s.out, extent(s.g.dne, s.g.dnb, ds));
                return true;
            }
            if (s.kind == S_ROPE_TABLE) {
                rd[0] = sp(s.in[0], 4);
                rd[1] = rd[0];
                wr = sp(be->rope_cs, s.n[0] / 2 * (int64_t) sizeof(float2));
                return true;
            }
            return false;
        };
        auto meet = [](Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; };
        std::vector<Step> out;
        out.reserve(steps.size() + 4);
        for (size_t i = 0; i < steps.size();) {
            Span rd[3][2], wr[3];
            size_t n = 0;
            while (n < 3 && i + n < steps.size() && spans(steps[i + n], rd[n], wr[n])) {
                bool free = true;
                for (size_t k = 0; k < n && free; k++)
                    free = !meet(wr[k], wr[n]) && !meet(wr[k], rd[n][0]) && !meet(wr[k], rd[n][1]) &&
                           !meet(wr[n], rd[k][0]) && !meet(wr[n], rd[k][1]);
                if (!free) break;
                n++;
            }
            if (n >= 2) {
                Step m = new_step(S_JOBS);
                m.n[0] = (int64_t) n;
                out.push_back(m);
            }
            const size_t take = std::max<size_t>(n, 1);
            for (size_t k = 0; k < take; k++) out.push_back(steps[i + k]);
            i += take;
        }
        steps.swap(out);
    }

    // The chain ending at node f (members before it, in order).
    void chain(const ggml_cgraph * g, const std::vector<int> & idx) {
        const ggml_tensor * first = g->nodes[idx.front()];
        const ggml_tensor * last = g->nodes[idx.back()];
        if (first->op == GGML_OP_FLASH_ATTN_EXT) {  // [attention, reshape, mul_mat (, add)]
            const ggml_tensor * mm = g->nodes[idx[2]];
            const ggml_tensor * res = idx.size() == 4 ? (last->src[0] == mm ? last->src[1] : last->src[0]) : nullptr;
            return attn_mulmat(first, mm, res, last);
        }
        if (first->op == GGML_OP_RMS_NORM) {
            const ggml_tensor * mul = g->nodes[idx[1]];
            if (idx.size() == 2) return rmsnorm(first, mul->src[1], mul);
            const ggml_tensor * mm = g->nodes[idx[2]];
            float eps;
            std::memcpy(&eps, &first->op_params[0], 4);
            const ggml_tensor * res = idx.size() == 4 ? (last->src[0] == mm ? last->src[1] : last->src[0]) : nullptr;
            return mulmat(mm, first->src[0], mul->src[1], eps, res, last);
        }
        if (first->op == GGML_OP_GLU) {
            const ggml_tensor * mm = g->nodes[idx[1]];
            const ggml_tensor * res = idx.size() == 3 ? (last->src[0] == mm ? last->src[1] : last->src[0]) : nullptr;
            return swiglu_mulmat(first, mm, res, last);
        }
        // mul_mat -> add
        const ggml_tensor * res = last->src[0] == first ? last->src[1] : last->src[0];
        return mulmat(first, first->src[1], nullptr, 0.0f, res, last);
    }
};

// ------------------------------------------------------------------------------- running

// A small step as a job of k_small_jobs (the same arguments as its own launch below).
SmallJob small_job(const ggml_backend * be, const Step & s) {
    if (s.kind == S_GETROWS)
        return small_job_get_rows(s.type, s.in[0], s.n[0], s.n[1], (const int32_t *) s.in[1], s.n[2], (float *) s.out);
    if (s.kind == S_CPY) return small_job_cpy(s.in[0], s.type, s.out, s.op, s.g, s.n[0]);
    require(s.kind == S_ROPE_TABLE, "small jobs: get_rows, cpy or rope table steps only");
    return small_job_rope_table((const int32_t *) s.in[0], (int) s.n[0], s.f[0], s.f[1], s.f[2], nullptr, be->rope_cs);
}

void run_step(const ggml_backend * be, const Step & s) {
    hipStream_t st = be->stream;
    switch (s.kind) {
        case S_MULMAT: {
            const int wt = s.type;
            const int64_t N = s.n[0], K = s.n[1], M = s.n[2], ldx = s.n[3], ldy = s.n[4];
            const float * x = (const float *) s.in[1];
            const float * nw = (const float *) s.in[2];
            const float * res = (const float *) s.in[3];
            float * y = (float *) s.out;
            if (M == 1 && (wt == T_Q4_0 || wt == T_Q8_0) && row_gemv_fits(wt, K)) {
                const WeightLayout L = weight_layout(wt, N, K);
                RowArgs a{};
                a.wqs = (const uint8_t *) s.in[0] + L.qs;
                a.wd = (const uint16_t *) ((const uint8_t *) s.in[0] + L.d);
                a.N = (int) N;
                a.nb = (int) (K / QK);
                a.x = x;
                a.norm_w = nw;
                a.eps = s.f[0];
                a.y = y;
                a.res = res;
                launch_row_gemv(wt, nw ? PRO_NORM : PRO_PLAIN, EPI_STORE, a, st);
                return;
            }
            // one launch, the row (normalized and) quantized in it
            if (M == 1 && (nw ? row_gemv_kq_norm_fits(wt, N, K) : row_gemv_kq_fits(wt, N, K)) && aligned(x, 16)) {
                launch_row_gemv_kq(wt, s.in[0], N, K, x, nw, s.f[0], y, res, st);
                return;
            }
            // a folded norm reaches a K-quant weight only through the row kernel above
            require(!nw || wt == T_Q4_0 || wt == T_Q8_0, "mul_mat: a normalized row for a K-quant weight off its row kernel");
            if (nw) launch_rmsnorm_q8(x, ldx, nw, s.f[0], M, K, be->ws, st);
            else launch_act_quant(wt, x, ldx, M, K, be->ws, st);
            if (M <= 8) launch_gemv(wt, s.in[0], N, K, be->ws, M, y, ldy, st, res);
            else if (is_kquant(wt)) launch_gemm_kq(wt, s.in[0], N, K, be->ws, M, y, ldy, st, res);
            else launch_gemm(wt, s.in[0], N, K, be->ws, M, y, ldy, st, res);
            return;
        }
        case S_ROPE_TABLE:
            launch_rope_table((const int32_t *) s.in[0], (int) s.n[0], s.f[0], s.f[1], s.f[2], nullptr, be->rope_cs,
                              st);
            return;
        case S_QKV_ROPE: {
            const uint8_t * w[3] = {(const uint8_t *) s.in[0], (const uint8_t *) s.in[3], (const uint8_t *) s.in[4]};
            if (is_kquant(s.type)) {
                const int vtype = (int) s.m[0];
                const int nqk = vtype == s.type ? 3 : 2;  // v of another type: a launch of its own
                RowKqArgs a{};
                require(row_gemv_kq_ranges(s.type, nqk, w, s.n, s.n[3], a), "q / k / v rope: weights do not fit one launch");
                a.x = (const float *) s.in[1];
                a.norm_w = (const float *) s.in[2];
                a.eps = s.f[0];
                a.y = (float *) s.out;
                a.pos = (const int *) s.in[5];
                a.rope_cs = be->rope_cs;
                a.kc = (uint16_t *) s.out2[0];
                a.vc = (uint16_t *) s.out2[1];
                a.H = (int) s.n[4];
                a.Hkv = (int) s.n[5];
                a.D = (int) s.n[6];
                a.ctx = s.n[7];
                launch_row_gemv_kq_epi(s.type, PRO_NORM, EPI_ROPE_KV, a, st);
                if (nqk == 2) {
                    RowKqArgs b{};
                    row_gemv_kq_one(vtype, w[2], s.n[2], s.n[3], b);
                    b.x = a.x;
                    b.norm_w = a.norm_w;
                    b.eps = a.eps;
                    b.pos = a.pos;
                    b.vc = a.vc;
                    b.Hkv = a.Hkv;
                    b.D = a.D;
                    b.ctx = a.ctx;
                    launch_row_gemv_kq_epi(vtype, PRO_NORM, EPI_V_CACHE, b, st);
                }
                return;
            }
            RowArgs a{};
            require(row_gemv_ranges(s.type, 3, w, s.n, s.n[3], a), "q / k / v rope: weights do not fit one launch");
            a.x = (const float *) s.in[1];
            a.norm_w = (const float *) s.in[2];
            a.eps = s.f[0];
            a.y = (float *) s.out;
            a.pos = (const int *) s.in[5];
            a.rope_cs = be->rope_cs;
            a.kc = (uint16_t *) s.out2[0];
            a.vc = (uint16_t *) s.out2[1];
            a.H = (int) s.n[4];
            a.Hkv = (int) s.n[5];
            a.D = (int) s.n[6];
            a.ctx = s.n[7];
            launch_row_gemv(s.type, PRO_NORM, EPI_ROPE_KV, a, st);
            return;
        }
        case S_GATE_UP: {
            const uint8_t * w[2] = {(const uint8_t *) s.in[0], (const uint8_t *) s.in[3]};
            if (is_kquant(s.type)) {
                RowKqArgs a{};
                require(row_gemv_kq_ranges(s.type, 2, w, s.n, s.n[3], a), "gate / up: weights do not fit one launch");
                a.x = (const float *) s.in[1];
                a.norm_w = (const float *) s.in[2];
                a.eps = s.f[0];
                a.y = (float *) s.out;
                launch_row_gemv_kq_epi(s.type, PRO_NORM, EPI_SWIGLU, a, st);
                return;
            }
            RowArgs a{};
            require(row_gemv_ranges(s.type, 2, w, s.n, s.n[3], a), "gate / up: weights do not fit one launch");
            a.x = (const float *) s.in[1];
            a.norm_w = (const float *) s.in[2];
            a.eps = s.f[0];
            a.y = (float *) s.out;
            launch_row_gemv(s.type, PRO_NORM, EPI_SWIGLU, a, st);
            return;
        }
        case S_MULMAT3: {
            const int n = s.in[4] ? 3 : 2;
            const uint8_t * w[3] = {(const uint8_t *) s.in[0], (const uint8_t *) s.in[3], (const uint8_t *) s.in[4]};
            if (is_kquant(s.type)) {
                RowKqArgs a{};
                require(row_gemv_kq_ranges(s.type, n, w, s.n, s.n[3], a), "mul_mat group: weights do not fit one launch");
                a.x = (const float *) s.in[1];
                a.norm_w = (const float *) s.in[2];
                a.eps = s.f[0];
                a.r_y[0] = (float *) s.out;
                a.r_y[1] = (float *) s.out2[0];
                a.r_y[2] = (float *) s.out2[1];
                launch_row_gemv_kq_epi(s.type, PRO_NORM, EPI_STORE, a, st);
                return;
            }
            RowArgs a{};
            require(row_gemv_ranges(s.type, n, w, s.n, s.n[3], a), "mul_mat group: weights do not fit one launch");
            a.x = (const float *) s.in[1];
            a.norm_w = (const float *) s.in[2];
            a.eps = s.f[0];
            a.r_y[0] = (float *) s.out;
            a.r_y[1] = (float *) s.out2[0];
            a.r_y[2] = (float *) s.out2[1];
            launch_row_gemv(s.type, PRO_NORM, EPI_STORE, a, st);
            return;
        }
        case S_SWIGLU_MULMAT: {
            const int64_t N = s.n[0], K = s.n[1], M = s.n[2], n = s.n[3];
            if (M == 1 && (s.type == T_Q4_0 || s.type == T_Q8_0) && row_gemv_fits(s.type, K) &&
                aligned(s.in[1], 16) && aligned(s.in[2], 16)) {  // one launch: silu(g) * u quantized in the GEMV
                const WeightLayout L = weight_layout(s.type, N, K);
                RowArgs a{};
                a.wqs = (const uint8_t *) s.in[0] + L.qs;
                a.wd = (const uint16_t *) ((const uint8_t *) s.in[0] + L.d);
                a.N = (int) N;
                a.nb = (int) (K / QK);
                a.x = (const float *) s.in[1];
                a.up = (const float *) s.in[2];
                a.y = (float *) s.out;
                a.res = (const float *) s.in[3];
                launch_row_gemv(s.type, PRO_SWIGLU, EPI_STORE, a, st);
                return;
            }
            launch_swiglu_q8((const float *) s.in[1], (const float *) s.in[2], n, n, M, be->ws, st);
            if (M <= 8) launch_gemv(s.type, s.in[0], N, K, be->ws, M, (float *) s.out, N, st, (const float *) s.in[3]);
            else launch_gemm(s.type, s.in[0], N, K, be->ws, M, (float *) s.out, N, st, (const float *) s.in[3]);
            return;
        }
        case S_RMSNORM:
            launch_rms_norm((const float *) s.in[0], s.n[0], (float *) s.out, s.n[2], (const float *) s.in[1], s.n[1],
                            s.n[2], s.f[0], st);
            return;
        case S_BINARY:
            if (s.n[2]) launch_binary_bcast(s.op, (const float *) s.in[0], (const float *) s.in[1], (float *) s.out, &s.m[0], &s.m[4], st);
            else launch_binary(s.op, (const float *) s.in[0], (const float *) s.in[1], (float *) s.out, s.n[0], s.n[1], st);
            return;
        case S_SCALE:
            launch_scale((const float *) s.in[0], (float *) s.out, s.n[0], s.f[0], s.f[1], st);
            return;
        case S_CPY:
            launch_cpy(s.in[0], s.type, s.out, s.op, s.g, s.n[0], st);
            return;
        case S_GETROWS:
            launch_get_rows(s.type, s.in[0], s.n[0], s.n[1], (const int32_t *) s.in[1], s.n[2], (float *) s.out, st);
            return;
        case S_SETROWS:
            launch_set_rows_f16(s.out, s.n[0], s.n[1], (const float *) s.in[0], s.n[2], s.n[3],
                                (const int32_t *) s.in[1], s.n[4], s.n[5], s.n[6], s.n[7], st);
            return;
        case S_SETROWS2: {
            const SetRowsSecond r2{(uint16_t *) s.out2[0], s.m[0], s.m[1], (const float *) s.in[3], s.m[2], s.m[3],
                                   (int) s.m[4], (int) s.m[5], s.m[6]};
            launch_set_rows_f16(s.out, s.n[0], s.n[1], (const float *) s.in[0], s.n[2], s.n[3],
                                (const int32_t *) s.in[1], s.n[4], s.n[5], s.n[6], s.n[7], st, &r2);
            return;
        }
        case S_ROPE2: {
            const RopeSecond r2{(const float *) s.in[3], s.m[0], s.m[1], (float *) s.out2[0], s.m[2], s.m[3], s.m[4]};
            launch_rope_neox((const float *) s.in[0], s.n[0], s.n[1], (float *) s.out, s.n[2], s.n[3],
                             (const int32_t *) s.in[1], s.n[4], s.n[5], s.n[6], (int) s.n[7], s.f[0], s.f[1], s.f[2],
                             (const float *) s.in[2], st, &r2);
            return;
        }
        case S_ROPE:
            launch_rope_neox((const float *) s.in[0], s.n[0], s.n[1], (float *) s.out, s.n[2], s.n[3],
                             (const int32_t *) s.in[1], s.n[4], s.n[5], s.n[6], (int) s.n[7], s.f[0], s.f[1], s.f[2],
                             (const float *) s.in[2], st);
            return;
        case S_FATTN:
            launch_flash_attn((const float *) s.in[0], s.n[0], s.n[1], s.in[1], s.n[2], s.n[3], s.in[2], s.n[4], s.n[5],
                              s.in[3], s.n[6], (float *) s.out, (int) s.n[7], (int) s.n[7], (int) s.n[8], (int) s.n[9],
                              (int) s.n[10], (int) s.n[11], s.f[0], be->ws, be->ws_size, st);
            return;
        case S_SWIGLU:
            launch_swiglu((const float *) s.in[0], (const float *) s.in[1], (float *) s.out, s.n[0], st);
            return;
        case S_UNARY:
            launch_unary(s.op, (const float *) s.in[0], (float *) s.out, s.n[0], s.f[0], s.f[1], st);
            return;
        case S_REPEAT:
            launch_repeat((const float *) s.in[0], (float *) s.out, s.g, s.n[0], st);
            return;
        case S_NORM:
            launch_norm((const float *) s.in[0], (float *) s.out, s.n[0], s.n[1], s.f[0], st);
            return;
        case S_MULMAT_F: {
            const int64_t anb[4] = {1, s.m[4], s.m[5], s.m[6]}, bnb[4] = {1, s.n[4], s.n[5], s.n[6]};
            launch_mul_mat_f(s.type == GGML_TYPE_F16, s.in[0], &s.m[0], anb, (const float *) s.in[1], &s.n[0], bnb,
                             (float *) s.out, st);
            return;
        }
        case S_ROWSUM:
            launch_row_sum((const float *) s.in[0], (float *) s.out, s.n[0], s.n[1], s.op != 0, st);
            return;
        case S_SOFTMAX:
            launch_soft_max((const float *) s.in[0], (float *) s.out, s.n[0], s.n[1], s.n[2], s.n[3], s.in[1],
                            s.type == GGML_TYPE_F16, s.n[4], s.n[5], s.n[6], s.n[7], s.n[8], s.f[0], st);
            return;
        case S_ARGMAX:
            if (s.in[1]) launch_argmax_split((const float *) s.in[0], s.n[0], s.n[1], s.n[2], (int32_t *) s.out,
                                             (void *) s.in[1], st);
            else launch_argmax((const float *) s.in[0], s.n[0], s.n[1], s.n[2], (int32_t *) s.out, st);
            return;
        case S_ATTN_MULMAT: {
            const int64_t D = s.n[5], H = s.n[6], Hkv = s.n[7], n_kv = s.n[8], N = s.n[9], K = s.n[10];
            const int GS = (int) s.g.sne[0], nsplit = (int) s.g.sne[1], chunk = (int) s.g.sne[2];
            float * po = (float *) be->ws;
            float2 * pml = (float2 *) ((uint8_t *) be->ws + align256((size_t) H * nsplit * D * 4));
            float * row = (float *) ((uint8_t *) pml + align256((size_t) H * nsplit * 8));
            launch_attn_decode((const float *) s.in[0], s.n[0], s.in[1], s.n[1], s.n[2], s.in[2], s.n[3], s.n[4],
                               (int) D, (int) H, (int) Hkv, (int) n_kv, nullptr, s.f[0], nsplit, chunk, (int) n_kv, GS,
                               row, po, pml, st, nullptr, s.in[3], 16);
            if (is_kquant(s.type)) {  // the K-quant row GEMV, the row merged (or read) in its prologue
                RowKqArgs a{};
                row_gemv_kq_one(s.type, s.in[4], N, K, a);
                a.y = (float *) s.out;
                a.res = (const float *) s.in[5];
                if (nsplit == 1) {
                    a.x = row;
                    launch_row_gemv_kq_epi(s.type, PRO_PLAIN, EPI_STORE, a, st);
                } else {
                    a.part_o = po;
                    a.part_ml = pml;
                    a.nsplit = nsplit;
                    a.D = (int) D;
                    launch_row_gemv_kq_epi(s.type, PRO_MERGE, EPI_STORE, a, st);
                }
                return;
            }
            const WeightLayout L = weight_layout(s.type, N, K);
            RowArgs a{};
            a.wqs = (const uint8_t *) s.in[4] + L.qs;
            a.wd = (const uint16_t *) ((const uint8_t *) s.in[4] + L.d);
            a.N = (int) N;
            a.nb = (int) (K / QK);
            a.y = (float *) s.out;
            a.res = (const float *) s.in[5];
            if (nsplit == 1) {  // the kernel wrote the normalized row
                a.x = row;
                launch_row_gemv(s.type, PRO_PLAIN, EPI_STORE, a, st);
            } else {
                a.part_o = po;
                a.part_ml = pml;
                a.nsplit = nsplit;
                a.D = (int) D;
                launch_row_gemv(s.type, PRO_MERGE, EPI_STORE, a, st);
            }
            return;
        }
    }
}

// The plan's steps in order; an S_JOBS marker launches the steps it covers as one kernel.
void run_steps(const ggml_backend * be) {
    const std::vector<Step> & v = be->steps;
    for (size_t i = 0; i < v.size(); i++) {
        if (v[i].kind != S_JOBS) {
            run_step(be, v[i]);
            continue;
        }
        const int n = (int) v[i].n[0];
        require(n >= 1 && n <= 3 && i + (size_t) n < v.size(), "small jobs: bad run");
        SmallJob j[3];
        for (int k = 0; k < n; k++) j[k] = small_job(be, v[i + 1 + (size_t) k]);
        launch_small_jobs(j, n, be->stream);
        i += (size_t) n;
    }
}

// Gives every view of g its base's memory (views made before their base was allocated, or whose
// base has moved since).
void refresh_views(ggml_cgraph * g) {
    for (auto * list : {&g->leafs, &g->nodes})
        for (ggml_tensor * t : *list)
            if (t->view_src && t->view_src->data) {
                t->data = (char *) t->view_src->data + t->view_offs;
                t->buffer = t->view_src->buffer;
            }
}

// Plans (or replays) g on the backend's stream; waits for it unless `async`.
enum ggml_status compute(ggml_backend * be, ggml_cgraph * g, bool async = false) {
    require(g != nullptr, "graph is NULL");
    require(g->error.empty(), g->error);
    if (g->nodes.empty()) return GGML_STATUS_SUCCESS;
    set_device(be);
    refresh_views(g);
    std::vector<uintptr_t> fp = fingerprint(g);
    if (be->use_graphs) {  // unchanged since the last compute: replay without planning
        auto it = be->graphs.find(g);
        if (it != be->graphs.end() && it->second.exec && it->second.fp == fp) {
            check_hip(hipGraphLaunch(it->second.exec, be->stream), "hipGraphLaunch");
            if (!async) check_hip(hipStreamSynchronize(be->stream), "graph compute");
            return GGML_STATUS_SUCCESS;
        }
    }
    const Chains c = find_chains(g, be->fuse);
    be->steps.clear();
    Planner p{be, be->steps};
    p.folded = &c.folded;
    std::vector<int> idx;
    for (int i = 0; i < (int) g->nodes.size(); i++) {
        if (c.member[i]) continue;
        if (c.sib[i] >= 0) {
            const size_t gi = (size_t) c.sib[i];
            const std::vector<int> & grp = c.groups[gi];
            if (i == c.first[gi]) {
                if (c.kind[gi] == 0) p.mulmat_group(g, grp);
                else if (c.kind[gi] == 3) p.qkv_rope(g, grp);
                else if (c.kind[gi] == 4) p.gate_up(g, grp);
                else p.pair(g->nodes[grp[0]], g->nodes[grp[1]]);
            }
            continue;
        }
        idx.clear();
        for (int j = 0; j < i; j++)  // members of the chain ending here, in order
            if (c.member[j] && !c.in_fold[j] && c.end[j] == i) idx.push_back(j);
        if (idx.empty()) {
            p.node(g->nodes[i]);
        } else {
            idx.push_back(i);
            p.chain(g, idx);
        }
    }
    p.fold_result_copies(g);
    p.group_small_steps();
    ensure_ws(be, p.ws_need);
    std::vector<uint8_t> sig((const uint8_t *) be->steps.data(),
                             (const uint8_t *) (be->steps.data() + be->steps.size()));
    const uint8_t * wsp = (const uint8_t *) &be->ws;
    sig.insert(sig.end(), wsp, wsp + sizeof(void *));
    if (!be->use_graphs) {
        run_steps(be);
    } else {
        Cached & cc = be->graphs[g];
        if (!cc.exec || cc.sig != sig) {
            if (cc.exec) check_hip(hipGraphExecDestroy(cc.exec), "hipGraphExecDestroy");
            cc.exec = nullptr;
            cc.sig.clear();
            cc.fp.clear();
            check_hip(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            hipGraph_t graph = nullptr;
            try {
                run_steps(be);
            } catch (...) {
                (void) hipStreamEndCapture(be->stream, &graph);
                if (graph) (void) hipGraphDestroy(graph);
                throw;
            }
            check_hip(hipStreamEndCapture(be->stream, &graph), "hipStreamEndCapture");
            const hipError_t e = hipGraphInstantiate(&cc.exec, graph, nullptr, nullptr, 0);
            (void) hipGraphDestroy(graph);
            check_hip(e, "hipGraphInstantiate");
            cc.sig = std::move(sig);
        }
        cc.fp = std::move(fp);
        check_hip(hipGraphLaunch(cc.exec, be->stream), "hipGraphLaunch");
    }
    if (!async) check_hip(hipStreamSynchronize(be->stream), "graph compute");
    return GGML_STATUS_SUCCESS;
}

// ------------------------------------------------------------------------- graph allocator

// First-fit placement of byte ranges (256-byte granules) with merging of freed neighbours.
struct Arena {
    std::map<size_t, size_t> holes;  // offset -> size, below top
    size_t top = 0, peak = 0;
    size_t take(size_t n) {
        n = align256(std::max<size_t>(n, 1));
        for (auto it = holes.begin(); it != holes.end(); ++it) {
            if (it->second < n) continue;
            const size_t off = it->first, left = it->second - n;
            holes.erase(it);
            if (left) holes[off + n] = left;
            return off;
        }
        const size_t off = top;
        top += n;
        peak = std::max(peak, top);
        return off;
    }
    void give(size_t off, size_t n) {
        n = align256(std::max<size_t>(n, 1));
        auto it = holes.emplace(off, n).first;
        auto nx = std::next(it);
        if (nx != holes.end() && it->first + it->second == nx->first) {
            it->second += nx->second;
            holes.erase(nx);
        }
        if (it != holes.begin()) {
            auto pv = std::prev(it);
            if (pv->first + pv->second == it->first) {
                pv->second += it->second;
                holes.erase(it);
                it = pv;
            }
        }
        if (it->first + it->second == top) {
            top = it->first;
            holes.erase(it);
        }
    }
};

// Offsets for every tensor of g this allocator places; the buffer size they need.
size_t place(ggml_gallocr * ga, ggml_cgraph * g, std::vector<std::pair<ggml_tensor *, size_t>> & where) {
    require(g->error.empty(), g->error);
    const int n = (int) g->nodes.size();
    const Chains c = find_chains(g, ga->be->fuse);
    // Needs memory: no data yet (or placed by this allocator before), not a view, not folded.
    // Tensors of graphs placed earlier are never touched: their contexts may be gone.
    auto needs = [&](const ggml_tensor * t) { return !t->view_src && (!t->data || t->buffer == &ga->buf); };
    std::unordered_map<const ggml_tensor *, int> last;
    std::unordered_map<const ggml_tensor *, bool> keep;
    for (ggml_tensor * t : g->leafs) keep[t] = true;
    for (int i = 0; i < n; i++) {
        const ggml_tensor * t = g->nodes[i];
        if (t->flags & (GGML_TENSOR_FLAG_OUTPUT | GGML_TENSOR_FLAG_INPUT)) keep[base_of(t)] = true;
        for (const ggml_tensor * s : t->src) {
            if (!s) continue;
            const ggml_tensor * b = base_of(s);
            last[b] = std::max(last.count(b) ? last[b] : -1, c.end[i]);
        }
    }
    keep[base_of(g->nodes[n - 1])] = true;
    Arena A;
    for (ggml_tensor * t : g->leafs)
        if (needs(t)) where.emplace_back(t, A.take(alloc_size(t)));
    std::vector<std::vector<const ggml_tensor *>> dies(n);
    for (auto & kv : last)
        if (!keep.count(kv.first)) dies[kv.second].push_back(kv.first);
    std::unordered_map<const ggml_tensor *, size_t> off;
    for (int i = 0; i < n; i++) {
        ggml_tensor * t = g->nodes[i];
        if (c.sib[i] >= 0) {  // one launch at the group's first node writes every result
            const size_t gi = (size_t) c.sib[i];
            const std::vector<int> & grp = c.groups[gi];
            if (i == c.first[gi]) {
                // kind 3 writes rope_q's result only (and the caches in place), kind 4 the glu's
                const int only = c.kind[gi] == 3 ? 3 : c.kind[gi] == 4 ? 2 : -1;
                const size_t nres = only >= 0 ? 1 : grp.size();
                for (size_t q = 0; q < nres; q++) {
                    ggml_tensor * u = g->nodes[grp[only >= 0 ? (size_t) only : q]];
                    if (!needs(u)) continue;
                    const size_t o = A.take(alloc_size(u));
                    off[u] = o;
                    where.emplace_back(u, o);
                }
            }
        } else if (!c.member[i] && needs(t)) {
            const size_t o = A.take(alloc_size(t));
            off[t] = o;
            where.emplace_back(t, o);
        }
        for (const ggml_tensor * b : dies[i]) {
            auto it = off.find(b);
            if (it != off.end()) A.give(it->second, alloc_size(b));
        }
    }
    return A.peak;
}

}  // namespace

// ---------------------------------------------------------------------------------- C API

extern "C" {

ggml_backend_t ggml_backend_hip_init(int device) {
    ggml_backend * be = nullptr;
    const int rc = guarded([&] {
        int n = 0;
        check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
        require(device >= 0 && device < n, "HIP device " + std::to_string(device) + " of " + std::to_string(n));
        hipDeviceProp_t pr;
        check_hip(hipGetDeviceProperties(&pr, device), "hipGetDeviceProperties");
        require(std::strncmp(pr.gcnArchName, "gfx950", 6) == 0,
                std::string("device ") + std::to_string(device) + " is " + pr.gcnArchName + ", not gfx950");
        auto b = std::make_unique<ggml_backend>();
        b->device = device;
        b->name = "HIP" + std::to_string(device);
        b->buft.be = b.get();
        check_hip(hipSetDevice(device), "hipSetDevice");
        check_hip(hipStreamCreate(&b->stream), "hipStreamCreate");
        be = b.release();
    });
    if (rc) (void) hipGetLastError();
    return be;
}

bool ggml_backend_is_hip(ggml_backend_t backend) { return backend != nullptr; }

void ggml_backend_free(ggml_backend_t backend) { delete backend; }

const char * ggml_backend_name(ggml_backend_t backend) { return backend ? backend->name.c_str() : "NULL"; }

void ggml_backend_synchronize(ggml_backend_t backend) {
    if (backend) (void) hipStreamSynchronize(backend->stream);
}

ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return backend ? &backend->buft : nullptr;
}

const char * ggml_backend_buft_name(ggml_backend_buffer_type_t buft) {
    return buft ? buft->be->name.c_str() : "NULL";
}

void ggml_backend_hip_set_use_graphs(ggml_backend_t backend, bool use) {
    if (backend) backend->use_graphs = use;
}

bool ggml_backend_supports_op(ggml_backend_t backend, const ggml_tensor * op) {
    if (!backend || !op) return false;
    std::vector<Step> steps;
    Planner p{backend, steps};
    p.dry = true;
    return guarded([&] { p.node(op); }) == 0;
}

}  // extern "C"

namespace gcq {

enum ggml_status graph_compute_async(ggml_backend_t backend, ggml_cgraph * cgraph) {
    enum ggml_status st = GGML_STATUS_FAILED;
    require(backend != nullptr, "graph compute: backend is NULL");
    st = compute(backend, cgraph, true);
    return st;
}

hipStream_t backend_stream(ggml_backend_t backend) { return backend ? backend->stream : nullptr; }

uint64_t backend_epoch(ggml_backend_t backend) { return backend ? backend->epoch : 0; }

void backend_activate(ggml_backend_t backend) {
    require(backend != nullptr, "backend is NULL");
    set_device(backend);
}

void backend_set_fusion(ggml_backend_t backend, bool on) {
    if (backend) backend->fuse = on;
}

}  // namespace gcq

extern "C" {

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, ggml_cgraph * cgraph) {
    enum ggml_status st = GGML_STATUS_FAILED;
    if (!backend) {
        set_error("ggml_backend_graph_compute: backend is NULL");
        return st;
    }
    if (guarded([&] { st = compute(backend, cgraph); })) return GGML_STATUS_FAILED;
    return st;
}

size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor * tensor) {
    return tensor ? alloc_size(tensor) : 0;
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(ggml_context * ctx, ggml_backend_buffer_type_t buft) {
    ggml_backend_buffer * buf = nullptr;
    guarded([&] {
        require(ctx && buft, "alloc_ctx_tensors: NULL context or buffer type");
        size_t total = 0;
        for (ggml_tensor * t : ctx->tensors)
            if (!t->data && !t->view_src) total += align256(alloc_size(t));
        if (total == 0) {
            set_error("alloc_ctx_tensors: no tensor without memory");
            return;
        }
        set_device(buft->be);
        auto b = std::make_unique<ggml_backend_buffer>();
        b->be = buft->be;
        check_hip(hipMalloc(&b->base, total), "hipMalloc");
        b->size = total;
        size_t off = 0;
        for (ggml_tensor * t : ctx->tensors) {
            if (t->data || t->view_src) continue;
            t->data = (char *) b->base + off;
            t->buffer = b.get();
            off += align256(alloc_size(t));
        }
        for (ggml_tensor * t : ctx->tensors)
            if (t->view_src && t->view_src->data) {
                t->data = (char *) t->view_src->data + t->view_offs;
                t->buffer = t->view_src->buffer;
            }
        buf = b.release();
    });
    return buf;
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(ggml_context * ctx, ggml_backend_t backend) {
    return ggml_backend_alloc_ctx_tensors_from_buft(ctx, ggml_backend_get_default_buffer_type(backend));
}

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->base) (void) hipFree(buffer->base);
    delete buffer;
}

size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer ? buffer->size : 0; }
void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) { return buffer ? buffer->base : nullptr; }
bool ggml_backend_buffer_is_host(ggml_backend_buffer_t) { return false; }

void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    if (!buffer || !buffer->base) return;
    guarded([&] {
        set_device(buffer->be);
        check_hip(hipMemset(buffer->base, value, buffer->size), "buffer_clear");
    });
}

void ggml_backend_tensor_set(ggml_tensor * t, const void * data, size_t offset, size_t size) {
    guarded([&] {
        require(t && data, "tensor_set: NULL tensor or data");
        const ggml_tensor * b = base_of(t);
        require(b->buffer && t->data, "tensor_set: " + tname(t) + " is not in a HIP buffer");
        const size_t nb = ggml_nbytes(t);
        require(offset + size <= nb, "tensor_set: " + std::to_string(offset + size) + " bytes into " + tname(t) +
                                         " of " + std::to_string(nb));
        ggml_backend * be = b->buffer->be;
        set_device(be);
        if (is_packed_type(t->type)) {
            require(t == b && offset == 0 && size == nb,
                    "tensor_set: a " + std::string(ggml_type_name(t->type)) +
                        " tensor is set whole (offset 0, ggml_nbytes bytes), not as a view or a part");
            void * tmp = nullptr;
            check_hip(hipMalloc(&tmp, size), "hipMalloc");
            hipError_t e = hipMemcpy(tmp, data, size, hipMemcpyHostToDevice);
            if (e == hipSuccess) {
                try {
                    launch_pack(t->type, tmp, ggml_nrows(t), t->ne[0], t->data, be->stream);
                } catch (...) {
                    (void) hipFree(tmp);
                    throw;
                }
                e = hipStreamSynchronize(be->stream);
            }
            (void) hipFree(tmp);
            check_hip(e, "tensor_set");
            return;
        }
        check_hip(hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice), "tensor_set");
    });
}

void ggml_backend_tensor_get(const ggml_tensor * t, void * data, size_t offset, size_t size) {
    guarded([&] {
        require(t && data, "tensor_get: NULL tensor or data");
        const ggml_tensor * b = base_of(t);
        require(b->buffer && t->data, "tensor_get: " + tname(t) + " is not in a HIP buffer");
        const size_t nb = ggml_nbytes(t);
        require(offset + size <= nb, "tensor_get: " + std::to_string(offset + size) + " bytes from " + tname(t) +
                                         " of " + std::to_string(nb));
        ggml_backend * be = b->buffer->be;
        set_device(be);
        check_hip(hipStreamSynchronize(be->stream), "tensor_get");
        if (is_packed_type(t->type)) {
            require(t == b && offset == 0 && size == nb,
                    "tensor_get: a " + std::string(ggml_type_name(t->type)) + " tensor is read whole");
            void * tmp = nullptr;
            check_hip(hipMalloc(&tmp, size), "hipMalloc");
            hipError_t e = hipSuccess;
            try {
                launch_unpack(t->type, t->data, ggml_nrows(t), t->ne[0], tmp, be->stream);
            } catch (...) {
                (void) hipFree(tmp);
                throw;
            }
            e = hipStreamSynchronize(be->stream);
            if (e == hipSuccess) e = hipMemcpy(data, tmp, size, hipMemcpyDeviceToHost);
            (void) hipFree(tmp);
            check_hip(e, "tensor_get");
            return;
        }
        check_hip(hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost), "tensor_get");
    });
}

void ggml_backend_tensor_memset(ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    guarded([&] {
        require(t && t->data && base_of(t)->buffer, "tensor_memset: tensor is not in a HIP buffer");
        require(!is_packed_type(t->type), "tensor_memset: not for quantized tensors");
        require(offset + size <= ggml_nbytes(t), "tensor_memset: range exceeds the tensor");
        set_device(base_of(t)->buffer->be);
        check_hip(hipMemset((char *) t->data + offset, value, size), "tensor_memset");
    });
}

void ggml_backend_tensor_copy(ggml_tensor * src, ggml_tensor * dst) {
    guarded([&] {
        require(src && dst && src->data && dst->data && base_of(src)->buffer && base_of(dst)->buffer,
                "tensor_copy: both tensors must be in HIP buffers");
        require(src->type == dst->type && ggml_are_same_shape(src, dst) && ggml_is_contiguous(src) &&
                    ggml_is_contiguous(dst),
                "tensor_copy: same type and shape, both contiguous");
        const size_t n = is_packed_type(src->type) ? alloc_size(src) : ggml_nbytes(src);
        if (is_packed_type(src->type)) require(src == base_of(src) && dst == base_of(dst), "tensor_copy: whole tensors");
        set_device(base_of(dst)->buffer->be);
        check_hip(hipMemcpy(dst->data, src->data, n, hipMemcpyDeviceToDevice), "tensor_copy");
    });
}

enum ggml_status ggml_backend_view_init(ggml_tensor * t) {
    if (!t || !t->view_src || !t->view_src->data) {
        set_error("view_init: not a view of a tensor with memory");
        return GGML_STATUS_FAILED;
    }
    t->data = (char *) t->view_src->data + t->view_offs;
    t->buffer = t->view_src->buffer;
    return GGML_STATUS_SUCCESS;
}

const char * ggml_status_to_string(enum ggml_status status) {
    switch (status) {
        case GGML_STATUS_ALLOC_FAILED: return "GGML status: error (failed to allocate memory)";
        case GGML_STATUS_FAILED: return "GGML status: error (operation failed)";
        case GGML_STATUS_SUCCESS: return "GGML status: success";
        case GGML_STATUS_ABORTED: return "GGML status: warning (operation aborted)";
    }
    return "GGML status: unknown";
}

// ------------------------------------------------------------------------------ ggml-alloc

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    if (!buft) {
        set_error("gallocr_new: buffer type is NULL");
        return nullptr;
    }
    auto * ga = new ggml_gallocr;
    ga->be = buft->be;
    ga->buf.be = buft->be;
    return ga;
}

void ggml_gallocr_free(ggml_gallocr_t ga) {
    if (!ga) return;
    if (ga->buf.base) (void) hipFree(ga->buf.base);
    delete ga;
}

bool ggml_gallocr_reserve(ggml_gallocr_t ga, ggml_cgraph * g) {
    if (!ga || !g) return false;
    return guarded([&] {
               std::vector<std::pair<ggml_tensor *, size_t>> where;
               const size_t need = place(ga, g, where);
               if (need > ga->buf.size) {
                   set_device(ga->be);
                   if (ga->buf.base) check_hip(hipFree(ga->buf.base), "hipFree");
                   ga->buf.base = nullptr;
                   ga->buf.size = 0;
                   check_hip(hipMalloc(&ga->buf.base, need), "hipMalloc compute buffer");
                   ga->buf.size = need;
               }
           }) == 0;
}

bool ggml_gallocr_alloc_graph(ggml_gallocr_t ga, ggml_cgraph * g) {
    if (!ga || !g) return false;
    return guarded([&] {
               std::vector<std::pair<ggml_tensor *, size_t>> where;
               const size_t need = place(ga, g, where);
               if (need > ga->buf.size) {
                   set_device(ga->be);
                   check_hip(hipDeviceSynchronize(), "gallocr");
                   if (ga->buf.base) check_hip(hipFree(ga->buf.base), "hipFree");
                   ga->buf.base = nullptr;
                   ga->buf.size = 0;
                   check_hip(hipMalloc(&ga->buf.base, need), "hipMalloc compute buffer");
                   ga->buf.size = need;
               }
               for (auto & w : where) {
                   w.first->data = (char *) ga->buf.base + w.second;
                   w.first->buffer = &ga->buf;
               }
               refresh_views(g);
           }) == 0;
}

size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t ga, int buffer_id) {
    return ga && buffer_id == 0 ? ga->buf.size : 0;
}

}  // extern "C"
