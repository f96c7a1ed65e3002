// ggml.hip - graph construction of the ggml API subset (include/ggml.h): contexts, tensors, views
// and op nodes, all host-side metadata. The nodes run in ggml_backend.hip.
//
// Shapes, strides and result types follow ggml's rules for each call (innermost-first ne, byte
// strides nb, views sharing their base's memory at view_offs); a call whose operands do not fit
// returns NULL with the reason in ggml_last_error().
#include "gcq_common.h"
#include "ggml_impl.h"

#include <cstdlib>
#include <cstring>

namespace gcq {
namespace {

struct TypeTraits {
    int type;
    const char * name;
    int64_t blck;
    size_t size;
};

// GGUF's block formats: elements per block, bytes per block.
constexpr TypeTraits kTypes[] = {
    {GGML_TYPE_F32, "f32", 1, 4},      {GGML_TYPE_F16, "f16", 1, 2},       {GGML_TYPE_Q4_0, "q4_0", 32, 18},
    {GGML_TYPE_Q4_1, "q4_1", 32, 20},  {GGML_TYPE_Q5_0, "q5_0", 32, 22},   {GGML_TYPE_Q5_1, "q5_1", 32, 24},
    {GGML_TYPE_Q8_0, "q8_0", 32, 34},  {GGML_TYPE_Q8_1, "q8_1", 32, 36},   {GGML_TYPE_Q2_K, "q2_K", 256, 84},
    {GGML_TYPE_Q3_K, "q3_K", 256, 110}, {GGML_TYPE_Q4_K, "q4_K", 256, 144}, {GGML_TYPE_Q5_K, "q5_K", 256, 176},
    {GGML_TYPE_Q6_K, "q6_K", 256, 210}, {GGML_TYPE_Q8_K, "q8_K", 256, 292}, {GGML_TYPE_I8, "i8", 1, 1},
    {GGML_TYPE_I16, "i16", 1, 2},      {GGML_TYPE_I32, "i32", 1, 4},       {GGML_TYPE_I64, "i64", 1, 8},
    {GGML_TYPE_F64, "f64", 1, 8},      {GGML_TYPE_BF16, "bf16", 1, 2},
};

const TypeTraits * traits(int type) {
    for (const auto & t : kTypes)
        if (t.type == type) return &t;
    return nullptr;
}

const char * kOpNames[GGML_OP_COUNT] = {"NONE",    "ADD",      "MUL",      "SCALE",    "CPY",
                                        "CONT",    "RESHAPE",  "VIEW",     "PERMUTE",  "TRANSPOSE",
                                        "GET_ROWS", "SET_ROWS", "RMS_NORM", "MUL_MAT",  "ROPE",
                                        "FLASH_ATTN_EXT", "ARGMAX", "GLU", "UNARY", "SOFT_MAX",
                                        "IM2COL", "CONV_2D_DIRECT", "SUB", "DIV", "NORM", "SUM_ROWS", "MEAN", "REPEAT", "CONCAT"};

// NULL with the reason recorded.
ggml_tensor * none(const std::string & why) {
    set_error(why);
    return nullptr;
}

std::string shape(const ggml_tensor * t) {
    std::string s = "[";
    for (int i = 0; i < 4; i++) s += std::to_string(t->ne[i]) + (i < 3 ? ", " : "]");
    return s;
}

// A new tensor of ctx: contiguous strides; a view of view_src at byte offset view_offs when given
// (resolved to the tensor owning the memory, as ggml does), else its own memory (host memory when
// the context allocates).
ggml_tensor * new_tensor(ggml_context * ctx, int type, int n_dims, const int64_t * ne, ggml_tensor * view_src,
                         size_t view_offs, const char * what) {
    if (!ctx) return none(std::string(what) + ": context is NULL");
    const TypeTraits * tt = traits(type);
    if (!tt) return none(std::string(what) + ": unknown type " + std::to_string(type));
    if (n_dims < 1 || n_dims > GGML_MAX_DIMS) return none(std::string(what) + ": 1 to 4 dims");
    auto * t = new ggml_tensor;
    std::memset(t, 0, sizeof(*t));
    t->type = (ggml_type) type;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = i < n_dims ? ne[i] : 1;
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] < 0) {
            delete t;
            return none(std::string(what) + ": negative size");
        }
    }
    if (t->ne[0] % tt->blck) {
        delete t;
        return none(std::string(what) + ": row of " + std::to_string(t->ne[0]) + " is not a multiple of " + tt->name +
                    "'s block of " + std::to_string(tt->blck));
    }
    t->nb[0] = tt->size;
    t->nb[1] = tt->size * (size_t) (t->ne[0] / tt->blck);
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    if (view_src) {
        if (view_src->view_src) {
            view_offs += view_src->view_offs;
            view_src = view_src->view_src;
        }
        const size_t need = ggml_nbytes(t);
        if (view_offs + need > ggml_nbytes(view_src)) {
            delete t;
            return none(std::string(what) + ": view of " + std::to_string(need) + " bytes at offset " +
                        std::to_string(view_offs) + " exceeds its source's " + std::to_string(ggml_nbytes(view_src)));
        }
        t->view_src = view_src;
        t->view_offs = view_offs;
        t->buffer = view_src->buffer;
        if (view_src->data) t->data = (char *) view_src->data + view_offs;
    } else if (!ctx->no_alloc) {
        const size_t n = ggml_nbytes(t);
        t->data = std::calloc(1, n ? n : 1);
        ctx->host_data.push_back(t->data);
    }
    ctx->tensors.push_back(t);
    return t;
}

ggml_tensor * dup_shape(ggml_context * ctx, const ggml_tensor * a, int type, const char * what) {
    return new_tensor(ctx, type, GGML_MAX_DIMS, a->ne, nullptr, 0, what);
}

void set_src(ggml_tensor * t, int op, std::initializer_list<ggml_tensor *> srcs) {
    t->op = (ggml_op) op;
    int i = 0;
    for (ggml_tensor * s : srcs) t->src[i++] = s;
}

template <class T> void set_param(ggml_tensor * t, int i, T v) {
    static_assert(sizeof(T) == 4, "32-bit parameter");
    std::memcpy(&t->op_params[i], &v, 4);
}

bool is_float(int type) { return type == GGML_TYPE_F32 || type == GGML_TYPE_F16; }

ggml_tensor * view_impl(ggml_context * ctx, ggml_tensor * a, int n_dims, const int64_t * ne, const size_t * nb,
                        size_t offset) {
    if (!a) return nullptr;
    ggml_tensor * t = new_tensor(ctx, a->type, n_dims, ne, a, offset, "ggml_view");
    if (!t) return nullptr;
    for (int i = 1; i < n_dims; i++) t->nb[i] = nb[i];
    for (int i = n_dims; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    if (t->view_offs + ggml_nbytes(t) > ggml_nbytes(t->view_src))
        return none("ggml_view: strided view exceeds its source's bytes");
    set_src(t, GGML_OP_VIEW, {a});
    std::memcpy(t->op_params, &offset, sizeof(offset));
    return t;
}

ggml_tensor * reshape_impl(ggml_context * ctx, ggml_tensor * a, int n_dims, const int64_t * ne) {
    if (!a) return nullptr;
    if (!ggml_is_contiguous(a)) return none("ggml_reshape: the source " + shape(a) + " is not contiguous");
    int64_t n = 1;
    for (int i = 0; i < n_dims; i++) n *= ne[i];
    if (n != ggml_nelements(a))
        return none("ggml_reshape: " + std::to_string(n) + " elements from " + std::to_string(ggml_nelements(a)));
    ggml_tensor * t = new_tensor(ctx, a->type, n_dims, ne, a, 0, "ggml_reshape");
    if (!t) return nullptr;
    set_src(t, GGML_OP_RESHAPE, {a});
    return t;
}

ggml_tensor * binary(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, int op, const char * what) {
    if (!a || !b) return nullptr;
    if (!ggml_can_repeat(b, a)) return none(std::string(what) + ": cannot broadcast " + shape(b) + " into " + shape(a));
    ggml_tensor * t = dup_shape(ctx, a, a->type, what);
    if (!t) return nullptr;
    set_src(t, op, {a, b});
    return t;
}

void visit(ggml_cgraph * g, ggml_tensor * t) {
    if (!t || g->visited.count(t)) return;
    g->visited.insert(t);
    for (int i = 0; i < GGML_MAX_SRC; i++) visit(g, t->src[i]);
    if (t->op == GGML_OP_NONE && !(t->flags & GGML_TENSOR_FLAG_PARAM)) {
        g->leafs.push_back(t);
    } else {
        if (g->nodes.size() >= g->size && g->error.empty())
            g->error = "graph of " + std::to_string(g->size) + " nodes is full (ggml_new_graph_custom)";
        g->nodes.push_back(t);
    }
}

}  // namespace

int64_t ggml_blck(int type) {
    const TypeTraits * t = traits(type);
    return t ? t->blck : 0;
}
size_t ggml_tsize(int type) {
    const TypeTraits * t = traits(type);
    return t ? t->size : 0;
}

}  // namespace gcq

using namespace gcq;

extern "C" {

const char * ggml_last_error(void) { return last_error(); }

// ------------------------------------------------------------------ context, types, shapes

ggml_context * ggml_init(ggml_init_params params) {
    auto * ctx = new ggml_context;
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

void ggml_free(ggml_context * ctx) {
    if (!ctx) return;
    for (ggml_tensor * t : ctx->tensors) delete t;
    for (void * p : ctx->host_data) std::free(p);
    for (ggml_cgraph * g : ctx->graphs) delete g;
    delete ctx;
}

size_t ggml_tensor_overhead(void) { return sizeof(ggml_tensor) + 32; }
size_t ggml_graph_overhead_custom(size_t size, bool) { return sizeof(ggml_cgraph) + 3 * size * sizeof(void *) + 64; }
size_t ggml_graph_overhead(void) { return ggml_graph_overhead_custom(GGML_DEFAULT_GRAPH_SIZE, false); }

size_t ggml_type_size(ggml_type type) { return ggml_tsize(type); }
int64_t ggml_blck_size(ggml_type type) { return ggml_blck(type); }
size_t ggml_row_size(ggml_type type, int64_t ne) {
    const int64_t b = ggml_blck(type);
    return b ? ggml_tsize(type) * (size_t) (ne / b) : 0;
}
const char * ggml_type_name(ggml_type type) {
    const TypeTraits * t = traits(type);
    return t ? t->name : "NONE";
}
bool ggml_is_quantized(ggml_type type) { return ggml_blck(type) > 1; }
const char * ggml_op_name(ggml_op op) { return op >= 0 && op < GGML_OP_COUNT ? kOpNames[op] : "?"; }
const char * ggml_op_desc(const ggml_tensor * t) { return t ? ggml_op_name(t->op) : "?"; }

int64_t ggml_nelements(const ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const ggml_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

// Bytes from the first element to one past the last, as ggml_nbytes.
size_t ggml_nbytes(const ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const int64_t blck = ggml_blck(t->type);
    size_t n;
    if (blck == 1) {
        n = ggml_tsize(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) n += (size_t) (t->ne[i] - 1) * t->nb[i];
    } else {
        n = (size_t) (t->ne[0] / blck) * t->nb[0];
        for (int i = 1; i < GGML_MAX_DIMS; i++) n += (size_t) (t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

// Rows packed one after another; dims of size 1 carry no stride requirement.
bool ggml_is_contiguous(const ggml_tensor * t) {
    size_t next = ggml_tsize(t->type);
    if (t->ne[0] != ggml_blck(t->type) && t->nb[0] != next) return false;
    next *= (size_t) (t->ne[0] / ggml_blck(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] == 1) continue;
        if (t->nb[i] != next) return false;
        next *= (size_t) t->ne[i];
    }
    return true;
}
bool ggml_is_transposed(const ggml_tensor * t) { return t->nb[0] > t->nb[1]; }
bool ggml_is_permuted(const ggml_tensor * t) {
    return t->nb[0] > t->nb[1] || t->nb[1] > t->nb[2] || t->nb[2] > t->nb[3];
}
bool ggml_is_vector(const ggml_tensor * t) { return t->ne[1] == 1 && t->ne[2] == 1 && t->ne[3] == 1; }
bool ggml_is_matrix(const ggml_tensor * t) { return t->ne[2] == 1 && t->ne[3] == 1; }
bool ggml_are_same_shape(const ggml_tensor * a, const ggml_tensor * b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}
// b can be repeated into a: every dim of a is a whole multiple of b's.
bool ggml_can_repeat(const ggml_tensor * b, const ggml_tensor * a) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (b->ne[i] == 0 ? a->ne[i] != 0 : a->ne[i] % b->ne[i] != 0) return false;
    return true;
}

// -------------------------------------------------------------------------------- tensors

ggml_tensor * ggml_new_tensor(ggml_context * ctx, ggml_type type, int n_dims, const int64_t * ne) {
    if (!ne) return none("ggml_new_tensor: ne is NULL");
    return new_tensor(ctx, type, n_dims, ne, nullptr, 0, "ggml_new_tensor");
}
ggml_tensor * ggml_new_tensor_1d(ggml_context * ctx, ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}
ggml_tensor * ggml_new_tensor_2d(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return ggml_new_tensor(ctx, type, 2, ne);
}
ggml_tensor * ggml_new_tensor_3d(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return ggml_new_tensor(ctx, type, 3, ne);
}
ggml_tensor * ggml_new_tensor_4d(ggml_context * ctx, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2,
                                 int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return ggml_new_tensor(ctx, type, 4, ne);
}

ggml_tensor * ggml_set_name(ggml_tensor * t, const char * name) {
    if (!t) return nullptr;
    std::strncpy(t->name, name ? name : "", GGML_MAX_NAME - 1);
    t->name[GGML_MAX_NAME - 1] = 0;
    return t;
}
const char * ggml_get_name(const ggml_tensor * t) { return t ? t->name : nullptr; }
ggml_tensor * ggml_get_tensor(ggml_context * ctx, const char * name) {
    if (!ctx || !name) return nullptr;
    for (ggml_tensor * t : ctx->tensors)
        if (std::strcmp(t->name, name) == 0) return t;
    return nullptr;
}
ggml_tensor * ggml_get_first_tensor(const ggml_context * ctx) {
    return ctx && !ctx->tensors.empty() ? ctx->tensors.front() : nullptr;
}
ggml_tensor * ggml_get_next_tensor(const ggml_context * ctx, ggml_tensor * t) {
    if (!ctx) return nullptr;
    for (size_t i = 0; i + 1 < ctx->tensors.size(); i++)
        if (ctx->tensors[i] == t) return ctx->tensors[i + 1];
    return nullptr;
}
void ggml_set_input(ggml_tensor * t) {
    if (t) t->flags |= GGML_TENSOR_FLAG_INPUT;
}
void ggml_set_output(ggml_tensor * t) {
    if (t) t->flags |= GGML_TENSOR_FLAG_OUTPUT;
}

// ---------------------------------------------------------------------------------- views

ggml_tensor * ggml_view_1d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, size_t offset) {
    const size_t nb[1] = {0};
    return view_impl(ctx, a, 1, &ne0, nb, offset);
}
ggml_tensor * ggml_view_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) {
    const int64_t ne[2] = {ne0, ne1};
    const size_t nb[2] = {0, nb1};
    return view_impl(ctx, a, 2, ne, nb, offset);
}
ggml_tensor * ggml_view_3d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1,
                           size_t nb2, size_t offset) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    const size_t nb[3] = {0, nb1, nb2};
    return view_impl(ctx, a, 3, ne, nb, offset);
}
ggml_tensor * ggml_view_4d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                           size_t nb1, size_t nb2, size_t nb3, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    const size_t nb[4] = {0, nb1, nb2, nb3};
    return view_impl(ctx, a, 4, ne, nb, offset);
}

// Same shape and strides as a, over a's memory (op NONE, as ggml's).
ggml_tensor * ggml_view_tensor(ggml_context * ctx, ggml_tensor * a) {
    if (!a) return nullptr;
    ggml_tensor * t = new_tensor(ctx, a->type, GGML_MAX_DIMS, a->ne, a, 0, "ggml_view_tensor");
    if (!t) return nullptr;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->nb[i] = a->nb[i];
    return t;
}

ggml_tensor * ggml_reshape(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    if (!b) return nullptr;
    return reshape_impl(ctx, a, GGML_MAX_DIMS, b->ne);
}
ggml_tensor * ggml_reshape_1d(ggml_context * ctx, ggml_tensor * a, int64_t ne0) {
    return reshape_impl(ctx, a, 1, &ne0);
}
ggml_tensor * ggml_reshape_2d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return reshape_impl(ctx, a, 2, ne);
}
ggml_tensor * ggml_reshape_3d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return reshape_impl(ctx, a, 3, ne);
}
ggml_tensor * ggml_reshape_4d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2,
                              int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return reshape_impl(ctx, a, 4, ne);
}

ggml_tensor * ggml_permute(ggml_context * ctx, ggml_tensor * a, int axis0, int axis1, int axis2, int axis3) {
    if (!a) return nullptr;
    const int ax[4] = {axis0, axis1, axis2, axis3};
    bool seen[4] = {false, false, false, false};
    for (int i = 0; i < 4; i++) {
        if (ax[i] < 0 || ax[i] > 3 || seen[ax[i]]) return none("ggml_permute: axes must be a permutation of 0..3");
        seen[ax[i]] = true;
    }
    ggml_tensor * t = ggml_view_tensor(ctx, a);
    if (!t) return nullptr;
    for (int i = 0; i < 4; i++) {
        t->ne[ax[i]] = a->ne[i];
        t->nb[ax[i]] = a->nb[i];
    }
    set_src(t, GGML_OP_PERMUTE, {a});
    for (int i = 0; i < 4; i++) t->op_params[i] = ax[i];
    return t;
}

ggml_tensor * ggml_transpose(ggml_context * ctx, ggml_tensor * a) {
    ggml_tensor * t = ggml_permute(ctx, a, 1, 0, 2, 3);
    if (t) t->op = GGML_OP_TRANSPOSE;
    return t;
}

// ------------------------------------------------------------------------------------ ops

ggml_tensor * ggml_cont(ggml_context * ctx, ggml_tensor * a) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_cont");
    if (!t) return nullptr;
    set_src(t, GGML_OP_CONT, {a});
    return t;
}

// a's elements, in a's row-major order, into b's (the result is a view of b).
ggml_tensor * ggml_cpy(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    if (!a || !b) return nullptr;
    if (ggml_nelements(a) != ggml_nelements(b))
        return none("ggml_cpy: " + std::to_string(ggml_nelements(a)) + " elements into " +
                    std::to_string(ggml_nelements(b)));
    ggml_tensor * t = ggml_view_tensor(ctx, b);
    if (!t) return nullptr;
    set_src(t, GGML_OP_CPY, {a, b});
    return t;
}

ggml_tensor * ggml_cast(ggml_context * ctx, ggml_tensor * a, ggml_type type) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, type, "ggml_cast");
    if (!t) return nullptr;
    set_src(t, GGML_OP_CPY, {a});
    return t;
}

ggml_tensor * ggml_add(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_ADD, "ggml_add");
}
ggml_tensor * ggml_mul(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_MUL, "ggml_mul");
}
ggml_tensor * ggml_sub(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_SUB, "ggml_sub");
}
ggml_tensor * ggml_div(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    return binary(ctx, a, b, GGML_OP_DIV, "ggml_div");
}

ggml_tensor * ggml_scale_bias(ggml_context * ctx, ggml_tensor * a, float s, float b) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_scale");
    if (!t) return nullptr;
    set_src(t, GGML_OP_SCALE, {a});
    set_param(t, 0, s);
    set_param(t, 1, b);
    return t;
}
ggml_tensor * ggml_scale(ggml_context * ctx, ggml_tensor * a, float s) { return ggml_scale_bias(ctx, a, s, 0.0f); }

ggml_tensor * ggml_mul_mat(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    if (!a || !b) return nullptr;
    if (a->ne[0] != b->ne[0] || b->ne[2] % a->ne[2] || b->ne[3] % a->ne[3])
        return none("ggml_mul_mat: cannot multiply " + shape(a) + " by " + shape(b));
    if (ggml_is_transposed(a)) return none("ggml_mul_mat: the weight operand is transposed");
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor * t = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0, "ggml_mul_mat");
    if (!t) return nullptr;
    set_src(t, GGML_OP_MUL_MAT, {a, b});
    return t;
}

// Precision lives in op_params[0] of a mul_mat and op_params[3] of a flash_attn_ext (after its
// three float parameters).
void ggml_prec_set_acc(ggml_tensor * t, ggml_prec prec) {
    if (!t) return;
    if (t->op == GGML_OP_MUL_MAT) t->op_params[0] = prec;
    else if (t->op == GGML_OP_FLASH_ATTN_EXT) t->op_params[3] = prec;
}
void ggml_mul_mat_set_prec(ggml_tensor * a, ggml_prec prec) { ggml_prec_set_acc(a, prec); }
void ggml_flash_attn_ext_set_prec(ggml_tensor * a, ggml_prec prec) { ggml_prec_set_acc(a, prec); }

ggml_tensor * ggml_rms_norm(ggml_context * ctx, ggml_tensor * a, float eps) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_rms_norm");
    if (!t) return nullptr;
    set_src(t, GGML_OP_RMS_NORM, {a});
    set_param(t, 0, eps);
    return t;
}

// op_params: [1] n_dims, [2] mode, [4] n_ctx_orig, then f32 [5] freq_base, [6] freq_scale,
// [7] ext_factor, [8] attn_factor, [9] beta_fast, [10] beta_slow.
ggml_tensor * ggml_rope_ext(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_tensor * c, int n_dims,
                            int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                            float attn_factor, float beta_fast, float beta_slow) {
    if (!a || !b) return nullptr;
    if (b->type != GGML_TYPE_I32 || !ggml_is_vector(b) || b->ne[0] != a->ne[2])
        return none("ggml_rope_ext: positions must be i32 [" + std::to_string(a->ne[2]) + "], got " + shape(b));
    if (c && (c->type != GGML_TYPE_F32 || c->ne[0] < n_dims / 2))
        return none("ggml_rope_ext: frequency factors must be f32 with n_dims/2 values");
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_rope_ext");
    if (!t) return nullptr;
    set_src(t, GGML_OP_ROPE, {a, b, c});
    t->op_params[1] = n_dims;
    t->op_params[2] = mode;
    t->op_params[4] = n_ctx_orig;
    set_param(t, 5, freq_base);
    set_param(t, 6, freq_scale);
    set_param(t, 7, ext_factor);
    set_param(t, 8, attn_factor);
    set_param(t, 9, beta_fast);
    set_param(t, 10, beta_slow);
    return t;
}

ggml_tensor * ggml_get_rows(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    if (!a || !b) return nullptr;
    if (b->type != GGML_TYPE_I32 || a->ne[2] != b->ne[1] || b->ne[3] != 1)
        return none("ggml_get_rows: rows " + shape(b) + " (i32) of " + shape(a));
    const int64_t ne[4] = {a->ne[0], b->ne[0], b->ne[1], b->ne[2]};
    ggml_tensor * t = new_tensor(ctx, a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32, 4, ne, nullptr, 0,
                                 "ggml_get_rows");
    if (!t) return nullptr;
    set_src(t, GGML_OP_GET_ROWS, {a, b});
    return t;
}

// The written rows' destination a is also src[2], so that a graph orders the write after a's
// producers and counts it among a's readers.
ggml_tensor * ggml_set_rows(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, ggml_tensor * c) {
    if (!a || !b || !c) return nullptr;
    if (a->ne[0] != b->ne[0] || a->ne[2] != b->ne[2] || a->ne[3] != b->ne[3] || c->ne[0] != b->ne[1] ||
        (c->type != GGML_TYPE_I32 && c->type != GGML_TYPE_I64) || !is_float(b->type))
        return none("ggml_set_rows: cannot write rows " + shape(b) + " at indices " + shape(c) + " into " + shape(a));
    ggml_tensor * t = ggml_view_tensor(ctx, a);
    if (!t) return nullptr;
    set_src(t, GGML_OP_SET_ROWS, {b, c, a});
    return t;
}

// op_params f32 [0] scale, [1] max_bias, [2] logit_softcap, i32 [3] precision.
ggml_tensor * ggml_flash_attn_ext(ggml_context * ctx, ggml_tensor * q, ggml_tensor * k, ggml_tensor * v,
                                  ggml_tensor * mask, float scale, float max_bias, float logit_softcap) {
    if (!q || !k || !v) return nullptr;
    if (k->ne[0] != q->ne[0] || v->ne[1] != k->ne[1] || k->ne[2] != v->ne[2] || k->ne[2] == 0 ||
        q->ne[2] % k->ne[2] || q->ne[3] != k->ne[3])
        return none("ggml_flash_attn_ext: q " + shape(q) + ", k " + shape(k) + ", v " + shape(v) + " do not fit");
    if (mask && (mask->ne[0] != k->ne[1] || mask->ne[1] < q->ne[1]))
        return none("ggml_flash_attn_ext: mask " + shape(mask) + " must be [n_kv, >= n_queries]");
    const int64_t ne[4] = {v->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    ggml_tensor * t = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0, "ggml_flash_attn_ext");
    if (!t) return nullptr;
    set_src(t, GGML_OP_FLASH_ATTN_EXT, {q, k, v, mask});
    set_param(t, 0, scale);
    set_param(t, 1, max_bias);
    set_param(t, 2, logit_softcap);
    t->op_params[3] = GGML_PREC_DEFAULT;
    return t;
}

// op_params [0] the gated unit (SWIGLU), [1] swapped (0).
ggml_tensor * ggml_swiglu_split(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b) {
    if (!a || !b) return nullptr;
    if (!ggml_are_same_shape(a, b) || a->type != b->type)
        return none("ggml_swiglu_split: gate " + shape(a) + " and up " + shape(b) + " differ");
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_swiglu_split");
    if (!t) return nullptr;
    set_src(t, GGML_OP_GLU, {a, b});
    t->op_params[0] = GGML_GLU_OP_SWIGLU;
    t->op_params[1] = 0;
    return t;
}

ggml_tensor * ggml_argmax(ggml_context * ctx, ggml_tensor * a) {
    if (!a) return nullptr;
    if (!ggml_is_matrix(a)) return none("ggml_argmax: needs a matrix, got " + shape(a));
    ggml_tensor * t = new_tensor(ctx, GGML_TYPE_I32, 1, &a->ne[1], nullptr, 0, "ggml_argmax");
    if (!t) return nullptr;
    set_src(t, GGML_OP_ARGMAX, {a});
    return t;
}

// ------------------------------------------------ elementwise, softmax and off-path constructors

namespace {
ggml_tensor * unary(ggml_context * ctx, ggml_tensor * a, int uop, const char * what) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, what);
    if (!t) return nullptr;
    set_src(t, GGML_OP_UNARY, {a});
    t->op_params[0] = uop;
    return t;
}
int64_t conv_out(int64_t in, int64_t k, int s, int p, int d) { return (in + 2 * p - d * (k - 1) - 1) / s + 1; }
}  // namespace

ggml_tensor * ggml_gelu(ggml_context * ctx, ggml_tensor * a) { return unary(ctx, a, GGML_UNARY_OP_GELU, "ggml_gelu"); }
ggml_tensor * ggml_tanh(ggml_context * ctx, ggml_tensor * a) { return unary(ctx, a, GGML_UNARY_OP_TANH, "ggml_tanh"); }
ggml_tensor * ggml_sqr(ggml_context * ctx, ggml_tensor * a) { return unary(ctx, a, GGML_UNARY_OP_SQR, "ggml_sqr"); }
ggml_tensor * ggml_gelu_erf(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_GELU_ERF, "ggml_gelu_erf");
}
ggml_tensor * ggml_silu(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_SILU, "ggml_silu");
}
ggml_tensor * ggml_relu(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_RELU, "ggml_relu");
}
ggml_tensor * ggml_sigmoid(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_SIGMOID, "ggml_sigmoid");
}
ggml_tensor * ggml_exp(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_EXP, "ggml_exp");
}
ggml_tensor * ggml_log(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_LOG, "ggml_log");
}
ggml_tensor * ggml_neg(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_NEG, "ggml_neg");
}
ggml_tensor * ggml_abs(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_ABS, "ggml_abs");
}
ggml_tensor * ggml_sqrt(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_SQRT, "ggml_sqrt");
}
ggml_tensor * ggml_sin(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_SIN, "ggml_sin");
}
ggml_tensor * ggml_cos(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_COS, "ggml_cos");
}
ggml_tensor * ggml_softplus(ggml_context * ctx, ggml_tensor * a) {
    return unary(ctx, a, GGML_UNARY_OP_SOFTPLUS, "ggml_softplus");
}

ggml_tensor * ggml_clamp(ggml_context * ctx, ggml_tensor * a, float min, float max) {
    ggml_tensor * t = unary(ctx, a, GGML_UNARY_OP_CLAMP, "ggml_clamp");
    if (!t) return nullptr;
    set_param(t, 1, min);
    set_param(t, 2, max);
    return t;
}

ggml_tensor * ggml_norm(ggml_context * ctx, ggml_tensor * a, float eps) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_norm");
    if (!t) return nullptr;
    set_src(t, GGML_OP_NORM, {a});
    set_param(t, 0, eps);
    return t;
}

namespace {
ggml_tensor * row_reduce(ggml_context * ctx, ggml_tensor * a, ggml_op op, const char * what) {
    if (!a) return nullptr;
    if (a->type != GGML_TYPE_F32) return none(std::string(what) + ": needs an f32 tensor");
    const int64_t ne[4] = {1, a->ne[1], a->ne[2], a->ne[3]};
    ggml_tensor * t = new_tensor(ctx, GGML_TYPE_F32, 4, ne, nullptr, 0, what);
    if (!t) return nullptr;
    set_src(t, op, {a});
    return t;
}
}  // namespace

ggml_tensor * ggml_repeat_4d(ggml_context * ctx, ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    if (!a) return nullptr;
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    for (int k = 0; k < 4; k++)
        if (ne[k] <= 0 || a->ne[k] <= 0 || ne[k] % a->ne[k] != 0)
            return none("ggml_repeat_4d: cannot tile " + shape(a) + " to a shape that is not a multiple of it");
    ggml_tensor * t = new_tensor(ctx, a->type, 4, ne, nullptr, 0, "ggml_repeat_4d");
    if (!t) return nullptr;
    set_src(t, GGML_OP_REPEAT, {a});
    return t;
}

ggml_tensor * ggml_concat(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, int dim) {
    if (!a || !b) return nullptr;
    if (dim < 0 || dim > 3 || a->type != b->type) return none("ggml_concat: dim 0-3 and one type");
    int64_t ne[4];
    for (int k = 0; k < 4; k++) {
        if (k != dim && a->ne[k] != b->ne[k])
            return none("ggml_concat: " + shape(a) + " and " + shape(b) + " differ outside dim " + std::to_string(dim));
        ne[k] = k == dim ? a->ne[k] + b->ne[k] : a->ne[k];
    }
    ggml_tensor * t = new_tensor(ctx, a->type, 4, ne, nullptr, 0, "ggml_concat");
    if (!t) return nullptr;
    set_src(t, GGML_OP_CONCAT, {a, b});
    t->op_params[0] = dim;
    return t;
}

ggml_tensor * ggml_sum_rows(ggml_context * ctx, ggml_tensor * a) { return row_reduce(ctx, a, GGML_OP_SUM_ROWS, "ggml_sum_rows"); }
ggml_tensor * ggml_mean(ggml_context * ctx, ggml_tensor * a) { return row_reduce(ctx, a, GGML_OP_MEAN, "ggml_mean"); }

ggml_tensor * ggml_soft_max_ext(ggml_context * ctx, ggml_tensor * a, ggml_tensor * mask, float scale,
                                float max_bias) {
    if (!a) return nullptr;
    ggml_tensor * t = dup_shape(ctx, a, a->type, "ggml_soft_max_ext");
    if (!t) return nullptr;
    set_src(t, GGML_OP_SOFT_MAX, {a, mask});
    set_param(t, 0, scale);
    set_param(t, 1, max_bias);
    return t;
}

ggml_tensor * ggml_im2col(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, int s0, int s1, int p0, int p1,
                          int d0, int d1, bool is_2D, ggml_type dst_type) {
    if (!a || !b) return nullptr;
    if (!is_2D) return none("ggml_im2col: only the 2-D form is declared here");
    if (s0 <= 0 || s1 <= 0 || d0 <= 0 || d1 <= 0 || a->ne[2] != b->ne[2]) return none("ggml_im2col: bad operands");
    const int64_t ne[4] = {a->ne[0] * a->ne[1] * a->ne[2], conv_out(b->ne[0], a->ne[0], s0, p0, d0),
                           conv_out(b->ne[1], a->ne[1], s1, p1, d1), b->ne[3]};
    ggml_tensor * t = new_tensor(ctx, dst_type, 4, ne, nullptr, 0, "ggml_im2col");
    if (!t) return nullptr;
    set_src(t, GGML_OP_IM2COL, {a, b});
    return t;
}

ggml_tensor * ggml_conv_2d_direct(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, int s0, int s1, int p0,
                                  int p1, int d0, int d1) {
    if (!a || !b) return nullptr;
    if (s0 <= 0 || s1 <= 0 || d0 <= 0 || d1 <= 0 || a->ne[2] != b->ne[2])
        return none("ggml_conv_2d_direct: bad operands");
    const int64_t ne[4] = {conv_out(b->ne[0], a->ne[0], s0, p0, d0), conv_out(b->ne[1], a->ne[1], s1, p1, d1),
                           a->ne[3], b->ne[3]};
    ggml_tensor * t = new_tensor(ctx, b->type, 4, ne, nullptr, 0, "ggml_conv_2d_direct");
    if (!t) return nullptr;
    set_src(t, GGML_OP_CONV_2D_DIRECT, {a, b});
    return t;
}

// --------------------------------------------------------------------------------- graphs

ggml_cgraph * ggml_new_graph_custom(ggml_context * ctx, size_t size, bool) {
    if (!ctx) {
        set_error("ggml_new_graph: context is NULL");
        return nullptr;
    }
    auto * g = new ggml_cgraph;
    g->size = size;
    ctx->graphs.push_back(g);
    return g;
}
ggml_cgraph * ggml_new_graph(ggml_context * ctx) { return ggml_new_graph_custom(ctx, GGML_DEFAULT_GRAPH_SIZE, false); }

void ggml_build_forward_expand(ggml_cgraph * g, ggml_tensor * t) {
    if (!g) return;
    if (!t) {
        if (g->error.empty()) g->error = std::string("a NULL tensor was added to the graph: ") + last_error();
        return;
    }
    visit(g, t);
}

int ggml_graph_n_nodes(ggml_cgraph * g) { return g ? (int) g->nodes.size() : 0; }
ggml_tensor * ggml_graph_node(ggml_cgraph * g, int i) {
    if (!g) return nullptr;
    const int n = (int) g->nodes.size();
    if (i < 0) i += n;
    return i >= 0 && i < n ? g->nodes[i] : nullptr;
}
void ggml_graph_add_node(ggml_cgraph * g, ggml_tensor * t) {
    if (!g || !t) return;
    if (g->nodes.size() >= g->size && g->error.empty()) g->error = "graph is full";
    g->nodes.push_back(t);
    g->visited.insert(t);
}
void ggml_graph_clear(ggml_cgraph * g) {
    if (!g) return;
    g->nodes.clear();
    g->leafs.clear();
    g->visited.clear();
    g->error.clear();
}

}  // extern "C"
