// capi.hip - the C ABI of libgcq (include/gcq.h) and the subset of ggml-compiler's runtime API that
// needs no program loader (include/ggml_compiler_rt.h). Every entry point validates its arguments
// on the host before anything is launched, then calls one of the launchers in the kernel files.
#include "gcq_common.h"

#include <cmath>
#include <cstring>
#include <mutex>

#include "../../include/gcq.h"
#include "../../include/ggml_compiler_rt.h"

namespace gcq {

// Launchers (kernel translation units).
void launch_encode(int type, const float * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_pack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_dequant(int type, const void * w, int64_t nrows, int64_t k, float * y, hipStream_t s);
void launch_act_quant(int wtype, const float * x, int64_t ldx, int64_t B, int64_t k, void * act, hipStream_t s);
void launch_act_to_ggml(int wtype, const void * act, int64_t B, int64_t k, void * out, hipStream_t s);
bool gemv_row_kq_fits(int type, int64_t N, int64_t K);
void launch_gemv_row_kq(int type, const void * w, int64_t N, int64_t K, const float * x, float * y, hipStream_t s);
bool row_gemv_kq_fits(int type, int64_t N, int64_t K);
bool row_gemv_kq_norm_fits(int type, int64_t N, int64_t K);
void launch_row_gemv_kq(int type, const void * w, int64_t N, int64_t K, const float * x, const float * norm_w, float eps,
                        float * y, const float * res, hipStream_t s);
void launch_gemv(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t B, float * y, int64_t ldy,
                 hipStream_t s, const float * res = nullptr);
void launch_isums(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t B, int32_t * out,
                  hipStream_t s);
void launch_gemm(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                 hipStream_t s, const float * res = nullptr);
void launch_gemm_block_isums(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, int blk,
                             int32_t * out, hipStream_t s);
bool gemm_kq_fits(int type, int64_t K);
void launch_gemm_kq(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                    hipStream_t s, const float * res = nullptr);
void launch_gemm_kq_isums(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, int sb,
                          int32_t * out, hipStream_t s);
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
void launch_argmax(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, hipStream_t s);
void launch_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev, hipStream_t s);
void launch_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab, hipStream_t s);

// ------------------------------------------------------------------------ errors, sizes

namespace {
thread_local std::string g_error;
thread_local uint64_t g_errors = 0;
}

void set_error(const std::string & msg) {
    g_error = msg;
    g_errors++;
}
uint64_t error_count() { return g_errors; }
const char * last_error() { return g_error.c_str(); }

void check_hip(hipError_t e, const char * what) {
    if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

void check_launch(const char * what) { check_hip(hipGetLastError(), what); }

size_t block_elems(int type) {
    switch (type) {
        case T_F32: case T_F16: case T_I32: return 1;
        case T_Q4_0: case T_Q8_0: return QK;
        case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_Q8_K: return QKK;
        default: return 0;
    }
}

size_t block_bytes(int type) {
    switch (type) {
        case T_F32: case T_I32: return 4;
        case T_F16: return 2;
        case T_Q4_0: return 18;
        case T_Q8_0: return 34;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        case T_Q8_K: return 292;
        default: return 0;
    }
}

size_t row_bytes(int type, int64_t n) {
    const size_t be = block_elems(type);
    if (!be || n < 0 || n % (int64_t) be) return 0;
    return block_bytes(type) * (size_t) (n / (int64_t) be);
}

WeightLayout weight_layout(int type, int64_t nrows, int64_t k) {
    WeightLayout L;
    if (type == T_Q4_0 || type == T_Q8_0) {
        const size_t nb = (size_t) nrows * (size_t) (k / QK);
        L.qs = 0;
        L.d = align256(nb * (type == T_Q4_0 ? 16 : 32));
        L.total = L.d + align256(nb * 2);
    } else if (type == T_Q6_K) {
        const Q6Regions R = q6_regions(nrows * (k / QKK));
        L.qs = R.ql;
        L.qh = R.qh;
        L.sc = R.sc;
        L.d = R.d;
        L.total = R.total;
    } else if (type == T_Q4_K || type == T_Q5_K) {
        const KqRegions R = kq_regions(type, nrows * (k / QKK));
        L.qs = R.qs;
        L.qh = R.qh;
        L.d = R.hdr;
        L.total = R.total;
    } else {
        L.total = align256(row_bytes(type, k) * (size_t) nrows);
    }
    return L;
}

ActLayout act_layout(int wtype, int64_t B, int64_t k) {
    ActLayout L;
    L.codes = 0;
    L.meta = align256((size_t) B * (size_t) k);
    if (is_kquant(wtype)) {
        L.d = L.meta + align256((size_t) B * (size_t) (k / 16) * 2);
        L.total = L.d + align256((size_t) B * (size_t) (k / QKK) * 4);
    } else {
        L.d = L.meta;
        L.total = L.meta + align256((size_t) B * (size_t) (k / QK) * 8);
    }
    return L;
}

// ------------------------------------------------------------------------------ checks

namespace {

bool is_weight_type(int t) { return t == T_Q4_0 || t == T_Q8_0 || is_kquant(t); }

void need_weight_type(int t) {
    require(is_weight_type(t),
            "unsupported weight type " + std::to_string(t) + " (Q4_0=2, Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14)");
}

void need_k(int t, int64_t k) {
    const int64_t be = (int64_t) block_elems(t);
    require(k > 0 && be > 0 && k % be == 0,
            "row length " + std::to_string(k) + " is not a positive multiple of the type's block size " +
                std::to_string(be));
}

void need_ptr(const void * p, const char * what, size_t align = 1) {
    require(p != nullptr, std::string(what) + " is NULL");
    require(aligned(p, align), std::string(what) + " must be " + std::to_string(align) + "-byte aligned");
}

// The decode-row GEMV's arguments for a packed weight w [N][K] and an f32 row x.
RowArgs row_args(int wtype, const void * w, int64_t N, int64_t K, const float * x) {
    const WeightLayout L = weight_layout(wtype, N, K);
    RowArgs a{};
    a.wqs = (const uint8_t *) w + L.qs;
    a.wd = (const uint16_t *) ((const uint8_t *) w + L.d);
    a.N = (int) N;
    a.nb = (int) (K / QK);
    a.x = x;
    return a;
}

void need_dims(int64_t v, const char * what, int64_t lo = 1, int64_t hi = INT32_MAX) {
    require(v >= lo && v <= hi, std::string(what) + " = " + std::to_string(v) + " out of range [" +
                                    std::to_string(lo) + ", " + std::to_string(hi) + "]");
}

}  // namespace

// ggml_mul_mat(W, x) with the caller's workspace for the quantized activation (gcq_mul_mat and
// gcq_mul_mat_noalloc): checks every argument, then launches on s. One row is quantized inside the
// decode-row GEMV; up to 8 rows go through the workspace into the multi-row GEMV; more rows into
// the int8 MFMA GEMM (Q4_0 / Q8_0) or, for the K-quants, the GEMV in groups of 8 rows.
void mul_mat_with_workspace(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx, int64_t M,
                            float * y, int64_t ldy, void * ws, size_t ws_size, hipStream_t s) {
    need_weight_type(wtype);
    need_k(wtype, K);
    need_dims(N, "N");
    need_dims(M, "M");
    require(ldy >= N, "ldy must be >= N");
    require(ldx >= K && ldx % 4 == 0, "ldx must be >= K and a multiple of 4");
    need_ptr(w, "w", 16);
    need_ptr(x, "x", 16);
    need_ptr(y, "y", 4);
    need_ptr(ws, "workspace", 256);
    const size_t need = mul_mat_workspace_bytes(wtype, M, K);
    require(ws_size >= need, "workspace of " + std::to_string(ws_size) + " bytes, need " + std::to_string(need));
    if (M == 1 && row_gemv_fits(wtype, K)) {
        RowArgs a = row_args(wtype, w, N, K, x);
        a.y = y;
        launch_row_gemv(wtype, PRO_PLAIN, EPI_STORE, a, s);
        return;
    }
    if (M == 1 && row_gemv_kq_fits(wtype, N, K)) return launch_row_gemv_kq(wtype, w, N, K, x, nullptr, 0.0f, y, nullptr, s);
    if (M == 1 && gemv_row_kq_fits(wtype, N, K)) return launch_gemv_row_kq(wtype, w, N, K, x, y, s);
    if (M <= 8) {
        launch_act_quant(wtype, x, ldx, M, K, ws, s);
        launch_gemv(wtype, w, N, K, ws, M, y, ldy, s);
    } else {
        launch_act_quant(wtype, x, ldx, M, K, ws, s);
        if (is_kquant(wtype)) launch_gemm_kq(wtype, w, N, K, ws, M, y, ldy, s);
        else launch_gemm(wtype, w, N, K, ws, M, y, ldy, s);
    }
}

// Workspace bytes of mul_mat_with_workspace (0 for arguments gcq_act_size rejects).
size_t mul_mat_workspace_bytes(int wtype, int64_t M, int64_t K) {
    if (!is_weight_type(wtype) || M <= 0 || !row_bytes(wtype, K)) return 0;
    return act_layout(wtype, M, K).total;
}

}  // namespace gcq

using namespace gcq;

// ----------------------------------------------------------------------------- C ABI

extern "C" {

const char * gcq_version(void) { return "libgcq 0.1 (gfx950 HIP)"; }

const char * gcq_last_error(void) { return last_error(); }

uint64_t gcq_error_count(void) { return error_count(); }

int gcq_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void) hipGetLastError();
        return 0;
    }
    return n;
}

size_t gcq_row_size(int type, int64_t n) {
    const size_t r = row_bytes(type, n);
    if (!r) set_error("row_size: unknown type or n not a multiple of the block size");
    return r;
}

size_t gcq_weight_size(int type, int64_t nrows, int64_t n_per_row) {
    if (!is_weight_type(type) || nrows <= 0 || !row_bytes(type, n_per_row)) {
        set_error("weight_size: bad type or shape");
        return 0;
    }
    return weight_layout(type, nrows, n_per_row).total;
}

size_t gcq_act_size(int wtype, int64_t B, int64_t K) {
    if (!is_weight_type(wtype) || B <= 0 || !row_bytes(wtype, K)) {
        set_error("act_size: bad type or shape");
        return 0;
    }
    return act_layout(wtype, B, K).total;
}

size_t gcq_mul_mat_workspace(int wtype, int64_t M, int64_t K) {
    return gcq_act_size(wtype, M, K);
}

size_t gcq_flash_attn_workspace(int Sq, int H, int Hkv, int Dv, int n_kv) {
    if (Sq <= 0 || H <= 0 || Hkv <= 0 || Dv <= 0 || n_kv <= 0) {
        set_error("flash_attn_workspace: bad shape");
        return 0;
    }
    return attn_workspace(Sq, H, Hkv, Dv, n_kv);
}

int gcq_quantize(int type, const float * src, int64_t nrows, int64_t n_per_row, void * dst, void * stream) {
    return guarded([&] {
        need_weight_type(type);
        need_k(type, n_per_row);
        need_dims(nrows, "nrows", 0, INT64_MAX / 4);
        if (nrows == 0) return;
        need_ptr(src, "src");
        need_ptr(dst, "dst");
        launch_encode(type, src, nrows, n_per_row, dst, as_stream(stream));
    });
}

int gcq_pack_weights(int type, const void * src, int64_t nrows, int64_t n_per_row, void * dst, void * stream) {
    return guarded([&] {
        need_weight_type(type);
        need_k(type, n_per_row);
        need_dims(nrows, "nrows", 1, INT32_MAX);
        need_ptr(src, "src", type == T_Q4_K || type == T_Q5_K ? 16 : 1);  // K-quants move 16-byte pieces
        need_ptr(dst, "dst", 16);
        launch_pack(type, src, nrows, n_per_row, dst, as_stream(stream));
    });
}

int gcq_dequantize(int type, const void * w, int64_t nrows, int64_t n_per_row, float * dst, void * stream) {
    return guarded([&] {
        need_weight_type(type);
        need_k(type, n_per_row);
        need_dims(nrows, "nrows", 1, INT32_MAX);
        need_ptr(w, "w", 16);
        need_ptr(dst, "dst", 4);
        launch_dequant(type, w, nrows, n_per_row, dst, as_stream(stream));
    });
}

int gcq_quantize_act(int wtype, const float * x, int64_t ldx, int64_t B, int64_t K, void * act, void * stream) {
    return guarded([&] {
        need_weight_type(wtype);
        need_k(wtype, K);
        need_dims(B, "B", 1, INT32_MAX);
        require(ldx >= K && ldx % 4 == 0, "ldx must be >= K and a multiple of 4");
        need_ptr(x, "x", 16);
        need_ptr(act, "act", 256);
        launch_act_quant(wtype, x, ldx, B, K, act, as_stream(stream));
    });
}

int gcq_act_to_ggml(int wtype, const void * act, int64_t B, int64_t K, void * dst, void * stream) {
    return guarded([&] {
        need_weight_type(wtype);
        need_k(wtype, K);
        need_dims(B, "B", 1, INT32_MAX);
        need_ptr(act, "act", 256);
        need_ptr(dst, "dst", 4);
        launch_act_to_ggml(wtype, act, B, K, dst, as_stream(stream));
    });
}

int gcq_mul_mat_q(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                  const float * res, void * stream) {
    return guarded([&] {
        need_weight_type(wtype);
        need_k(wtype, K);
        need_dims(N, "N");
        need_dims(M, "M");
        require(ldy >= N, "ldy must be >= N");
        need_ptr(w, "w", 16);
        need_ptr(act, "act", 256);
        need_ptr(y, "y", 4);
        if (res) need_ptr(res, "res", 4);
        if (M <= 8) {
            launch_gemv(wtype, w, N, K, act, M, y, ldy, as_stream(stream), res);
        } else if (is_kquant(wtype)) {
            launch_gemm_kq(wtype, w, N, K, act, M, y, ldy, as_stream(stream), res);
        } else {
            launch_gemm(wtype, w, N, K, act, M, y, ldy, as_stream(stream), res);
        }
    });
}

int gcq_mul_mat(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx, int64_t M, float * y,
                int64_t ldy, void * ws, size_t ws_size, void * stream) {
    return guarded([&] { mul_mat_with_workspace(wtype, w, N, K, x, ldx, M, y, ldy, ws, ws_size, as_stream(stream)); });
}

int gcq_rms_norm_mul_mat(int wtype, const void * w, int64_t N, int64_t K, const float * x, const float * norm_w,
                         float eps, float * y, const float * res, void * ws, size_t ws_size, void * stream) {
    return guarded([&] {
        require(wtype == T_Q4_0 || wtype == T_Q8_0, "rms_norm_mul_mat: weight type must be Q4_0 or Q8_0");
        need_k(wtype, K);
        need_dims(N, "N");
        need_ptr(w, "w", 16);
        need_ptr(x, "x", 16);
        if (norm_w) need_ptr(norm_w, "norm_w", 16);
        need_ptr(y, "y", 4);
        if (res) need_ptr(res, "res", 4);
        hipStream_t s = as_stream(stream);
        if (row_gemv_fits(wtype, K)) {
            RowArgs a = row_args(wtype, w, N, K, x);
            a.norm_w = norm_w;
            a.eps = eps;
            a.y = y;
            a.res = res;
            return launch_row_gemv(wtype, norm_w ? PRO_NORM : PRO_PLAIN, EPI_STORE, a, s);
        }
        need_ptr(ws, "workspace", 256);
        const size_t need = gcq_mul_mat_workspace(wtype, 1, K);
        require(ws_size >= need, "workspace of " + std::to_string(ws_size) + " bytes, need " + std::to_string(need));
        if (norm_w) launch_rmsnorm_q8(x, K, norm_w, eps, 1, K, ws, s);
        else launch_act_quant(wtype, x, K, 1, K, ws, s);
        launch_gemv(wtype, w, N, K, ws, 1, y, N, s, res);
    });
}

int gcq_block_isums(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t B, int32_t * out,
                    void * stream) {
    return guarded([&] {
        need_weight_type(wtype);
        need_k(wtype, K);
        need_dims(N, "N");
        need_dims(B, "B", 1, 8);
        need_ptr(w, "w", 16);
        need_ptr(act, "act", 256);
        need_ptr(out, "out", 4);
        launch_isums(wtype, w, N, K, act, B, out, as_stream(stream));
    });
}

int gcq_gemm_block_isums(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, int blk,
                         int32_t * out, void * stream) {
    return guarded([&] {
        need_weight_type(wtype);
        need_k(wtype, K);
        need_dims(N, "N");
        need_dims(M, "M");
        need_dims(blk, "blk", 0, K / block_elems(wtype) - 1);
        need_ptr(w, "w", 16);
        need_ptr(act, "act", 256);
        need_ptr(out, "out", 4);
        if (is_kquant(wtype)) launch_gemm_kq_isums(wtype, w, N, K, act, M, blk, out, as_stream(stream));
        else launch_gemm_block_isums(wtype, w, N, K, act, M, blk, out, as_stream(stream));
    });
}

int gcq_flash_attn_ext(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                       const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, float * out, int D,
                       int Dv, int Sq, int H, int Hkv, int n_kv, float scale, void * ws, size_t ws_size,
                       void * stream) {
    return guarded([&] {
        need_dims(Sq, "Sq");
        need_dims(H, "H");
        need_dims(Hkv, "Hkv");
        need_dims(n_kv, "n_kv");
        need_ptr(q, "q", 4);
        need_ptr(k, "k", 16);
        need_ptr(v, "v", 16);
        need_ptr(out, "out", 4);
        need_ptr(ws, "workspace", 256);
        require(k_j % 8 == 0 && v_j % 8 == 0 && k_h % 8 == 0 && v_h % 8 == 0,
                "K/V row and head strides must be multiples of 8 elements (16-byte rows)");
        require(k_j >= D && v_j >= Dv, "K/V row strides must cover a row");
        require(q_s >= 0 && q_h >= 0, "bad q strides");
        if (mask) require(m_s >= n_kv, "mask row stride must be >= n_kv");
        require(std::isfinite(scale), "scale must be finite");
        launch_flash_attn(q, q_h, q_s, k, k_h, k_j, v, v_h, v_j, mask, m_s, out, D, Dv, Sq, H, Hkv, n_kv, scale, ws,
                          ws_size, as_stream(stream));
    });
}

int gcq_rms_norm(const float * x, int64_t ldx, float * y, int64_t ldy, const float * w, int64_t rows, int64_t n,
                 float eps, void * stream) {
    return guarded([&] {
        need_dims(rows, "rows");
        need_dims(n, "n");
        require(ldx >= n && ldy >= n, "row strides must be >= n");
        need_ptr(x, "x", 4);
        need_ptr(y, "y", 4);
        launch_rms_norm(x, ldx, y, ldy, w, rows, n, eps, as_stream(stream));
    });
}

int gcq_rms_norm_q8(const float * x, int64_t ldx, const float * w, int64_t rows, int64_t n, float eps, void * act,
                    void * stream) {
    return guarded([&] {
        need_dims(rows, "rows");
        need_dims(n, "n");
        require(n % 32 == 0 && ldx >= n && ldx % 4 == 0, "n must be a multiple of 32, ldx >= n and a multiple of 4");
        need_ptr(x, "x", 16);
        need_ptr(w, "w", 16);
        need_ptr(act, "act", 256);
        launch_rmsnorm_q8(x, ldx, w, eps, rows, n, act, as_stream(stream));
    });
}

int gcq_swiglu_q8(const float * g, const float * u, int64_t ld, int64_t rows, int64_t n, void * act, void * stream) {
    return guarded([&] {
        need_dims(rows, "rows");
        need_dims(n, "n");
        require(n % 32 == 0 && ld >= n && ld % 4 == 0, "n must be a multiple of 32, ld >= n and a multiple of 4");
        need_ptr(g, "g", 16);
        need_ptr(u, "u", 16);
        need_ptr(act, "act", 256);
        launch_swiglu_q8(g, u, ld, n, rows, act, as_stream(stream));
    });
}

int gcq_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, int64_t so_s, int64_t so_h,
                  const int32_t * pos, int64_t D, int64_t H, int64_t S, int n_dims, float freq_base, float freq_scale,
                  float attn_factor, const float * ff, void * stream) {
    return guarded([&] {
        need_dims(D, "D");
        need_dims(H, "H");
        need_dims(S, "S");
        require(n_dims > 0 && n_dims % 2 == 0 && n_dims <= D, "n_dims must be even and <= D");
        require(freq_base > 0.0f, "freq_base must be positive");
        need_ptr(x, "x", 4);
        need_ptr(out, "out", 4);
        need_ptr(pos, "pos", 4);
        launch_rope_neox(x, sx_s, sx_h, out, so_s, so_h, pos, D, H, S, n_dims, freq_base, freq_scale, attn_factor, ff,
                         as_stream(stream));
    });
}

int gcq_set_rows_f16(void * dst, int64_t dst_h, int64_t dst_j, const float * src, int64_t src_h, int64_t src_j,
                     const int32_t * idx, int64_t n, int64_t D, int64_t Hrows, int64_t dst_rows, void * stream) {
    return guarded([&] {
        need_dims(n, "n");
        need_dims(D, "D");
        need_dims(Hrows, "Hrows");
        need_dims(dst_rows, "dst_rows", 1, INT64_MAX);
        require(D % 8 == 0 && dst_j % 8 == 0 && dst_h % 8 == 0, "f16 rows must be 16-byte aligned (D, strides % 8)");
        need_ptr(dst, "dst", 16);
        need_ptr(src, "src", 4);
        need_ptr(idx, "idx", 4);
        launch_set_rows_f16(dst, dst_h, dst_j, src, src_h, src_j, idx, n, D, Hrows, dst_rows, as_stream(stream));
    });
}

int gcq_get_rows(int type, const void * table, int64_t nrows, int64_t D, const int32_t * idx, int64_t n, float * out,
                 void * stream) {
    return guarded([&] {
        require(type == T_F32 || type == T_F16 || type == T_Q4_0 || type == T_Q8_0 || is_kquant(type),
                "get_rows: table type must be F32, F16, Q4_0, Q8_0, Q4_K, Q5_K or Q6_K");
        need_k(type, D);
        need_dims(nrows, "nrows");
        need_dims(n, "n");
        need_ptr(table, "table", 4);
        need_ptr(idx, "idx", 4);
        need_ptr(out, "out", 4);
        launch_get_rows(type, table, nrows, D, idx, n, out, as_stream(stream));
    });
}

int gcq_swiglu(const float * g, const float * u, float * y, int64_t n, void * stream) {
    return guarded([&] {
        need_dims(n, "n", 0, INT64_MAX);
        need_ptr(g, "g");
        need_ptr(u, "u");
        need_ptr(y, "y");
        launch_swiglu(g, u, y, n, as_stream(stream));
    });
}

int gcq_add(const float * a, const float * b, float * y, int64_t n, int64_t nb, void * stream) {
    return guarded([&] {
        need_dims(nb, "nb", 1, INT64_MAX);
        require(n % nb == 0, "n must be a multiple of nb");
        need_ptr(a, "a");
        need_ptr(b, "b");
        need_ptr(y, "y");
        launch_binary(0, a, b, y, n, nb, as_stream(stream));
    });
}

int gcq_mul(const float * a, const float * b, float * y, int64_t n, int64_t nb, void * stream) {
    return guarded([&] {
        need_dims(nb, "nb", 1, INT64_MAX);
        require(n % nb == 0, "n must be a multiple of nb");
        need_ptr(a, "a");
        need_ptr(b, "b");
        need_ptr(y, "y");
        launch_binary(1, a, b, y, n, nb, as_stream(stream));
    });
}

int gcq_argmax(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, void * stream) {
    return guarded([&] {
        need_dims(rows, "rows");
        need_dims(n, "n");
        require(ldx >= n, "ldx must be >= n");
        need_ptr(x, "x", 4);
        need_ptr(out, "out", 4);
        launch_argmax(x, ldx, rows, n, out, as_stream(stream));
    });
}

int gcq_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev, void * stream) {
    return guarded([&] {
        need_dims(n, "n", 0, INT64_MAX);
        need_ptr(dst, "dst", 4);
        launch_fill_normal(dst, n, seed, offset, stddev, as_stream(stream));
    });
}

int gcq_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab, void * stream) {
    return guarded([&] {
        need_dims(n, "n", 0, INT64_MAX);
        require(vocab > 0, "vocab must be positive");
        need_ptr(dst, "dst", 4);
        launch_fill_ids(dst, n, seed, offset, vocab, as_stream(stream));
    });
}

// ------------------------------------------------------- ggml_compiler_rt.h (loader-free subset)

const char * ggml_compiler_version(void) { return "ggml_compiler_rt (libgcq 0.1, gfx950 HIP)"; }

const char * ggml_compiler_last_error(void) { return last_error(); }

ggml_compiler_options ggml_compiler_default_options(void) {
    ggml_compiler_options o{};
    o.backend = GGML_COMPILER_BACKEND_AUTO;
    o.device = 0;
    o.n_threads = 0;
    o.allow_cpu_fallback = false;
    return o;
}

bool ggml_compiler_has_backend(ggml_compiler_backend backend) {
    if (backend == GGML_COMPILER_BACKEND_HIP || backend == GGML_COMPILER_BACKEND_AUTO) return gcq_device_count() > 0;
    return false;  // this library has no CPU or CUDA backend
}

static int parse_type(const char * type) {
    require(type != nullptr, "type is NULL");
    const std::string t(type);
    if (t == "f32") return T_F32;
    if (t == "f16") return T_F16;
    if (t == "q4_0") return T_Q4_0;
    if (t == "q8_0") return T_Q8_0;
    if (t == "q4_K" || t == "q4_k") return T_Q4_K;
    if (t == "q5_K" || t == "q5_k") return T_Q5_K;
    if (t == "q6_K" || t == "q6_k") return T_Q6_K;
    fail("unknown or unsupported type '" + t + "' (f32, f16, q4_0, q8_0, q4_K, q5_K, q6_K)");
}

size_t ggml_compiler_row_size(const char * type, int64_t n) {
    try {
        const int t = parse_type(type);
        const size_t r = row_bytes(t, n);
        require(r != 0, "row length " + std::to_string(n) + " is not a multiple of " + type + "'s block size");
        return r;
    } catch (const Fail & e) {
        set_error(e.msg);
        return 0;
    }
}

// f32 rows in host memory -> ggml block bytes in host memory, encoded on the GPU.
size_t ggml_compiler_quantize(const char * type, const float * src, int64_t nrows, int64_t n_per_row, void * dst,
                              size_t dst_size) {
    size_t written = 0;
    float * dsrc = nullptr;
    void * ddst = nullptr;
    const int rc = guarded([&] {
        const int t = parse_type(type);
        require(n_per_row > 0 && n_per_row % (int64_t) block_elems(t) == 0,
                std::string("row length ") + std::to_string(n_per_row) + " is not a multiple of " + type +
                    "'s block size " + std::to_string(block_elems(t)));
        require(nrows >= 0, "nrows must be >= 0");
        const size_t bytes = row_bytes(t, n_per_row) * (size_t) nrows;
        require(dst_size >= bytes, "destination buffer too small");
        if (nrows == 0) return;
        need_ptr(src, "src");
        need_ptr(dst, "dst");
        if (t == T_F32) {
            std::memcpy(dst, src, bytes);
            written = bytes;
            return;
        }
        require(gcq_device_count() > 0, "no HIP device: quantization runs on the GPU");
        const size_t in_bytes = (size_t) nrows * (size_t) n_per_row * sizeof(float);
        check_hip(hipMalloc(&dsrc, in_bytes), "hipMalloc");
        check_hip(hipMalloc(&ddst, bytes), "hipMalloc");
        check_hip(hipMemcpy(dsrc, src, in_bytes, hipMemcpyHostToDevice), "copy in");
        if (t == T_F16) {
            launch_encode(T_F16, dsrc, nrows, n_per_row, ddst, nullptr);
        } else {
            launch_encode(t, dsrc, nrows, n_per_row, ddst, nullptr);
        }
        check_hip(hipMemcpy(dst, ddst, bytes, hipMemcpyDeviceToHost), "copy out");
        written = bytes;
    });
    if (dsrc) (void) hipFree(dsrc);
    if (ddst) (void) hipFree(ddst);
    return rc == 0 ? written : 0;
}

}  // extern "C"
