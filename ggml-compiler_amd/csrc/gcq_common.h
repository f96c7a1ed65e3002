// gcq_common.h - shared definitions of libgcq's HIP kernels and C ABI (gfx950 only).
//
// Type ids are GGUF's (ggml_type): F32=0, F16=1, Q4_0=2, Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14,
// Q8_K=15, I32=26.
//
// Device layouts (all offsets 256-byte aligned, see gcq_layout below):
//  * Weights ("packed"): what gcq_pack_weights makes from ggml's block rows.
//      Q4_0: nibbles [N][K/32][16 B], then fp16 scales [N][K/32]. Byte j of a block's 16 holds
//            element j (low nibble) and j+16 (high nibble), stored code = q + 8, as in ggml.
//      Q8_0: codes [N][K/32][32 B], then fp16 scales [N][K/32].
//      Q4_K, Q5_K: ggml's 144- / 176-byte super-blocks split by field: nibbles (qs[128])
//            [N][K/256][128 B], then (Q5_K) the fifth bits (qh[32]) [N][K/256][32 B], then the
//            headers {d, dmin, scales[12]} [N][K/256][16 B], each field's bytes in ggml's order, so
//            that consecutive lanes read consecutive 16-byte pieces of the nibbles.
//      Q6_K: ggml's 210-byte super-block split by field: ql[128] [N][K/256][128 B], then qh[64]
//            [N][K/256][64 B], then scales[16] [N][K/256][16 B], then fp16 d [N][K/256] (each
//            field's bytes in ggml's order, so loads stay 16-byte aligned and consecutive lanes
//            read consecutive pieces of the low bits).
//  * Quantized activations ("act"), rows of the batch b < B:
//      Q8_0 (for Q4_0 / Q8_0 weights): codes [B][K] int8, then per 32-block {float d, int sum}
//            [B][K/32]: d is the fp16 scale ggml stores (as its exact f32 value) and sum the
//            block's code sum (used to fold Q4_0's -8 offset into one integer term).
//      Q8_K (for Q4_K / Q5_K / Q6_K weights): codes [B][K] int8, then bsums int16 [B][K/16] (ggml's sums of 16
//            codes), then d float [B][K/256].
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>

#include <cstddef>
#include <cstdint>
#include <string>

namespace gcq {

enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15, T_I32 = 26 };

// K-quant weights: 256-value super-blocks, Q8_K activations.
__host__ __device__ inline bool is_kquant(int t) { return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

constexpr int QK = 32;    // Q4_0 / Q8_0 block
constexpr int QKK = 256;  // K-quant super-block

// ------------------------------------------------------------------------------ host helpers

void set_error(const std::string & msg);
const char * last_error();
uint64_t error_count();  // errors recorded by this thread so far

struct Fail {
    std::string msg;
};
[[noreturn]] inline void fail(const std::string & msg) { throw Fail{msg}; }
inline void require(bool ok, const std::string & msg) {
    if (!ok) fail(msg);
}
void check_hip(hipError_t e, const char * what);
void check_launch(const char * what);

inline hipStream_t as_stream(void * s) { return reinterpret_cast<hipStream_t>(s); }

// Device queries (attributes, occupancy, symbol addresses) that the first call on a device makes,
// possibly while the calling thread captures a stream into a HIP graph: the thread's capture mode
// is relaxed for their duration, so that no such query invalidates the capture.
struct RelaxedCapture {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    bool ok;
    RelaxedCapture() { ok = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess; }
    ~RelaxedCapture() {
        if (ok) (void) hipThreadExchangeStreamCaptureMode(&mode);
    }
    RelaxedCapture(const RelaxedCapture &) = delete;
    RelaxedCapture & operator=(const RelaxedCapture &) = delete;
};
__host__ __device__ inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }
inline bool aligned(const void * p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t block_elems(int type);   // elements per block, 0 if unknown
size_t block_bytes(int type);   // bytes per block in ggml's layout
size_t row_bytes(int type, int64_t n);

// Byte offsets inside a packed weight and a quantized activation buffer.
struct WeightLayout {
    size_t qs = 0, d = 0, total = 0;
    size_t qh = 0;  // Q5_K: the fifth bits (Q4_K / Q5_K: d is the headers' region); Q6_K: qh
    size_t sc = 0;  // Q6_K: the scales
};
// The packed Q4_K / Q5_K regions of nb super-blocks, byte offsets from the weight: nibbles
// [nb][128], Q5_K's fifth bits [nb][32], headers (d, dmin, scales[12]) [nb][16].
struct KqRegions {
    size_t qs, qh, hdr, total;
};
__host__ __device__ inline KqRegions kq_regions(int type, int64_t nb) {
    const size_t q = align256((size_t) nb * 128);
    const size_t h = type == T_Q5_K ? q + align256((size_t) nb * 32) : q;
    return {0, q, h, h + align256((size_t) nb * 16)};
}
// The packed Q6_K regions of nb super-blocks: ql [nb][128], qh [nb][64], scales [nb][16], d [nb] fp16.
struct Q6Regions {
    size_t ql, qh, sc, d, total;
};
__host__ __device__ inline Q6Regions q6_regions(int64_t nb) {
    const size_t qh = align256((size_t) nb * 128), sc = qh + align256((size_t) nb * 64);
    const size_t d = sc + align256((size_t) nb * 16);
    return {0, qh, sc, d, d + align256((size_t) nb * 2)};
}
// Byte x of ggml's first 208 bytes of super-block bi (ql[128] at 0, qh[64] at 128, scales[16] at
// 192) in a packed Q6_K weight: its offset from the weight. 16-byte pieces stay 16-byte aligned.
__host__ __device__ inline size_t q6_off(const Q6Regions & R, int64_t bi, int x) {
    return x < 128 ? R.ql + (size_t) bi * 128 + x
                   : x < 192 ? R.qh + (size_t) bi * 64 + (x - 128) : R.sc + (size_t) bi * 16 + (x - 192);
}
WeightLayout weight_layout(int type, int64_t nrows, int64_t k);
struct ActLayout {
    size_t codes = 0, meta = 0, d = 0, total = 0;
};
ActLayout act_layout(int wtype, int64_t B, int64_t k);

// Split-K plan of the decode attention (attn.hip).
struct AttnPlan {
    int nsplit, chunk;
};
AttnPlan attn_plan(int Sq, int Hkv, int n_kv);

// Byte ranges a kernel's spare workgroups read ahead of their use, so that the next launches find
// them in the 256 MB Infinity Cache instead of HBM (contents unchanged; nothing is written but a
// sink word on an impossible value).
struct Prefetch {
    const uint8_t * p[2] = {nullptr, nullptr};
    size_t n[2] = {0, 0};  // bytes, multiples of 16
    unsigned int * sink = nullptr;
    int wgs = 0;  // workgroups given to it
};

// Workgroup w of `wgs` reads its share of the ranges (16 B per thread per step) and folds it into
// an xor that is stored only if it equals a constant, so the loads are kept.
__device__ __forceinline__ void prefetch_share(const Prefetch & pf, int w, int nthreads) {
    unsigned acc = 0u;
    const size_t stride = (size_t) pf.wgs * nthreads;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint4 * q = reinterpret_cast<const uint4 *>(pf.p[r]);
        const size_t n16 = pf.n[r] / 16;
        for (size_t i = (size_t) w * nthreads + threadIdx.x; i < n16; i += 4 * stride) {
            uint4 v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = q[min(i + k * stride, n16 - 1)];
#pragma unroll
            for (int k = 0; k < 4; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    if (acc == 0x9e3779b9u) *pf.sink = acc;
}

// Arguments of the decode-row GEMV (rowgemv.hip): one f32 activation row times a packed Q4_0 /
// Q8_0 weight, with the node before (prologue) and after (epilogue) the mul_mat in one launch.
enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_MERGE = 2, PRO_SWIGLU = 3 };
// EPI_V_CACHE (K-quant row GEMV only): the v rows alone, pairs written to the f16 v cache at pos.
enum { EPI_STORE = 0, EPI_ROPE_KV = 1, EPI_SWIGLU = 2, EPI_V_CACHE = 3 };

struct RowArgs {
    const uint8_t * wqs;
    const uint16_t * wd;
    int N, nb;  // packed weight rows, blocks per row
    // prologue
    const float * x;          // PRO_SWIGLU: the gate row
    const float * norm_w;
    const float * up;         // PRO_SWIGLU: the up row
    float eps;
    const float * part_o;     // [H][nsplit][D]
    const float2 * part_ml;   // [H][nsplit] (max, exp-sum)
    int nsplit;
    // epilogue
    float * y;  // EPI_STORE [N], EPI_SWIGLU [N/2], EPI_ROPE_KV: roped q [H*D]
    const float * res;
    const int * pos;
    const float2 * rope_cs;  // EPI_ROPE_KV: (cos, sin) of rotation index i at pos, i < D/2
    uint16_t * kc;  // [Hkv][ctx][D] f16
    uint16_t * vc;
    int64_t ctx;
    int H, Hkv, D;
    int xc;  // set by launch_row_gemv: the x waves take row groups too (PLAIN / NORM)
    // set by launch_row_gemv for EPI_ROPE_KV: floor(2^32 / (D/2)) + 1, so that x / (D/2) =
    // mulhi(x, hd_magic) for every 0 <= x < 2^32 / (D/2) (one scalar multiply, no branch)
    uint32_t hd_magic;
    // Several weights of one row length read by the same row (q / k / v, gate / up), EPI_STORE:
    // rows [r_end[k-1], r_end[k]) are weight k's, its codes and scales at byte offsets r_qs[k] /
    // r_d[k] from wqs / wd (spans qs_span / d_span bytes, < 2 GB), its results to r_y[k].
    int nr;  // 0: one weight
    int r_end[3];
    uint32_t r_qs[3], r_d[3], qs_span, d_span;
    float * r_y[3];
};

void launch_row_gemv(int type, int pro, int epi, const RowArgs & a, hipStream_t s);

// Byte offsets and spans of up to 3 packed weights (qs[k], d[k], N[k] rows of K) for RowArgs'
// ranges; false when they span 2 GB or more.
bool row_gemv_ranges(int type, int n, const uint8_t * const * w, const int64_t * N, int64_t K, RowArgs & a);

// The K-quant decode-row GEMV (rowgemv_kq.hip): a packed Q4_K / Q5_K / Q6_K weight times one f32
// row, quantized to Q8_K (optionally rms-normalized or merged from attention partials first)
// inside the launch.
struct RowKqArgs {
    const uint8_t * w;     // the packed weight; several weights: the lowest of them
    const float * x;       // the activation row [K]
    float * y;             // EPI_STORE [N], EPI_SWIGLU [N/2], EPI_ROPE_KV: roped q [H*D]
    const float * res;     // EPI_STORE with one weight, optional: y = res + W x
    const float * norm_w;  // y = W (rms_norm(x) * norm_w) (ggml_rms_norm then ggml_mul)
    float eps;
    int N, ntask;          // rows (of all weights), 32-value tasks per row (K / 32)
    int xc;                // set by the launch: the x waves take row groups too
    // Weight k's nibbles, fifth bits (Q5_K) and headers at byte offsets r_qs[k], r_qh[k], r_hdr[k]
    // from w, the weights spanning `span` bytes (< 2 GB). Several weights of one row length read by
    // the same row: rows [r_end[k-1], r_end[k]) are weight k's; EPI_STORE writes weight k's results
    // to r_y[k]. Row pairs as RowArgs' (q / k / v rope, gate / up).
    int nr;  // 0 or 1: one weight
    int r_end[3];
    uint32_t r_qs[3], r_qh[3], r_hdr[3], span;
    uint32_t r_d[3];  // Q6_K: weight k's fp16 d (its r_qs / r_qh / r_hdr: ql, qh, scales)
    float * r_y[3];
    // PRO_MERGE: the attention row from split partials o [H][nsplit][D], (max, exp-sum) [H][nsplit]
    const float * part_o;
    const float2 * part_ml;
    int nsplit;
    // EPI_ROPE_KV: the position, its (cos, sin) table, the f16 caches [Hkv][ctx][D]
    const int * pos;
    const float2 * rope_cs;
    uint16_t * kc;
    uint16_t * vc;
    int64_t ctx;
    int H, Hkv, D;      // D: also PRO_MERGE's head size
    uint32_t hd_magic;  // set by the launch: x / (D/2) = mulhi(x, hd_magic)
};

// Offsets and span of up to 3 K-quant weights (N[k] rows of K) for RowKqArgs' ranges; false when
// they span 2 GB or more.
bool row_gemv_kq_ranges(int type, int n, const uint8_t * const * w, const int64_t * N, int64_t K, RowKqArgs & a);
// Whether launch_row_gemv_kq_epi runs this epilogue on rows of K values (the row-pair epilogues
// take rows of at most 4096 values).
bool row_gemv_kq_epi_fits(int type, int epi, int64_t K);
void launch_row_gemv_kq_epi(int type, int pro, int epi, const RowKqArgs & a, hipStream_t s);
// One packed weight of N rows of K as RowKqArgs' weight fields (w, ranges, span, N, ntask).
void row_gemv_kq_one(int type, const void * w, int64_t N, int64_t K, RowKqArgs & a);

// Shapes and byte strides of a strided copy / conversion (elementwise.hip).
struct Cpy4 {
    int64_t sne[4], snb[4], dne[4], dnb[4];
};
void launch_cpy(const void * src, int st, void * dst, int dt, const Cpy4 & g, int64_t n, hipStream_t s);

// One get_rows / cpy / rope-table job of k_small_jobs (n threads, one element each).
enum { SJ_GETROWS = 0, SJ_CPY = 1, SJ_ROPE_TABLE = 2 };
struct SmallJob {
    int kind, type, type2, D;  // get_rows: table type, row length; cpy: source, destination type; rope: n_dims
    int64_t n, rows;           // threads; get_rows: table rows
    const void * src;          // table / cpy source / positions
    const void * aux;          // get_rows: indices; rope: frequency factors (or null)
    void * dst;
    float f[3];  // rope: theta_scale, freq_scale, attn_factor
    Cpy4 g;      // cpy: shapes and strides
};
struct SmallJobs {
    SmallJob j[3];
    int nj;
    unsigned first[3];  // job k's first block
};
SmallJob small_job_get_rows(int type, const void * tab, int64_t nrows_tab, int64_t D, const int32_t * idx, int64_t n,
                            float * out);
SmallJob small_job_cpy(const void * src, int st, void * dst, int dt, const Cpy4 & g, int64_t n);
SmallJob small_job_rope_table(const int32_t * pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                              const float * ff, float2 * cs);
void launch_small_jobs(const SmallJob * jobs, int n, hipStream_t s);

// A second tensor for one launch of rope / set_rows (q and k; k and v of a layer), same positions.
struct RopeSecond {
    const float * x;
    int64_t sx_s, sx_h;
    float * out;
    int64_t so_s, so_h, H;
};
struct SetRowsSecond {
    uint16_t * dst;
    int64_t dst_h, dst_j;
    const float * src;
    int64_t src_h, src_j;
    int D, Hrows;
    int64_t dst_rows;
};
void launch_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, int64_t so_s, int64_t so_h,
                      const int32_t * pos, int64_t D, int64_t H, int64_t S, int n_dims, float freq_base,
                      float freq_scale, float attn_factor, const float * ff, hipStream_t s,
                      const RopeSecond * r2 = nullptr);
void launch_set_rows_f16(void * dst, int64_t dst_h, int64_t dst_j, const float * src, int64_t src_h, int64_t src_j,
                         const int32_t * idx, int64_t n, int64_t D, int64_t Hrows, int64_t dst_rows, hipStream_t s,
                         const SetRowsSecond * r2 = nullptr);
void launch_rope_table(const int32_t * pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                       const float * ff, float2 * cs, hipStream_t s);
void launch_scale(const float * x, float * y, int64_t n, float sc, float b, hipStream_t s);
// Elementwise functions of k_unary (the numbering is ggml_unary_op's in include/ggml.h).
enum UnaryOp : int {
    UN_ABS = 0, UN_NEG = 1, UN_TANH = 2, UN_RELU = 3, UN_SIGMOID = 4, UN_GELU = 7, UN_SILU = 10, UN_EXP = 11,
    UN_GELU_ERF = 12, UN_SOFTPLUS = 13, UN_SQR = 100, UN_SQRT = 101, UN_LOG = 102, UN_SIN = 103, UN_COS = 104,
    UN_CLAMP = 105,
};
bool unary_known(int op);
// lo / hi: clamp's bounds (unused by the other functions).
void launch_unary(int op, const float * x, float * y, int64_t n, float lo, float hi, hipStream_t s);
// Per contiguous row of n: (x - mean) / sqrt(var + eps) (norm); the sum, or the mean (sum / n).
void launch_norm(const float * x, float * y, int64_t rows, int64_t n, float eps, hipStream_t s);
// dst (contiguous f32, shape g.dne) = src tiled: element c of dst reads src at c % g.sne (byte strides g.snb).
void launch_repeat(const float * src, float * dst, const Cpy4 & g, int64_t n, hipStream_t s);
void launch_row_sum(const float * x, float * y, int64_t rows, int64_t n, bool mean, hipStream_t s);
// softmax(x * scale + mask) over rows of n; rows = r1 * r2 * r3 (x and y contiguous); mask row
// (i1, i2 % m2, i3 % m3) at element strides mld, ms2, ms3, f16 when mask_f16, or no mask.
void launch_soft_max(const float * x, float * y, int64_t n, int64_t r1, int64_t r2, int64_t r3, const void * mask,
                     bool mask_f16, int64_t mld, int64_t ms2, int64_t ms3, int64_t m2, int64_t m3, float scale,
                     hipStream_t s);
bool row_gemv_fits(int type, int64_t K);
int row_gemv_merge_max();
// ggml_mul_mat(W, x) of f32 rows with the caller's workspace (the body of gcq_mul_mat and
// gcq_mul_mat_noalloc); throws on a bad argument. mul_mat_workspace_bytes: the workspace it needs.
void mul_mat_with_workspace(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx, int64_t M,
                            float * y, int64_t ldy, void * ws, size_t ws_size, hipStream_t s);
size_t mul_mat_workspace_bytes(int wtype, int64_t M, int64_t K);

// Wraps a C-ABI body: 0 on success, -1 with last_error set on failure.
template <class F>
int guarded(F && f) {
    try {
        f();
        return 0;
    } catch (const Fail & e) {
        set_error(e.msg);
    } catch (const std::exception & e) {
        set_error(e.what());
    } catch (...) {
        set_error("unknown error");
    }
    return -1;
}

// ---------------------------------------------------------------------------- device helpers

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}
// The NEOX rotation of the pair (x0, x1) by (cos, sin). Every rope site (the rope kernel, the
// GEMV epilogues) calls this one expression, so each compiles to the same operations whatever
// contraction its caller's scope allows.
__device__ __forceinline__ float2 rope_pair(float x0, float x1, float2 cs) {
    return make_float2(x0 * cs.x - x1 * cs.y, x0 * cs.y + x1 * cs.x);
}
// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 in the default rounding mode).
__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16) f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// fp32 -> fp16 bits, round to nearest even, in integer arithmetic. Used for every stored quant
// scale: it keeps -0 and fp16 subnormals exact, whatever the compiler folds around a conversion
// instruction (a multiply feeding v_cvt_f16_f32 may become v_fma_mix with a +0 addend, which
// turns -0 into +0).
__device__ __forceinline__ uint16_t f2h_exact(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);
    if (ax >= 0x47800000u) return (uint16_t) (sign | 0x7c00u);
    if (ax < 0x38800000u) {
        const uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t) sign;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t) (sign | h);
    }
    uint32_t h = (((ax >> 23) - 112) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t) (sign | h);
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// int32 dot of one Q4_0 weight block (16 nibble bytes, stored code = q + 8) with a Q8_0 activation
// block (codes xa: elements 0-15, xb: 16-31; xsum = their code sum): sum (q - 8) x.
__device__ __forceinline__ int dot_blk_q4_0(const uint4 w, const int4 xa, const int4 xb, int xsum) {
    int s = 0;
    s = sdot4((int) (w.x & 0x0F0F0F0Fu), xa.x, s);
    s = sdot4((int) (w.y & 0x0F0F0F0Fu), xa.y, s);
    s = sdot4((int) (w.z & 0x0F0F0F0Fu), xa.z, s);
    s = sdot4((int) (w.w & 0x0F0F0F0Fu), xa.w, s);
    s = sdot4((int) ((w.x >> 4) & 0x0F0F0F0Fu), xb.x, s);
    s = sdot4((int) ((w.y >> 4) & 0x0F0F0F0Fu), xb.y, s);
    s = sdot4((int) ((w.z >> 4) & 0x0F0F0F0Fu), xb.z, s);
    s = sdot4((int) ((w.w >> 4) & 0x0F0F0F0Fu), xb.w, s);
    return s - 8 * xsum;
}

// int32 dot of one Q8_0 weight block (codes wa: elements 0-15, wb: 16-31) with a Q8_0 activation block.
__device__ __forceinline__ int dot_blk_q8_0(const uint4 wa, const uint4 wb, const int4 xa, const int4 xb) {
    int s = 0;
    s = sdot4((int) wa.x, xa.x, s);
    s = sdot4((int) wa.y, xa.y, s);
    s = sdot4((int) wa.z, xa.z, s);
    s = sdot4((int) wa.w, xa.w, s);
    s = sdot4((int) wb.x, xb.x, s);
    s = sdot4((int) wb.y, xb.y, s);
    s = sdot4((int) wb.z, xb.z, s);
    s = sdot4((int) wb.w, xb.w, s);
    return s;
}

// Counters in LDS through which the wavefronts of one workgroup hand LDS data to each other
// without a workgroup barrier (a barrier would also wait for wavefronts stalled on issuing memory
// loads). A wavefront's LDS operations complete in order, so the writer waits for its LDS writes
// (lgkmcnt only: its global loads stay in flight) before counting, and the reader's LDS reads
// after the wait see them; the signal fences keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void lds_signal(unsigned int * f) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
    __hip_atomic_fetch_add(f, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_wait(unsigned int * f, unsigned int n) {
    while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < n) __builtin_amdgcn_s_sleep(1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A 32-bit store that reaches the device-coherent level (sc1), for partials another kernel's
// workgroups on other XCDs read.
__device__ __forceinline__ void st_co_f(float * p, float v) {
    __hip_atomic_store(reinterpret_cast<unsigned *>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Streaming (non-temporal) loads for data read once per launch (weights, KV rows): they do not
// displace the L2's reused lines, and HBM streams measurably faster with them on gfx950.
__device__ __forceinline__ uint4 ld_nt(const uint4 * p) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4 t = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// Cross-lane reductions on DPP (VALU lane moves) instead of LDS permutes. Within a group of 2O
// lanes, step O pairs each lane with lane ^ O (O = 1, 2: quad permutes) or with its mirror
// (O = 4, 8: row half-mirror, row mirror); once each half of the group holds one value, both pair
// the same two halves, so a reduction gives the xor butterfly's result bit for bit. Across the four
// 16-lane rows of a wavefront the row results are read with readlane and combined as the
// butterfly's last two steps would: (row0 . row1) . (row2 . row3).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int O>
__device__ __forceinline__ int lane_pair_i(int v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8, "DPP pairs within 16 lanes");
    return dpp_i<O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x141 : 0x140>(v);
}
template <int O>
__device__ __forceinline__ float lane_pair(float v) { return __int_as_float(lane_pair_i<O>(__float_as_int(v))); }
template <int O>
__device__ __forceinline__ double lane_pair(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = lane_pair_i<O>((int) (b & 0xffffffffll)), hi = lane_pair_i<O>((int) (b >> 32));
    return __longlong_as_double(((long long) hi << 32) | (unsigned int) lo);
}

// Lane l ^ 8 exactly (row rotate by 8), for values that differ within the 8-lane halves.
__device__ __forceinline__ float lane_xor8(float v) { return __int_as_float(dpp_i<0x128>(__float_as_int(v))); }

template <class T> __device__ __forceinline__ T op_add(T a, T b) { return a + b; }
__device__ __forceinline__ float fmaxf_op(float a, float b) { return fmaxf(a, b); }

// Reduction over each group of W lanes (W in 1..16, a power of two), every lane getting its
// group's result.
template <int W, class T, T (*OP)(T, T)>
__device__ __forceinline__ T group_reduce(T v) {
    if constexpr (W >= 2) v = OP(v, lane_pair<1>(v));
    if constexpr (W >= 4) v = OP(v, lane_pair<2>(v));
    if constexpr (W >= 8) v = OP(v, lane_pair<4>(v));
    if constexpr (W >= 16) v = OP(v, lane_pair<8>(v));
    return v;
}

// Pair sums across rows with gfx950's row swaps: lane l gets f(v[l & ~16], v[l | 16]) (X16) or
// f(v[l & ~32], v[l | 32]) (X32), the xor butterfly's pairs, low lane first.
template <int X, class F>
__device__ __forceinline__ float row_pair(float v, F f) {
    static_assert(X == 16 || X == 32, "row pairs");
    const unsigned u = __float_as_uint(v);
    if constexpr (X == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return f(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return f(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
}

// Sums of V values (V = 1..64, a power of two) over the wavefront's 64 lanes, scattered: at each
// of the six pair levels (lane ^ 32, ^ 16 with gfx950's row swaps, ^ 8 by a row rotate, the 8-lane
// mirror, ^ 2, ^ 1) a lane keeps the half of its values that its lane bit selects and adds its
// partner's copy of that half, until one value is left; later levels add it up plainly. Afterwards
// v[0] of lane l is the total of value l >> (6 - log2 V) (every total on 64 / V lanes). About two
// VALU operations per value, against some ten for a separate butterfly per value.
template <int V>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[V]) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "a power of two up to 64 values");
    const int lane = threadIdx.x & 63;
    auto lvl_swap = [&](auto X, auto n_c) {
        constexpr int n = decltype(n_c)::value;
        if constexpr (n > 1) {
#pragma unroll
            for (int j = 0; j < n / 2; j++) {
                const unsigned a = __float_as_uint(v[j]), b = __float_as_uint(v[j + n / 2]);
                const auto r = decltype(X)::value == 32 ? __builtin_amdgcn_permlane32_swap(a, b, false, false)
                                                        : __builtin_amdgcn_permlane16_swap(a, b, false, false);
                v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
        } else {
            v[0] = row_pair<decltype(X)::value>(v[0], [](float a, float b) { return a + b; });
        }
    };
    auto lvl_dpp = [&](auto O, auto n_c) {
        constexpr int n = decltype(n_c)::value, o = decltype(O)::value;
        auto partner = [](float x) { return o == 8 ? lane_xor8(x) : lane_pair<o>(x); };
        if constexpr (n > 1) {
            const bool hi = (lane & o) != 0;
#pragma unroll
            for (int j = 0; j < n / 2; j++) {
                const float keep = hi ? v[j + n / 2] : v[j], send = hi ? v[j] : v[j + n / 2];
                v[j] = keep + partner(send);
            }
        } else {
            v[0] = v[0] + partner(v[0]);
        }
    };
    using I = int;
    lvl_swap(std::integral_constant<I, 32>{}, std::integral_constant<I, V>{});
    lvl_swap(std::integral_constant<I, 16>{}, std::integral_constant<I, (V > 1 ? V / 2 : 1)>{});
    lvl_dpp(std::integral_constant<I, 8>{}, std::integral_constant<I, (V > 4 ? V / 4 : 1)>{});
    lvl_dpp(std::integral_constant<I, 4>{}, std::integral_constant<I, (V > 8 ? V / 8 : 1)>{});
    lvl_dpp(std::integral_constant<I, 2>{}, std::integral_constant<I, (V > 16 ? V / 16 : 1)>{});
    lvl_dpp(std::integral_constant<I, 1>{}, std::integral_constant<I, (V > 32 ? V / 32 : 1)>{});
}

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int) (b & 0xffffffffll), l), hi = __builtin_amdgcn_readlane((int) (b >> 32), l);
    return __longlong_as_double(((long long) hi << 32) | (unsigned int) lo);
}

template <class T, T (*OP)(T, T)>
__device__ __forceinline__ T wave_reduce(T v) {
    v = group_reduce<16, T, OP>(v);
    if constexpr (sizeof(T) == 8) {
        return OP(OP(readlane_d(v, 0), readlane_d(v, 16)), OP(readlane_d(v, 32), readlane_d(v, 48)));
    } else {
        return OP(OP(readlane_f(v, 0), readlane_f(v, 16)), OP(readlane_f(v, 32), readlane_f(v, 48)));
    }
}

// W = 64: the whole wavefront (wave-uniform result); W <= 16: each W-lane group; W = 32: each half.
template <int W = 64>
__device__ __forceinline__ float wave_sum(float v) {
    if constexpr (W == 64) return wave_reduce<float, op_add<float>>(v);
    else if constexpr (W == 32) return group_reduce<16, float, op_add<float>>(v) + __shfl_xor(group_reduce<16, float, op_add<float>>(v), 16, 64);
    else return group_reduce<W, float, op_add<float>>(v);
}
template <int W = 64>
__device__ __forceinline__ float wave_max(float v) {
    if constexpr (W == 64) return wave_reduce<float, fmaxf_op>(v);
    else if constexpr (W == 32) return fmaxf(group_reduce<16, float, fmaxf_op>(v), __shfl_xor(group_reduce<16, float, fmaxf_op>(v), 16, 64));
    else return group_reduce<W, float, fmaxf_op>(v);
}
__device__ __forceinline__ double wave_sum_d(double v) { return wave_reduce<double, op_add<double>>(v); }
template <int W = 64>
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// (max, first index) selection: a value wins if greater, or equal at a lower index; NaN never
// wins. The choice does not depend on the order values are offered in.
__device__ __forceinline__ void argmax_take(float & v, int & idx, float a, int i) {
    if (a > v || (a == v && i < idx)) {
        v = a;
        idx = i;
    }
}

// Values per workgroup of the sliced argmax: 256 threads x two 16-byte loads.
constexpr int kArgmaxSlice = 2048;

// (max, first index) of x[lo, hi) (hi - lo <= kArgmaxSlice) over a 256-thread workgroup, every
// thread calling it: both loads of a thread in flight together (16-byte when vec: x + lo 16-byte
// aligned), then the waves' results through LDS. (v, idx) = (-inf, INT_MAX) for an empty slice.
__device__ __forceinline__ void slice_argmax(const float * __restrict__ x, int lo, int hi, bool vec, float & v,
                                             int & idx) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int t = threadIdx.x;
    float q[2][4];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int e = lo + 4 * (t + 256 * u);
        if (vec && e + 3 < hi) {
            const float4 f = *reinterpret_cast<const float4 *>(x + e);
            q[u][0] = f.x;
            q[u][1] = f.y;
            q[u][2] = f.z;
            q[u][3] = f.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) q[u][c] = e + c < hi ? x[e + c] : -INFINITY;
        }
    }
    v = -INFINITY;
    idx = 0x7fffffff;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int e = lo + 4 * (t + 256 * u) + c;
            if (e < hi) argmax_take(v, idx, q[u][c], e);
        }
    for (int o = 32; o > 0; o >>= 1) argmax_take(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((t & 63) == 0) {
        sv[t >> 6] = v;
        si[t >> 6] = idx;
    }
    __syncthreads();
    v = sv[0];
    idx = si[0];
    for (int w = 1; w < 4; w++) argmax_take(v, idx, sv[w], si[w]);
    __syncthreads();
}

// 1/sqrt(mean(x^2) + eps) of one row, for a 256-thread block (all threads call it): squares
// rounded to f32, summed in double, mean rounded to f32, as ggml-cpu's rms_norm.
__device__ __forceinline__ float rms_scale(const float * xr, int n, float eps) {
    __shared__ double red[4];
    double s = 0.0;
    // Loads of 8 strides issued together, then summed in the same order as one at a time.
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * 256) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = i0 + 256 * k < n ? xr[i0 + 256 * k] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + 256 * k < n) s += (double) (v[k] * v[k]);
    }
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float mean = (float) ((red[0] + red[1] + red[2] + red[3]) / (double) n);
    return 1.0f / sqrtf(mean + eps);
}

// Q8_0 conversion (canonical variant, as quant.hip's k_act_q8_0) of one 32-value block held 4 per
// lane by 8 consecutive lanes; lane8 = the lane's index in its group of 8.
__device__ __forceinline__ void q8_block_store(float4 v, int8_t * codes, float2 * meta, int lane8) {
#pragma clang fp contract(off)
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group_reduce<8, float, fmaxf_op>(amax);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    const int q0 = (int) __builtin_rintf(v.x * id);
    const int q1 = (int) __builtin_rintf(v.y * id);
    const int q2 = (int) __builtin_rintf(v.z * id);
    const int q3 = (int) __builtin_rintf(v.w * id);
    *reinterpret_cast<int *>(codes + 4 * lane8) =
        (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3;
    s += lane_pair_i<1>(s);
    s += lane_pair_i<2>(s);
    s += lane_pair_i<4>(s);
    if (lane8 == 0) *meta = make_float2(h2f(f2h_exact(__fdiv_rn(amax, 127.0f))), __int_as_float(s));
}

// The same conversion of one 32-value block held 16 per lane by two neighbouring lanes (half = the
// lane's half of the block): codes of the block at codes[0..32), its (d, code sum) at *meta.
__device__ __forceinline__ void q8_half_block_store(const float (&v)[16], int8_t * codes, float2 * meta, int half) {
#pragma clang fp contract(off)
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, lane_pair<1>(amax));
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    int w[4];
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int packed = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int q = (int) __builtin_rintf(v[4 * k + j] * id);
            s += q;
            packed |= (q & 0xff) << (8 * j);
        }
        w[k] = packed;
    }
    *reinterpret_cast<int4 *>(codes + 16 * half) = make_int4(w[0], w[1], w[2], w[3]);
    s += lane_pair_i<1>(s);
    if (half == 0) *meta = make_float2(h2f(f2h_exact(__fdiv_rn(amax, 127.0f))), __int_as_float(s));
}

// rms_norm of one row of n (a multiple of 32) times w, quantized to Q8_0: codes [n], meta [n/32].
// Called by all 256 threads of a block.
__device__ __forceinline__ void rmsnorm_q8_row(const float * xr, int n, const float * w, float eps, int8_t * codes,
                                               float2 * meta) {
    const float scale = rms_scale(xr, n, eps);
    for (int e = threadIdx.x * 4; e < n; e += 1024) {  // 8 lanes per 32-block
        float4 v = *reinterpret_cast<const float4 *>(xr + e);
        const float4 wv = *reinterpret_cast<const float4 *>(w + e);
        v.x = (v.x * scale) * wv.x;
        v.y = (v.y * scale) * wv.y;
        v.z = (v.z * scale) * wv.z;
        v.w = (v.w * scale) * wv.w;
        q8_block_store(v, codes + (e & ~31), meta + e / 32, (e / 4) & 7);
    }
}

// Element c of a packed K-quant table row, as ggml's dequantize_row_q{4,5,6}_K computes it (products
// and the difference rounded one at a time): Q4_K / Q5_K d * sc * q - dmin * m, Q6_K d * sc * (q - 32).
__device__ __forceinline__ float kquant_table_value(int type, const uint8_t * tab, int64_t nrows, int D, int64_t r,
                                                    int c) {
    const int nsb = D / QKK, w = c % QKK;
    const int64_t bi = r * nsb + c / QKK;
    auto byte = [](const uint8_t * p, int i) { return (int) p[i]; };
    if (type == T_Q6_K) {
        const Q6Regions R = q6_regions(nrows * nsb);
        const uint16_t * dv = reinterpret_cast<const uint16_t *>(tab + R.d);
        const int h = w / 128, qq = (w % 128) / 32, l = w % 32;
        const int a = (int) tab[q6_off(R, bi, 64 * h + 32 * (qq & 1) + l)];
        const int qh = (int) tab[q6_off(R, bi, 128 + 32 * h + l)];
        const int q = ((qq < 2 ? a & 0xF : a >> 4) | (((qh >> (2 * qq)) & 3) << 4)) - 32;
        const int sc = (int) reinterpret_cast<const int8_t *>(tab + q6_off(R, bi, 192 + 8 * h))[l / 16 + 2 * qq];
        return __fmul_rn(__fmul_rn(h2f(dv[bi]), (float) sc), (float) q);
    }
    const KqRegions R = kq_regions(type, nrows * nsb);
    const uint8_t * b = tab + R.hdr + bi * 16;  // the header: d, dmin, scales[12]
    const int cc = w / 64, hi = (w % 64) >= 32, l = w % 32, j = 2 * cc + hi;  // sub-block j, value l
    const int x = byte(tab + R.qs + bi * 128, 32 * cc + l);
    int q = hi ? x >> 4 : x & 0xF;
    if (type == T_Q5_K) q += ((byte(tab + R.qh + bi * 32, l) >> j) & 1) << 4;
    int sc, m;  // get_scale_min_k4 on the 12 scale bytes at 4
    if (j < 4) {
        sc = byte(b, 4 + j) & 63;
        m = byte(b, 8 + j) & 63;
    } else {
        sc = (byte(b, 8 + j) & 0xF) | ((byte(b, j) >> 6) << 4);
        m = (byte(b, 8 + j) >> 4) | ((byte(b, 4 + j) >> 6) << 4);
    }
    const float d = h2f((uint16_t) (byte(b, 0) | (byte(b, 1) << 8))), dmin = h2f((uint16_t) (byte(b, 2) | (byte(b, 3) << 8)));
    return __fsub_rn(__fmul_rn(__fmul_rn(d, (float) sc), (float) q), __fmul_rn(dmin, (float) m));
}

// Element c of row r of a get_rows table (F32, F16, packed Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K of
// nrows x D); NaN for a row outside the table.
__device__ __forceinline__ float table_value(int type, const uint8_t * tab, int64_t nrows, int D, int64_t r, int c) {
    if (r < 0 || r >= nrows) return __builtin_nanf("");
    if (type == T_F32) return reinterpret_cast<const float *>(tab)[r * D + c];
    if (type == T_F16) return h2f(reinterpret_cast<const uint16_t *>(tab)[r * D + c]);
    if (type == T_Q4_K || type == T_Q5_K || type == T_Q6_K) return kquant_table_value(type, tab, nrows, D, r, c);
    const int nb = D / QK;
    const int64_t blk = r * nb + c / QK;
    const int e = c % QK;
    const size_t qbytes = (size_t) nrows * nb * (type == T_Q4_0 ? 16 : 32);
    const uint16_t * d = reinterpret_cast<const uint16_t *>(tab + align256(qbytes));
    if (type == T_Q4_0) {
        const uint8_t b = tab[blk * 16 + (e & 15)];
        return (float) ((e < 16 ? (b & 0xF) : (b >> 4)) - 8) * h2f(d[blk]);
    }
    return (float) reinterpret_cast<const int8_t *>(tab)[blk * 32 + e] * h2f(d[blk]);
}

// Counter-based splitmix64 (output i of a generator whose state starts at seed).
__device__ __forceinline__ uint64_t rnd64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

}  // namespace gcq
