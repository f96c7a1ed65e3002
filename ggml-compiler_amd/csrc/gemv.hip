// gemv.hip - quantized mat-vec for decode (batch 1..8): y[b, n] = sum_k W[n, k] x[b, k].
//
// Replaces ggml_mul_mat on a Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K weight with an f32 src1 of 1..8 rows
// (runtime/src/ops.cpp:107-119 -> runtime/include/ggml_compiler_ops.h:116-122). As ggml-cpu
// does, the activation is first quantized to the weight's vec_dot_type (quant.hip); each
// weight block then contributes an exact int32 dot sum times its fp16 scale(s), accumulated in
// fp32 (ggml vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0 / vec_dot_q{4,5,6}_K_q8_K).
//
// HBM-bound by the weight stream. One wavefront owns R rows; lane l takes blocks l, l+64, ...
// so each weight load instruction moves 64 x 16 B of one row contiguously. All of a lane's
// weight loads for a pass of 64*NBL blocks are issued before any math (NBL*R*16 B in flight
// per lane); the small activation (x codes + scales) is re-read from L1/L2 per block and
// reused across the R rows; integer dots use v_dot4_i32_i8; a butterfly over the wavefront
// finishes each output.
#include "gcq_common.h"

#include <algorithm>
#include <cstdlib>
#include <string>

namespace gcq {

// Integer dot of one Q4_0 block (16 B of nibbles) with one Q8_0 activation block (32 codes):
// sum_j (q_j - 8) * x_j, computed as sum q_j x_j - 8 sum x_j (xsum from the quantizer).
__device__ __forceinline__ int dot_q4_0(const uint4 w, const int4 xa, const int4 xb, int xsum) {
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

__device__ __forceinline__ int dot_q8_0(const uint4 wa, const uint4 wb, const int4 xa, const int4 xb) {
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

// One 64-value chunk c of a Q4_K super-block (32 bytes of nibbles: low = sub-block 2c, high =
// sub-block 2c+1) against 64 Q8_K codes: the two sub-block dots.
__device__ __forceinline__ void dot_q4_K_chunk(const uint4 wa, const uint4 wb, const int4 x0, const int4 x1,
                                               const int4 x2, const int4 x3, int & lo, int & hi) {
    const uint32_t w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int a = 0, b = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a = sdot4((int) (w[j] & 0x0F0F0F0Fu), xl[j], a);
        b = sdot4((int) ((w[j] >> 4) & 0x0F0F0F0Fu), xh[j], b);
    }
    lo = a;
    hi = b;
}

__device__ __forceinline__ void scale_min_k4_w(int j, const uint32_t s[3], int & sc, int & m) {
    auto byte = [&](int i) { return (int) ((s[i >> 2] >> (8 * (i & 3))) & 0xff); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Chunk c of a Q5_K super-block: the Q4_K nibbles plus the fifth bit of value l (l < 32) of
// sub-block 2c in bit 2c of qh[l], of sub-block 2c + 1 in bit 2c + 1.
__device__ __forceinline__ void dot_q5_K_chunk(const uint4 wa, const uint4 wb, const uint4 ha, const uint4 hb, int c,
                                               const int4 x0, const int4 x1, const int4 x2, const int4 x3, int & lo,
                                               int & hi) {
    const uint32_t w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    const uint32_t h[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int a = 0, b = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t ql = (w[j] & 0x0F0F0F0Fu) | (((h[j] >> (2 * c)) & 0x01010101u) << 4);
        const uint32_t qh = ((w[j] >> 4) & 0x0F0F0F0Fu) | (((h[j] >> (2 * c + 1)) & 0x01010101u) << 4);
        a = sdot4((int) ql, xl[j], a);
        b = sdot4((int) qh, xh[j], b);
    }
    lo = a;
    hi = b;
}

// Task (hh, jj) of a packed Q6_K super-block: 32 ql bytes at 64 hh + 32 jj (low nibbles: values
// 128 hh + 32 jj + l, high: + 64), the 32 qh bytes of half hh (2 bits per value at shift 2 jj and
// 2 jj + 4). d[k] = sum over the k-th of the task's four 16-value sub-blocks of q * x, q in 0..63
// (the stored code; the -32 offset is folded in with the bsums).
__device__ __forceinline__ void dot_q6_K_task(const uint4 la, const uint4 lb, const uint4 ha, const uint4 hb, int jj,
                                              const int4 x0, const int4 x1, const int4 x2, const int4 x3, int (&d)[4]) {
    const uint32_t w[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
    const uint32_t h[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t ql = (w[j] & 0x0F0F0F0Fu) | (((h[j] >> (2 * jj)) & 0x03030303u) << 4);
        const uint32_t qh = ((w[j] >> 4) & 0x0F0F0F0Fu) | (((h[j] >> (2 * jj + 4)) & 0x03030303u) << 4);
        s[j >> 2] = sdot4((int) ql, xl[j], s[j >> 2]);
        s[2 + (j >> 2)] = sdot4((int) qh, xh[j], s[2 + (j >> 2)]);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) d[k] = s[k];
}

// The task's int32 sum: sum_k sc_k * (d_k - 32 * bsum_k). sc8: the 8 scale bytes of half hh;
// bs01 / bs23: the two int16 bsums pairs of the task's low / high sub-blocks.
__device__ __forceinline__ int isum_q6_K_task(const int (&d)[4], const uint2 sc8, int jj, uint32_t bs01, uint32_t bs23) {
    const int s0 = (int) (int8_t) (sc8.x >> (16 * jj)), s1 = (int) (int8_t) (sc8.x >> (16 * jj + 8));
    const int s2 = (int) (int8_t) (sc8.y >> (16 * jj)), s3 = (int) (int8_t) (sc8.y >> (16 * jj + 8));
    const int b0 = (int) (int16_t) (bs01 & 0xffff), b1 = (int) (int16_t) (bs01 >> 16);
    const int b2 = (int) (int16_t) (bs23 & 0xffff), b3 = (int) (int16_t) (bs23 >> 16);
    return s0 * (d[0] - 32 * b0) + s1 * (d[1] - 32 * b1) + s2 * (d[2] - 32 * b2) + s3 * (d[3] - 32 * b3);
}

// ------------------------------------------------------------------ Q4_0 / Q8_0 kernel

template <int TYPE, int B, int R, int NBL>
__global__ __launch_bounds__(256) void k_gemv_q0(const uint8_t * __restrict__ wqs, const uint16_t * __restrict__ wd,
                                                 const int8_t * __restrict__ xc, const float2 * __restrict__ xm,
                                                 float * y, const float * res, int N, int nb, int ldy) {
    constexpr int CV = TYPE == T_Q4_0 ? 1 : 2;  // uint4 per block
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int K = nb * QK;
    const uint4 * qs = reinterpret_cast<const uint4 *>(wqs);
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = 0.0f;

    for (int base = 0; base < nb; base += 64 * NBL) {
        uint4 w[NBL][R][CV];
        uint32_t d[NBL][R];  // raw fp16 scale bits, one per register: converted where used, so no load waits
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = base + lane + 64 * i;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(row0 + r, N - 1);  // rows past N recompute N-1; never stored
                if (blk < nb) {
                    const size_t o = (size_t) row * nb + blk;
#pragma unroll
                    for (int c = 0; c < CV; c++) w[i][r][c] = qs[o * CV + c];
                    d[i][r] = wd[o];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = base + lane + 64 * i;
            if (blk >= nb) break;
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) blk * QK);
                const int4 xa = xp[0], xb = xp[1];
                const float2 m = xm[(size_t) b * nb + blk];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int s;
                    if constexpr (TYPE == T_Q4_0) s = dot_q4_0(w[i][r][0], xa, xb, __float_as_int(m.y));
                    else s = dot_q8_0(w[i][r][0], w[i][r][CV - 1], xa, xb);
                    acc[r][b] += ((float) s * h2f((uint16_t) d[i][r])) * m.x;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float v = wave_sum(acc[r][b]);
            if (lane == r * B + b && row0 + r < N) {
                const size_t o = (size_t) b * ldy + row0 + r;
                y[o] = res ? v + res[o] : v;
            }
        }
}

// Persistent variant for rows that fit one pass (nb <= 64*NBL): each wavefront keeps its lanes'
// activation blocks in registers for the whole launch and walks row groups g, g + waves, ...,
// loading the next group's weights before it reduces the current one, so a wavefront always has
// R*NBL*(16 or 32) bytes per lane of HBM reads in flight.
template <int TYPE, int B, int R, int NBL>
__global__ __launch_bounds__(256) void k_gemv_p(const uint8_t * __restrict__ wqs, const uint16_t * __restrict__ wd,
                                                const int8_t * __restrict__ xc, const float2 * __restrict__ xm,
                                                float * y, const float * res, int N, int nb, int ldy) {
    constexpr int CV = TYPE == T_Q4_0 ? 1 : 2;
    constexpr int NWV = 4;
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * NWV;
    const int ng = (N + R - 1) / R;
    const int K = nb * QK;
    const uint4 * qs = reinterpret_cast<const uint4 *>(wqs);

    uint4 w[NBL][R][CV];
    uint32_t d[NBL][R];  // raw fp16 scale bits, one per register: converted where used, so no load waits
    auto load = [&](int g, uint4 (&wv)[NBL][R][CV], uint32_t (&dv)[NBL][R]) {
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = min(lane + 64 * i, nb - 1);  // lanes past the row reload its last block, unused
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(g * R + r, N - 1);
                const size_t o = (size_t) row * nb + blk;
#pragma unroll
                for (int c = 0; c < CV; c++) wv[i][r][c] = qs[o * CV + c];
                dv[i][r] = wd[o];
            }
        }
    };

    int g = blockIdx.x * NWV + (threadIdx.x >> 6);
    if (g < ng) load(g, w, d);  // first weights in flight before the activation loads

    int4 xa[NBL][B], xb[NBL][B];
    float2 xmv[NBL][B];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int blk = lane + 64 * i;
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (blk < nb) {
                const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) blk * QK);
                xa[i][b] = xp[0];
                xb[i][b] = xp[1];
                xmv[i][b] = xm[(size_t) b * nb + blk];
            }
        }
    }

    while (g < ng) {
        const int gn = g + nw;
        uint4 wn[NBL][R][CV];
        uint32_t dn[NBL][R];
        if (gn < ng) load(gn, wn, dn);
        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < B; b++) acc[r][b] = 0.0f;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            if (lane + 64 * i >= nb) break;
#pragma unroll
            for (int b = 0; b < B; b++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int s;
                    if constexpr (TYPE == T_Q4_0) s = dot_q4_0(w[i][r][0], xa[i][b], xb[i][b], __float_as_int(xmv[i][b].y));
                    else s = dot_q8_0(w[i][r][0], w[i][r][CV - 1], xa[i][b], xb[i][b]);
                    acc[r][b] += ((float) s * h2f((uint16_t) d[i][r])) * xmv[i][b].x;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < B; b++) {
                const float v = wave_sum(acc[r][b]);
                if (lane == r * B + b && g * R + r < N) {
                    const size_t o = (size_t) b * ldy + g * R + r;
                    y[o] = res ? v + res[o] : v;
                }
            }
#pragma unroll
        for (int i = 0; i < NBL; i++)
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int c = 0; c < CV; c++) w[i][r][c] = wn[i][r][c];
                d[i][r] = dn[i][r];
            }
        g = gn;
    }
}

// Batched rows (B = 2..8), K-sliced, for Q4_0 / Q8_0 / Q4_K / Q5_K weights. A lane's task is 32
// values of every weight row: a Q4_0 / Q8_0 block, or for the K-quants a half chunk of a 256-value
// super-block (16 bytes of nibbles: values 16 h .. 16 h + 15 of the chunk's two 32-value
// sub-blocks 2c and 2c + 1). A workgroup of KW = ceil(tasks / 64) wavefronts covers a whole row,
// wavefront w owning tasks 64 w + lane, and every lane keeps its task's activation (all B rows:
// codes and scales, and the terms that do not depend on the weight row) in registers for the whole
// launch, so the activation is read once per wavefront rather than once per weight row. The
// workgroup walks batches of R weight rows, the next two batches' weights in flight; per row a
// lane forms its task's B products (the int32 dot sums exact, as ggml's, then fp32 scaling), the
// wavefront reduce-scatters the batch's R x B products (wave_reduce_scatter), and the KW slices'
// sums meet in LDS, added in slice order by the first wavefront, which stores the batch. Rows
// past N read zeros (past the buffer's end) and are not stored; lanes past the row read the next
// row's weights, which their zero activation scale cancels.
//
// Per task and batch row b (x: Q8_0 / Q8_K codes of the task's values, d_x their scale):
//   Q4_0: ((sum q x) d_x - 8 (sum x) d_x) d_w (q the stored 0..15 code);  Q8_0: (sum q x) d_x d_w
//   Q4_K / Q5_K: (sc0 s0 + sc1 s1) d d_x - dmin (m0 bs0 + m1 bs1) d_x, s0 / s1 the task's two
//     16-value dots with sub-blocks 2c / 2c + 1 and bs0 / bs1 the matching Q8_K bsums.
template <int TYPE>
struct KsFmt {
    static constexpr bool KQ = TYPE == T_Q4_K || TYPE == T_Q5_K;
    static constexpr int WV = TYPE == T_Q8_0 ? 2 : TYPE == T_Q5_K ? 3 : KQ ? 2 : 1;  // 16-byte loads per row
};

struct KsArgs {
    const uint8_t * w;      // Q4_0 / Q8_0: packed codes; K-quants: the packed weight (nibbles first)
    const uint16_t * wd;    // Q4_0 / Q8_0: packed fp16 scales
    const int8_t * xc;      // activation codes [B][K]
    const float2 * xm;      // Q8_0 activation: (d, code sum) [B][K / 32]
    const int16_t * xbs;    // Q8_K activation: bsums [B][K / 16]
    const float * xd;       // Q8_K activation: d [B][K / 256]
    const float * x;        // FQ: the f32 activation row itself (one row, quantized in the kernel)
    float * y;
    const float * res;
    int N, ntask, ldy;      // ntask: tasks per row (K / 32)
    uint32_t kq_qh, kq_hdr, kq_bytes;  // K-quants: the fifth bits' and headers' offsets, the weight's size
};

template <int TYPE, int B, int R, bool FQ = false>
__global__ __launch_bounds__(512) void k_gemv_ks(const KsArgs a) {
    using F = KsFmt<TYPE>;
    static_assert(!FQ || (B == 1 && F::KQ), "the activation is quantized in the kernel for one K-quant row");
    constexpr int WV = F::WV;
    constexpr int BP = B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;  // B padded to a power of two
    constexpr int LG = BP == 1 ? 0 : BP == 2 ? 1 : BP == 4 ? 2 : 3;
    __shared__ float part[2][8][R][BP];  // [batch parity][slice][row][b]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, KW = blockDim.x >> 6;
    const int K = a.ntask * QK;
    const int t = wave * 64 + lane;  // this lane's task
    const bool live = t < a.ntask;
    const int tt = live ? t : 0;
    const int nb = a.ntask;                       // Q4_0 / Q8_0: blocks per row
    const int sb = tt >> 3, c = (tt >> 1) & 3, h = tt & 1;  // K-quants: super-block, chunk, half
    const uint32_t csh = 16u * (uint32_t) (c & 1);         // the chunk's scale bytes within their words
    const bool chi = c >= 2;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.w), 0,
        (int) (F::KQ ? (size_t) a.kq_bytes : (size_t) a.N * nb * (TYPE == T_Q4_0 ? 16 : 32)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(a.wd), 0, F::KQ ? 0 : (int) (((size_t) a.N * nb + 1) / 2 * 4), 0x00020000);
    const int nbatch = (a.N + R - 1) / R;
    const int G = gridDim.x;

    // The activation first, then the first two batches' weights: the loads complete in issue
    // order, so at every batch the wait is for the older batch only.
    int4 xa[B], xb[B];  // the task's 32 codes (K-quants: xa = sub-block 2c's 16, xb = 2c + 1's)
    float xs[B];        // d_x (Q4_0 / Q8_0) or d_x of the super-block (K-quants)
    float xo[B], xo2[B];  // Q4_0: -8 (sum x) d_x; K-quants: bs0 d_x, bs1 d_x
    float2 xmv[B];
    int bsv[B][2];
#pragma unroll
    for (int b = 0; b < B; b++) {
        const int8_t * xr = a.xc + (size_t) b * K;
        if constexpr (FQ) {
            // ggml's quantize_row_q8_K (as k_act_q8_K) of the super-block, whose 256 values are
            // the 32 of each of its 8 lanes (consecutive, aligned): max = the signed value of the
            // first largest |x|, iscale = -127 / max, q = min(127, rint(iscale x)), d = 1 / iscale,
            // zeros for an all-zero block; this lane's two bsums are the sums of its two 16s.
#pragma clang fp contract(off)
            const int il = 64 * c + 16 * h;
            const float * xf = a.x + sb * QKK + il;
            float vv[32];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 lo4 = *reinterpret_cast<const float4 *>(xf + 4 * k);
                const float4 hi4 = *reinterpret_cast<const float4 *>(xf + 32 + 4 * k);
                vv[4 * k] = lo4.x;
                vv[4 * k + 1] = lo4.y;
                vv[4 * k + 2] = lo4.z;
                vv[4 * k + 3] = lo4.w;
                vv[16 + 4 * k] = hi4.x;
                vv[16 + 4 * k + 1] = hi4.y;
                vv[16 + 4 * k + 2] = hi4.z;
                vv[16 + 4 * k + 3] = hi4.w;
            }
            float ax = 0.0f, mx = 0.0f;
            int idx = 1 << 30;
#pragma unroll
            for (int j = 0; j < 32; j++) {  // in index order: the 16 of sub-block 2c, then of 2c + 1
                if (fabsf(vv[j]) > ax) {
                    ax = fabsf(vv[j]);
                    mx = vv[j];
                    idx = il + (j < 16 ? j : 16 + j);
                }
            }
            auto take = [&](float ax2, float mx2, int idx2) {
                if (ax2 > ax || (ax2 == ax && idx2 < idx)) {
                    ax = ax2;
                    mx = mx2;
                    idx = idx2;
                }
            };
            {
                const float a1 = lane_pair<1>(ax), m1 = lane_pair<1>(mx);
                const int i1 = lane_pair_i<1>(idx);
                take(a1, m1, i1);
                const float a2 = lane_pair<2>(ax), m2 = lane_pair<2>(mx);
                const int i2 = lane_pair_i<2>(idx);
                take(a2, m2, i2);
                const float a4 = lane_pair<4>(ax), m4 = lane_pair<4>(mx);
                const int i4 = lane_pair_i<4>(idx);
                take(a4, m4, i4);
            }
            int qv[32];
            float dq = 0.0f;
            if (ax != 0.0f) {
                const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const int r = (int) __builtin_rintf(iscale * vv[j]);
                    qv[j] = r < 127 ? r : 127;
                }
                dq = __fdiv_rn(1.0f, iscale);
            } else {
#pragma unroll
                for (int j = 0; j < 32; j++) qv[j] = 0;
            }
            int pk[8], s0 = 0, s1 = 0;
#pragma unroll
            for (int k = 0; k < 8; k++)
                pk[k] = (qv[4 * k] & 0xff) | ((qv[4 * k + 1] & 0xff) << 8) | ((qv[4 * k + 2] & 0xff) << 16) |
                        ((qv[4 * k + 3] & 0xff) << 24);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                s0 += qv[j];
                s1 += qv[16 + j];
            }
            xa[b] = make_int4(pk[0], pk[1], pk[2], pk[3]);
            xb[b] = make_int4(pk[4], pk[5], pk[6], pk[7]);
            bsv[b][0] = s0;
            bsv[b][1] = s1;
            xmv[b].x = dq;
        } else if constexpr (F::KQ) {
            const int e = sb * QKK + 64 * c + 16 * h;
            xa[b] = *reinterpret_cast<const int4 *>(xr + e);
            xb[b] = *reinterpret_cast<const int4 *>(xr + e + 32);
            const int16_t * bs = a.xbs + (size_t) b * (K / 16) + sb * 16 + 4 * c + h;
            bsv[b][0] = bs[0];
            bsv[b][1] = bs[2];
            xmv[b].x = a.xd[(size_t) b * (K / QKK) + sb];
        } else {
            const int4 * xp = reinterpret_cast<const int4 *>(xr + (size_t) tt * QK);
            xa[b] = xp[0];
            xb[b] = xp[1];
            xmv[b] = a.xm[(size_t) b * nb + tt];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 w[R][WV], wn[R][WV];
    uint32_t d[R], dn[R];
    auto load = [&](int tb, uint4 (&wv)[R][WV], uint32_t (&dv)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            if constexpr (F::KQ) {
                // header (d, dmin, scales), the half chunk's 16 code bytes (piece tt of the row's
                // nibbles: consecutive lanes, consecutive pieces), [Q5_K: the half's 16 qh bytes];
                // rows past N read zeros (an offset past the weight)
                const int row = tb * R + r;
                const uint32_t bi = (uint32_t) row * (uint32_t) (a.ntask / 8) + (uint32_t) sb;
                const bool rin = row < a.N;
                const uint32_t offs[3] = {rin ? a.kq_hdr + 16u * bi : 0x80000000u,
                                          rin ? 16u * ((uint32_t) row * (uint32_t) a.ntask + (uint32_t) tt) : 0x80000000u,
                                          rin ? a.kq_qh + 32u * bi + 16u * (uint32_t) h : 0x80000000u};
                const auto hq = __builtin_amdgcn_raw_buffer_load_b128(rq, offs[0], 0, 0);  // shared by 8 lanes
                wv[r][0] = make_uint4(hq[0], hq[1], hq[2], hq[3]);
#pragma unroll
                for (int v = 1; v < WV; v++) {
                    const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, offs[v], 0, 2);
                    wv[r][v] = make_uint4(q[0], q[1], q[2], q[3]);
                }
                dv[r] = 0u;
            } else {
                const uint32_t o = (uint32_t) (tb * R + r) * (uint32_t) nb + (uint32_t) t;
#pragma unroll
                for (int v = 0; v < WV; v++) {
                    const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, (o * WV + v) * 16u, 0, 2);
                    wv[r][v] = make_uint4(q[0], q[1], q[2], q[3]);
                }
                dv[r] = __builtin_amdgcn_raw_buffer_load_b32(rd, (o >> 1) * 4u, 0, 0);
            }
        }
    };
    int tb = blockIdx.x;
    load(tb, w, d);
    __builtin_amdgcn_sched_barrier(0);
    load(tb + G, wn, dn);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < B; b++) {
        xs[b] = live ? xmv[b].x : 0.0f;
        if constexpr (F::KQ) {
            xo[b] = (float) bsv[b][0] * xs[b];
            xo2[b] = (float) bsv[b][1] * xs[b];
        } else {
            xo[b] = TYPE == T_Q4_0 ? (float) (-8 * __float_as_int(xmv[b].y)) * xs[b] : 0.0f;
            xo2[b] = 0.0f;
        }
    }

    constexpr int V = R * BP, LV = LG + (R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4);
    static_assert(V <= 64 && (1 << LV) == V, "R and B padded: a power of two up to 64 products");
    // clamp on the first dot of a chain: the three-operand form with a zero start (no register
    // set to zero first); the sums never come near the int32 limits
    auto dot16 = [](const int (&q)[4], const int4 x) {
        int s = __builtin_amdgcn_sdot4(q[0], x.x, 0, true);
        s = sdot4(q[1], x.y, s);
        s = sdot4(q[2], x.z, s);
        return sdot4(q[3], x.w, s);
    };
    auto batch = [&](int tbi, const uint4 (&wv)[R][WV], const uint32_t (&dv)[R], int par) {
        float v[V];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int lo[4], hi[4];
            const uint32_t q[4] = {wv[r][F::KQ ? 1 : 0].x, wv[r][F::KQ ? 1 : 0].y, wv[r][F::KQ ? 1 : 0].z,
                                   wv[r][F::KQ ? 1 : 0].w};
            if constexpr (TYPE == T_Q8_0) {
                lo[0] = (int) wv[r][0].x;
                lo[1] = (int) wv[r][0].y;
                lo[2] = (int) wv[r][0].z;
                lo[3] = (int) wv[r][0].w;
                hi[0] = (int) wv[r][1].x;
                hi[1] = (int) wv[r][1].y;
                hi[2] = (int) wv[r][1].z;
                hi[3] = (int) wv[r][1].w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo[j] = (int) (q[j] & 0x0F0F0F0Fu);
                    hi[j] = (int) ((q[j] >> 4) & 0x0F0F0F0Fu);
                }
            }
            if constexpr (TYPE == T_Q5_K) {  // the fifth bits: bit 2c of qh[l] (sub-block 2c), 2c + 1
                const uint32_t qh[4] = {wv[r][2].x, wv[r][2].y, wv[r][2].z, wv[r][2].w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo[j] |= (int) (((qh[j] >> (2 * c)) & 0x01010101u) << 4);
                    hi[j] |= (int) (((qh[j] >> (2 * c + 1)) & 0x01010101u) << 4);
                }
            }
            if constexpr (F::KQ) {
                // The 6-bit scales and mins of sub-blocks 2c and 2c + 1 (ggml's get_scale_min_k4),
                // both at once: header bytes 4-15 hold scales[12]; c < 2: sc = scales[2c..2c+1] & 63,
                // m = scales[2c+4..2c+5] & 63; c >= 2: sc = (scales[2c+4..] & 15) | (scales[2c-4..] >> 6) << 4,
                // m = (scales[2c+4..] >> 4) | (scales[2c..] >> 6) << 4.
                const uint4 hd = wv[r][0];
                const uint32_t A = hd.y >> csh, M = hd.z >> csh, H = hd.w >> csh;
                // chunks 2, 3 take the high form; chosen by a mask (a select here became a branch)
                const uint32_t chim = chi ? 0xFFFFFFFFu : 0u;
                const uint32_t scp = (chim & ((H & 0x0F0Fu) | ((A >> 2) & 0x3030u))) | (~chim & (A & 0x3F3Fu));
                const uint32_t mp = (chim & (((H >> 4) & 0x0F0Fu) | ((M >> 2) & 0x3030u))) | (~chim & (M & 0x3F3Fu));
                const int sc0 = (int) (scp & 0xFFu), sc1 = (int) ((scp >> 8) & 0xFFu);
                const int m0 = (int) (mp & 0xFFu), m1 = (int) ((mp >> 8) & 0xFFu);
                const float dd = h2f((uint16_t) (hd.x & 0xffff)), dmin = h2f((uint16_t) (hd.x >> 16));
                const float fm0 = (float) m0 * dmin, fm1 = (float) m1 * dmin;
#pragma unroll
                for (int b = 0; b < BP; b++) {
                    if (b < B) {
                        const int isc = sc0 * dot16(lo, xa[b]) + sc1 * dot16(hi, xb[b]);
                        const float fmin = __builtin_fmaf(fm0, xo[b], fm1 * xo2[b]);
                        v[r * BP + b] = __builtin_fmaf((float) isc * dd, xs[b], -fmin);
                    } else {
                        v[r * BP + b] = 0.0f;
                    }
                }
            } else {
                // scale index row * nb + t: its parity picks the half (t's parity is the lane's)
                const int row = min(tbi * R + r, a.N - 1);
                const uint32_t sh = (uint32_t) (((lane ^ (row & nb)) & 1) << 4);
                const float dw = h2f((uint16_t) (dv[r] >> sh));
#pragma unroll
                for (int b = 0; b < BP; b++) {
                    if (b < B) {
                        int s = dot16(lo, xa[b]);
                        s = sdot4(hi[0], xb[b].x, s);
                        s = sdot4(hi[1], xb[b].y, s);
                        s = sdot4(hi[2], xb[b].z, s);
                        s = sdot4(hi[3], xb[b].w, s);
                        v[r * BP + b] = __builtin_fmaf((float) s, xs[b], xo[b]) * dw;
                    } else {
                        v[r * BP + b] = 0.0f;
                    }
                }
            }
        }
        wave_reduce_scatter<V>(v);
        if ((lane & ((64 >> LV) - 1)) == 0) {
            const int idx = lane >> (6 - LV);
            part[par][wave][idx / BP][idx % BP] = v[0];
        }
        // LDS writes complete and every slice's written (the weight loads in flight are not waited for)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (wave == 0 && lane < R * BP) {
            const int r = lane / BP, b = lane % BP, row = tbi * R + r;
            float sum = part[par][0][r][b];
            for (int k = 1; k < KW; k++) sum += part[par][k][r][b];
            if (b < B && row < a.N) {
                const size_t o = (size_t) b * a.ldy + row;
                a.y[o] = a.res ? sum + a.res[o] : sum;
            }
        }
    };
    while (tb < nbatch) {
        batch(tb, w, d, 0);
        load(tb + 2 * G, w, d);
        tb += G;
        if (tb >= nbatch) break;
        batch(tb, wn, dn, 1);
        load(tb + 2 * G, wn, dn);
        tb += G;
    }
}

// ----------------------------------------------------------------------------- Q4_K kernel

// Lane task = (super-block, 64-value chunk): 4 tasks per super-block, NBL tasks per lane per
// pass. Per task: the 16-byte header (d, dmin, packed scales), 32 bytes of nibbles.
template <int B, int R, int NBL>
__global__ __launch_bounds__(256) void k_gemv_q4_K(const uint8_t * __restrict__ w, const int8_t * __restrict__ xc,
                                                   const int16_t * __restrict__ xbs, const float * __restrict__ xd,
                                                   float * y, const float * res, int N, int nsb, int ldy) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int K = nsb * QKK;
    const int ntask = nsb * 4;
    const KqRegions L = kq_regions(T_Q4_K, (int64_t) N * nsb);
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = 0.0f;

    for (int base = 0; base < ntask; base += 64 * NBL) {
        uint4 hdr[NBL][R], qa[NBL][R], qb[NBL][R];
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t < ntask) {
                const int sb = t >> 2, c = t & 3;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + r, N - 1);
                    const size_t bi = (size_t) row * nsb + sb;
                    const uint4 * q = reinterpret_cast<const uint4 *>(w + L.qs + bi * 128);
                    hdr[i][r] = reinterpret_cast<const uint4 *>(w + L.hdr)[bi];
                    qa[i][r] = q[2 * c];
                    qb[i][r] = q[2 * c + 1];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t >= ntask) break;
            const int sb = t >> 2, c = t & 3;
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) sb * QKK + 64 * c);
                const int4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
                const int2 bs = *reinterpret_cast<const int2 *>(xbs + (size_t) b * (K / 16) + sb * 16 + 4 * c);
                const int bs01 = (int) (int16_t) (bs.x & 0xffff) + (int) (int16_t) (bs.x >> 16);
                const int bs23 = (int) (int16_t) (bs.y & 0xffff) + (int) (int16_t) (bs.y >> 16);
                const float dx = xd[(size_t) b * nsb + sb];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t sc3[3] = {hdr[i][r].y, hdr[i][r].z, hdr[i][r].w};
                    int sc0, m0, sc1, m1, lo, hi;
                    scale_min_k4_w(2 * c, sc3, sc0, m0);
                    scale_min_k4_w(2 * c + 1, sc3, sc1, m1);
                    dot_q4_K_chunk(qa[i][r], qb[i][r], x0, x1, x2, x3, lo, hi);
                    const int isc = sc0 * lo + sc1 * hi;
                    const int imin = m0 * bs01 + m1 * bs23;
                    const float dw = h2f((uint16_t) (hdr[i][r].x & 0xffff)) * dx;
                    const float dm = h2f((uint16_t) (hdr[i][r].x >> 16)) * dx;
                    acc[r][b] += dw * (float) isc - dm * (float) imin;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float v = wave_sum(acc[r][b]);
            if (lane == r * B + b && row0 + r < N) {
                const size_t o = (size_t) b * ldy + row0 + r;
                y[o] = res ? v + res[o] : v;
            }
        }
}

// ------------------------------------------------------------------- Q5_K / Q6_K kernels

// Q5_K: the Q4_K task walk (super-block, 64-value chunk) with the 32 qh bytes loaded per task.
template <int B, int R, int NBL>
__global__ __launch_bounds__(256) void k_gemv_q5_K(const uint8_t * __restrict__ w, const int8_t * __restrict__ xc,
                                                   const int16_t * __restrict__ xbs, const float * __restrict__ xd,
                                                   float * y, const float * res, int N, int nsb, int ldy) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int K = nsb * QKK;
    const int ntask = nsb * 4;
    const KqRegions L = kq_regions(T_Q5_K, (int64_t) N * nsb);
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = 0.0f;

    for (int base = 0; base < ntask; base += 64 * NBL) {
        uint4 hdr[NBL][R], ha[NBL][R], hb[NBL][R], qa[NBL][R], qb[NBL][R];
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t < ntask) {
                const int sb = t >> 2, c = t & 3;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + r, N - 1);
                    const size_t bi = (size_t) row * nsb + sb;
                    const uint4 * q = reinterpret_cast<const uint4 *>(w + L.qs + bi * 128);
                    const uint4 * qh = reinterpret_cast<const uint4 *>(w + L.qh + bi * 32);
                    hdr[i][r] = reinterpret_cast<const uint4 *>(w + L.hdr)[bi];
                    ha[i][r] = qh[0];
                    hb[i][r] = qh[1];
                    qa[i][r] = q[2 * c];
                    qb[i][r] = q[2 * c + 1];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t >= ntask) break;
            const int sb = t >> 2, c = t & 3;
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) sb * QKK + 64 * c);
                const int4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
                const int2 bs = *reinterpret_cast<const int2 *>(xbs + (size_t) b * (K / 16) + sb * 16 + 4 * c);
                const int bs01 = (int) (int16_t) (bs.x & 0xffff) + (int) (int16_t) (bs.x >> 16);
                const int bs23 = (int) (int16_t) (bs.y & 0xffff) + (int) (int16_t) (bs.y >> 16);
                const float dx = xd[(size_t) b * nsb + sb];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t sc3[3] = {hdr[i][r].y, hdr[i][r].z, hdr[i][r].w};
                    int sc0, m0, sc1, m1, lo, hi;
                    scale_min_k4_w(2 * c, sc3, sc0, m0);
                    scale_min_k4_w(2 * c + 1, sc3, sc1, m1);
                    dot_q5_K_chunk(qa[i][r], qb[i][r], ha[i][r], hb[i][r], c, x0, x1, x2, x3, lo, hi);
                    const int isc = sc0 * lo + sc1 * hi;
                    const int imin = m0 * bs01 + m1 * bs23;
                    const float dw = h2f((uint16_t) (hdr[i][r].x & 0xffff)) * dx;
                    const float dm = h2f((uint16_t) (hdr[i][r].x >> 16)) * dx;
                    acc[r][b] += dw * (float) isc - dm * (float) imin;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float v = wave_sum(acc[r][b]);
            if (lane == r * B + b && row0 + r < N) {
                const size_t o = (size_t) b * ldy + row0 + r;
                y[o] = res ? v + res[o] : v;
            }
        }
}

// Q6_K (packed: ql / qh / scales / d fields): lane task = (super-block, half hh, ql
// part jj), 4 tasks per super-block: 32 ql + 32 qh bytes, the half's 8 scale bytes and d.
template <int B, int R, int NBL>
__global__ __launch_bounds__(256) void k_gemv_q6_K(const uint8_t * __restrict__ wqs, const uint16_t * __restrict__ wd,
                                                   const int8_t * __restrict__ xc, const int16_t * __restrict__ xbs,
                                                   const float * __restrict__ xd, float * y, const float * res, int N,
                                                   int nsb, int ldy) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int K = nsb * QKK;
    const int ntask = nsb * 4;
    const Q6Regions R6 = q6_regions((int64_t) N * nsb);
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = 0.0f;

    for (int base = 0; base < ntask; base += 64 * NBL) {
        uint4 la[NBL][R], lb[NBL][R], ha[NBL][R], hb[NBL][R];
        uint2 sc[NBL][R];
        uint32_t dw[NBL][R];
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t < ntask) {
                const int sb = t >> 2, hh = (t >> 1) & 1, jj = t & 1;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + r, N - 1);
                    const size_t blk = (size_t) row * nsb + sb;
                    auto piece = [&](int k) { return *reinterpret_cast<const uint4 *>(wqs + q6_off(R6, blk, 16 * k)); };
                    la[i][r] = piece(4 * hh + 2 * jj);
                    lb[i][r] = piece(4 * hh + 2 * jj + 1);
                    ha[i][r] = piece(8 + 2 * hh);
                    hb[i][r] = piece(9 + 2 * hh);
                    sc[i][r] = *reinterpret_cast<const uint2 *>(wqs + q6_off(R6, blk, 192 + 8 * hh));
                    dw[i][r] = wd[blk];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = base + lane + 64 * i;
            if (t >= ntask) break;
            const int sb = t >> 2, hh = (t >> 1) & 1, jj = t & 1;
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int8_t * xb = xc + (size_t) b * K + (size_t) sb * QKK + 128 * hh + 32 * jj;
                const int4 * xp = reinterpret_cast<const int4 *>(xb);
                const int4 * xq = reinterpret_cast<const int4 *>(xb + 64);
                const int4 x0 = xp[0], x1 = xp[1], x2 = xq[0], x3 = xq[1];
                const uint32_t * bsw = reinterpret_cast<const uint32_t *>(xbs + (size_t) b * (K / 16) + sb * 16 + 8 * hh + 2 * jj);
                const uint32_t bs01 = bsw[0], bs23 = bsw[2];
                const float dx = xd[(size_t) b * nsb + sb];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int dd[4];
                    dot_q6_K_task(la[i][r], lb[i][r], ha[i][r], hb[i][r], jj, x0, x1, x2, x3, dd);
                    const int is = isum_q6_K_task(dd, sc[i][r], jj, bs01, bs23);
                    acc[r][b] += (h2f((uint16_t) dw[i][r]) * dx) * (float) is;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float v = wave_sum(acc[r][b]);
            if (lane == r * B + b && row0 + r < N) {
                const size_t o = (size_t) b * ldy + row0 + r;
                y[o] = res ? v + res[o] : v;
            }
        }
}

// -------------------------------------------------------------------- integer-sum dumps

// The int32 block sums the GEMV kernels form, written out for bit-exact comparison:
// Q4_0 / Q8_0: out[b][n][blk]; Q4_K: out[b][n][sb][10] = 8 sub-block dots, isc, imin.
__global__ void k_isums_q0(int type, const uint8_t * wqs, const uint16_t *, const int8_t * xc, const float2 * xm,
                           int32_t * out, int N, int nb, int B) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) B * N * nb) return;
    const int blk = (int) (t % nb);
    const int n = (int) ((t / nb) % N);
    const int b = (int) (t / ((int64_t) nb * N));
    const int K = nb * QK;
    const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) blk * QK);
    const size_t o = (size_t) n * nb + blk;
    int s;
    if (type == T_Q4_0) {
        s = dot_q4_0(reinterpret_cast<const uint4 *>(wqs)[o], xp[0], xp[1], __float_as_int(xm[(size_t) b * nb + blk].y));
    } else {
        const uint4 * q = reinterpret_cast<const uint4 *>(wqs) + 2 * o;
        s = dot_q8_0(q[0], q[1], xp[0], xp[1]);
    }
    out[t] = s;
}

__global__ void k_isums_q4_K(const uint8_t * w, const int8_t * xc, const int16_t * xbs, int32_t * out, int N, int nsb,
                             int B) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) B * N * nsb) return;
    const int sb = (int) (t % nsb);
    const int n = (int) ((t / nsb) % N);
    const int b = (int) (t / ((int64_t) nsb * N));
    const int K = nsb * QKK;
    const KqRegions L = kq_regions(T_Q4_K, (int64_t) N * nsb);
    const size_t bi = (size_t) n * nsb + sb;
    const uint4 * p = reinterpret_cast<const uint4 *>(w + L.qs + bi * 128);  // the nibbles, 2 x 16 B per chunk
    const uint4 hdr = reinterpret_cast<const uint4 *>(w + L.hdr)[bi];
    const uint32_t sc3[3] = {hdr.y, hdr.z, hdr.w};
    int32_t * o = out + t * 10;
    int isc = 0, imin = 0;
    for (int c = 0; c < 4; c++) {
        const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) sb * QKK + 64 * c);
        int lo, hi, sc0, m0, sc1, m1;
        dot_q4_K_chunk(p[2 * c], p[2 * c + 1], xp[0], xp[1], xp[2], xp[3], lo, hi);
        scale_min_k4_w(2 * c, sc3, sc0, m0);
        scale_min_k4_w(2 * c + 1, sc3, sc1, m1);
        const int16_t * bs = xbs + (size_t) b * (K / 16) + sb * 16 + 4 * c;
        o[2 * c] = lo;
        o[2 * c + 1] = hi;
        isc += sc0 * lo + sc1 * hi;
        imin += m0 * (bs[0] + bs[1]) + m1 * (bs[2] + bs[3]);
    }
    o[8] = isc;
    o[9] = imin;
}

// Q5_K: out[b][n][sb][10] as Q4_K (q = the 5-bit code).
__global__ void k_isums_q5_K(const uint8_t * w, const int8_t * xc, const int16_t * xbs, int32_t * out, int N, int nsb,
                             int B) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) B * N * nsb) return;
    const int sb = (int) (t % nsb);
    const int n = (int) ((t / nsb) % N);
    const int b = (int) (t / ((int64_t) nsb * N));
    const int K = nsb * QKK;
    const KqRegions L = kq_regions(T_Q5_K, (int64_t) N * nsb);
    const size_t bi = (size_t) n * nsb + sb;
    const uint4 * p = reinterpret_cast<const uint4 *>(w + L.qs + bi * 128);   // the nibbles
    const uint4 * ph = reinterpret_cast<const uint4 *>(w + L.qh + bi * 32);   // the fifth bits
    const uint4 hdr = reinterpret_cast<const uint4 *>(w + L.hdr)[bi];
    const uint32_t sc3[3] = {hdr.y, hdr.z, hdr.w};
    int32_t * o = out + t * 10;
    int isc = 0, imin = 0;
    for (int c = 0; c < 4; c++) {
        const int4 * xp = reinterpret_cast<const int4 *>(xc + (size_t) b * K + (size_t) sb * QKK + 64 * c);
        int lo, hi, sc0, m0, sc1, m1;
        dot_q5_K_chunk(p[2 * c], p[2 * c + 1], ph[0], ph[1], c, xp[0], xp[1], xp[2], xp[3], lo, hi);
        scale_min_k4_w(2 * c, sc3, sc0, m0);
        scale_min_k4_w(2 * c + 1, sc3, sc1, m1);
        const int16_t * bs = xbs + (size_t) b * (K / 16) + sb * 16 + 4 * c;
        o[2 * c] = lo;
        o[2 * c + 1] = hi;
        isc += sc0 * lo + sc1 * hi;
        imin += m0 * (bs[0] + bs[1]) + m1 * (bs[2] + bs[3]);
    }
    o[8] = isc;
    o[9] = imin;
}

// Q6_K: out[b][n][sb][17] = the 16 sub-block sums of (q - 32) * x, then sum_j sc_j * those.
__global__ void k_isums_q6_K(const uint8_t * wqs, const int8_t * xc, const int16_t * xbs, int32_t * out, int N,
                             int nsb, int B) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) B * N * nsb) return;
    const int sb = (int) (t % nsb);
    const int n = (int) ((t / nsb) % N);
    const int b = (int) (t / ((int64_t) nsb * N));
    const int K = nsb * QKK;
    const size_t blk = (size_t) n * nsb + sb;
    const Q6Regions R6 = q6_regions((int64_t) N * nsb);
    uint4 p[13];  // ggml's first 208 bytes of the super-block, from their fields
    for (int k = 0; k < 13; k++) p[k] = *reinterpret_cast<const uint4 *>(wqs + q6_off(R6, blk, 16 * k));
    int32_t * o = out + t * 17;
    int total = 0;
    for (int task = 0; task < 4; task++) {
        const int hh = task >> 1, jj = task & 1;
        const int8_t * xb = xc + (size_t) b * K + (size_t) sb * QKK + 128 * hh + 32 * jj;
        const int4 * xp = reinterpret_cast<const int4 *>(xb);
        const int4 * xq = reinterpret_cast<const int4 *>(xb + 64);
        int dd[4];
        dot_q6_K_task(p[4 * hh + 2 * jj], p[4 * hh + 2 * jj + 1], p[8 + 2 * hh], p[9 + 2 * hh], jj, xp[0], xp[1], xq[0],
                      xq[1], dd);
        const int16_t * bs = xbs + (size_t) b * (K / 16) + sb * 16;
        const int s0 = 8 * hh + 2 * jj;
        const int sub[4] = {s0, s0 + 1, s0 + 4, s0 + 5};
        for (int k = 0; k < 4; k++) o[sub[k]] = dd[k] - 32 * bs[sub[k]];
        const uint2 sc8 = *reinterpret_cast<const uint2 *>(wqs + q6_off(R6, blk, 192 + 8 * hh));
        const uint32_t * bsw = reinterpret_cast<const uint32_t *>(bs + s0);
        total += isum_q6_K_task(dd, sc8, jj, bsw[0], bsw[2]);
    }
    o[16] = total;
}

// -------------------------------------------------------------------------------- dispatch

// Compute units of the current device (cached per thread and device).
int cu_count() {
    static thread_local int dev = -1, cus = 0;
    int d = 0;
    check_hip(hipGetDevice(&d), "hipGetDevice");
    if (d != dev) {
        RelaxedCapture relaxed;
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d), "CU count");
        dev = d;
    }
    return cus;
}

namespace {

// Rows per wavefront and blocks-per-lane per pass, by batch size and row length.
constexpr int kR = 2;
constexpr int kRp = 2;        // rows per wavefront step of the persistent kernel
constexpr int kWgPerCu = 4;   // persistent grid: workgroups per CU

unsigned persistent_grid(int N, int waves_per_wg, int wg_per_cu) {
    const int groups = (N + kRp - 1) / kRp;
    return (unsigned) std::max(1, std::min((groups + waves_per_wg - 1) / waves_per_wg, cu_count() * wg_per_cu));
}

template <int TYPE, int B, int NBL>
void run_p(const uint8_t * w, const WeightLayout & L, const int8_t * xc, const float2 * xm, float * y, const float * res, int N, int nb,
           int ldy, hipStream_t s) {
    k_gemv_p<TYPE, B, kRp, NBL><<<persistent_grid(N, 4, kWgPerCu), 256, 0, s>>>(
        w + L.qs, (const uint16_t *) (w + L.d), xc, xm, y, res, N, nb, ldy);
}

int pick_nbl(int tasks) {  // tasks per row (blocks, or Q4_K chunks)
    const int per_lane = (tasks + 63) / 64;
    if (per_lane <= 1) return 1;
    if (per_lane <= 2) return 2;
    if (per_lane <= 4) return 4;
    return 8;
}

template <int TYPE, int B, int NBL>
void run_q0(const uint8_t * w, const WeightLayout & L, const int8_t * xc, const float2 * xm, float * y, const float * res,
            int N, int nb, int ldy, hipStream_t s) {
    const unsigned grid = (unsigned) ((N + 4 * kR - 1) / (4 * kR));
    k_gemv_q0<TYPE, B, kR, NBL><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), xc, xm, y, res, N, nb, ldy);
}

// The K-sliced kernel (k_gemv_ks) for batches of 2..8 rows: ceil(tasks / 64) wavefronts per
// workgroup, as many workgroups as are resident at once (at most), each with the same number of
// row batches.
template <int TYPE, int B, int R, bool FQ = false>
void run_ks(const KsArgs & a, hipStream_t s) {
    const int kw = (a.ntask + 63) / 64;
    static thread_local int occ[9] = {0};  // resident workgroups per CU, by wavefronts per workgroup
    if (occ[kw] == 0) {
        RelaxedCapture relaxed;
        check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ[kw], reinterpret_cast<const void *>(&k_gemv_ks<TYPE, B, R, FQ>),
                                                               kw * 64, 0),
                  "gemv occupancy");
        occ[kw] = std::max(occ[kw], 1);
    }
    const int nbatch = (a.N + R - 1) / R, maxg = cu_count() * occ[kw];
    const int per = (nbatch + maxg - 1) / maxg;
    const unsigned grid = (unsigned) ((nbatch + per - 1) / per);
    k_gemv_ks<TYPE, B, R, FQ><<<grid, kw * 64, 0, s>>>(a);
}

// Rows per batch of the K-sliced kernel: R B products reduce-scattered at once (measured: Q4_0 /
// Q8_0 at B <= 2 best with 8, the rest with 4).
template <int TYPE, int B>
void run_ks_b(const KsArgs & a, hipStream_t s) {
    run_ks<TYPE, B, (B <= 2 && !KsFmt<TYPE>::KQ ? 8 : 4)>(a, s);
}

template <int TYPE>
void run_ks_t(int B, const KsArgs & a, hipStream_t s) {
    switch (B) {
        case 1: return run_ks<TYPE, 1, 4>(a, s);
        case 2: return run_ks_b<TYPE, 2>(a, s);
        case 3: return run_ks_b<TYPE, 3>(a, s);
        case 4: return run_ks_b<TYPE, 4>(a, s);
        case 5: return run_ks_b<TYPE, 5>(a, s);
        case 6: return run_ks_b<TYPE, 6>(a, s);
        case 7: return run_ks_b<TYPE, 7>(a, s);
        default: return run_ks_b<TYPE, 8>(a, s);
    }
}

// The K-sliced kernel takes rows of up to 512 tasks (K <= 16384) in batches of 2..8 rows (K-quants:
// 1..8, the one-row case as the kernel that quantizes the row itself).
bool ks_fits(int type, int64_t K, int64_t B) {
    return B >= (is_kquant(type) ? 1 : 2) && B <= 8 && K % QK == 0 && K / QK <= 512 &&
           (type == T_Q4_0 || type == T_Q8_0 || ((type == T_Q4_K || type == T_Q5_K) && K % QKK == 0));
}

template <int TYPE, int B>
void run_q0_nbl(int nbl, const uint8_t * w, const WeightLayout & L, const int8_t * xc, const float2 * xm, float * y,
                const float * res, int N, int nb, int ldy, hipStream_t s) {
    if constexpr (B <= 4) {  // rows of up to 128 blocks: the persistent kernel
        if (nbl == 1) return run_p<TYPE, B, 1>(w, L, xc, xm, y, res, N, nb, ldy, s);
        if (nbl == 2) return run_p<TYPE, B, 2>(w, L, xc, xm, y, res, N, nb, ldy, s);
    }
    if (nbl == 8) nbl = 4;  // long rows: two passes of 256 blocks measured faster than one of 512
    switch (nbl) {
        case 1: run_q0<TYPE, B, 1>(w, L, xc, xm, y, res, N, nb, ldy, s); break;
        case 2: run_q0<TYPE, B, 2>(w, L, xc, xm, y, res, N, nb, ldy, s); break;
        case 4: run_q0<TYPE, B, 4>(w, L, xc, xm, y, res, N, nb, ldy, s); break;
        default: run_q0<TYPE, B, 8>(w, L, xc, xm, y, res, N, nb, ldy, s); break;
    }
}

template <int B, int NBL>
void run_q4k(const uint8_t * w, const int8_t * xc, const int16_t * xbs, const float * xd, float * y, const float * res,
             int N, int nsb, int ldy, hipStream_t s) {
    const unsigned grid = (unsigned) ((N + 4 * kR - 1) / (4 * kR));
    k_gemv_q4_K<B, kR, NBL><<<grid, 256, 0, s>>>(w, xc, xbs, xd, y, res, N, nsb, ldy);
}

template <int B, int NBL>
void run_q5k(const uint8_t * w, const int8_t * xc, const int16_t * xbs, const float * xd, float * y, const float * res,
             int N, int nsb, int ldy, hipStream_t s) {
    const unsigned grid = (unsigned) ((N + 4 * kR - 1) / (4 * kR));
    k_gemv_q5_K<B, kR, NBL><<<grid, 256, 0, s>>>(w, xc, xbs, xd, y, res, N, nsb, ldy);
}

template <int B, int NBL>
void run_q6k(const uint8_t * w, const WeightLayout & L, const int8_t * xc, const int16_t * xbs, const float * xd,
             float * y, const float * res, int N, int nsb, int ldy, hipStream_t s) {
    const unsigned grid = (unsigned) ((N + 4 * kR - 1) / (4 * kR));
    k_gemv_q6_K<B, kR, NBL><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), xc, xbs, xd, y, res, N, nsb,
                                                 ldy);
}

// Q5_K / Q6_K hold 5 x 16 B of loads per (task, row): at most 2 tasks per lane per pass.
template <int B>
void run_k56_nbl(int type, int nbl, const uint8_t * w, const WeightLayout & L, const int8_t * xc, const int16_t * xbs,
                 const float * xd, float * y, const float * res, int N, int nsb, int ldy, hipStream_t s) {
    if (type == T_Q5_K) {
        if (nbl == 1) run_q5k<B, 1>(w, xc, xbs, xd, y, res, N, nsb, ldy, s);
        else run_q5k<B, 2>(w, xc, xbs, xd, y, res, N, nsb, ldy, s);
    } else {
        if (nbl == 1) run_q6k<B, 1>(w, L, xc, xbs, xd, y, res, N, nsb, ldy, s);
        else run_q6k<B, 2>(w, L, xc, xbs, xd, y, res, N, nsb, ldy, s);
    }
}

template <int B>
void run_q4k_nbl(int nbl, const uint8_t * w, const int8_t * xc, const int16_t * xbs, const float * xd, float * y,
                 const float * res, int N, int nsb, int ldy, hipStream_t s) {
    switch (nbl) {
        case 1: run_q4k<B, 1>(w, xc, xbs, xd, y, res, N, nsb, ldy, s); break;
        case 2: run_q4k<B, 2>(w, xc, xbs, xd, y, res, N, nsb, ldy, s); break;
        case 4: run_q4k<B, 4>(w, xc, xbs, xd, y, res, N, nsb, ldy, s); break;
        default: run_q4k<B, 8>(w, xc, xbs, xd, y, res, N, nsb, ldy, s); break;
    }
}

}  // namespace

// One f32 row times a Q4_K / Q5_K weight in one launch, the row quantized to Q8_K in the kernel
// (k_gemv_ks<..., FQ>): K a multiple of 256 up to 16384, up to kKsRowMaxN rows (measured: beyond,
// the separate quantization plus the one-row K-quant kernels is faster: 4096 x 28672 Q4_K 15.8 us
// against 16.9 fused, Q5_K 19.6 against 24.3), the weight below 2 GB.
constexpr int64_t kKsRowMaxN = 8192;

bool gemv_row_kq_fits(int type, int64_t N, int64_t K) {
    return (type == T_Q4_K || type == T_Q5_K) && K % QKK == 0 && K > 0 && K / QK <= 512 && N > 0 && N <= kKsRowMaxN &&
           weight_layout(type, N, K).total < 0x80000000ull;
}

void launch_gemv_row_kq(int type, const void * w, int64_t N, int64_t K, const float * x, float * y, hipStream_t s) {
    require(gemv_row_kq_fits(type, N, K), "gemv row: Q4_K / Q5_K, K a multiple of 256 up to 16384");
    KsArgs k{};
    const WeightLayout L = weight_layout(type, N, K);
    k.w = (const uint8_t *) w;
    k.kq_qh = (uint32_t) L.qh;
    k.kq_hdr = (uint32_t) L.d;
    k.kq_bytes = (uint32_t) L.total;
    k.x = x;
    k.y = y;
    k.N = (int) N;
    k.ntask = (int) (K / QK);
    k.ldy = (int) N;
    if (type == T_Q4_K) run_ks<T_Q4_K, 1, 4, true>(k, s);
    else run_ks<T_Q5_K, 1, 4, true>(k, s);
    check_launch("gemv row");
}

// y [B][ldy] (first N columns written) from packed weights and a quantized activation; with res,
// y = res + W x (res has y's layout and may be y itself).
void launch_gemv(int type, const void * wv, int64_t N, int64_t K, const void * act, int64_t B, float * y, int64_t ldy,
                 hipStream_t s, const float * res) {
    const uint8_t * w = (const uint8_t *) wv;
    const ActLayout A = act_layout(type, B, K);
    const uint8_t * a = (const uint8_t *) act;
    const uint64_t ks_bytes = is_kquant(type) ? (uint64_t) weight_layout(type, N, K).total
                                              : (uint64_t) N * (uint64_t) (K / QK) * (type == T_Q4_0 ? 16u : 32u);
    if (ks_fits(type, K, B) && (B > 1 || N <= kKsRowMaxN) && ks_bytes < 0x80000000ull) {
        const bool kq = is_kquant(type);
        const WeightLayout L = weight_layout(type, N, K);
        KsArgs k{};
        k.w = kq ? w : w + L.qs;
        k.wd = kq ? nullptr : (const uint16_t *) (w + L.d);
        k.kq_qh = kq ? (uint32_t) L.qh : 0u;
        k.kq_hdr = kq ? (uint32_t) L.d : 0u;
        k.kq_bytes = kq ? (uint32_t) L.total : 0u;
        k.xc = (const int8_t *) (a + A.codes);
        k.xm = kq ? nullptr : (const float2 *) (a + A.meta);
        k.xbs = kq ? (const int16_t *) (a + A.meta) : nullptr;
        k.xd = kq ? (const float *) (a + A.d) : nullptr;
        k.y = y;
        k.res = res;
        k.N = (int) N;
        k.ntask = (int) (K / QK);
        k.ldy = (int) ldy;
        if (type == T_Q4_0) run_ks_t<T_Q4_0>((int) B, k, s);
        else if (type == T_Q8_0) run_ks_t<T_Q8_0>((int) B, k, s);
        else if (type == T_Q4_K) run_ks_t<T_Q4_K>((int) B, k, s);
        else run_ks_t<T_Q5_K>((int) B, k, s);
        check_launch("gemv");
        return;
    }
    if (type == T_Q4_0 || type == T_Q8_0) {
        const WeightLayout L = weight_layout(type, N, K);
        const int nb = (int) (K / QK);
        const int nbl = pick_nbl(nb);
        const int8_t * xc = (const int8_t *) (a + A.codes);
        const float2 * xm = (const float2 *) (a + A.meta);
#define GCQ_Q0(TY)                                                                                     \
    switch (B) {                                                                                       \
        case 1: run_q0_nbl<TY, 1>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 2: run_q0_nbl<TY, 2>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 3: run_q0_nbl<TY, 3>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 4: run_q0_nbl<TY, 4>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 5: run_q0_nbl<TY, 5>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 6: run_q0_nbl<TY, 6>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        case 7: run_q0_nbl<TY, 7>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;             \
        default: run_q0_nbl<TY, 8>(nbl, w, L, xc, xm, y, res, (int) N, nb, (int) ldy, s); break;            \
    }
        if (type == T_Q4_0) {
            GCQ_Q0(T_Q4_0)
        } else {
            GCQ_Q0(T_Q8_0)
        }
#undef GCQ_Q0
    } else if (type == T_Q4_K) {
        const int nsb = (int) (K / QKK);
        const int nbl = pick_nbl(nsb * 4);
        const int8_t * xc = (const int8_t *) (a + A.codes);
        const int16_t * xbs = (const int16_t *) (a + A.meta);
        const float * xd = (const float *) (a + A.d);
        switch (B) {
            case 1: run_q4k_nbl<1>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 2: run_q4k_nbl<2>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 3: run_q4k_nbl<3>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 4: run_q4k_nbl<4>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 5: run_q4k_nbl<5>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 6: run_q4k_nbl<6>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 7: run_q4k_nbl<7>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            default: run_q4k_nbl<8>(nbl, w, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
        }
    } else if (type == T_Q5_K || type == T_Q6_K) {
        const WeightLayout L = weight_layout(type, N, K);
        const int nsb = (int) (K / QKK);
        const int nbl = std::min(pick_nbl(nsb * 4), 2);
        const int8_t * xc = (const int8_t *) (a + A.codes);
        const int16_t * xbs = (const int16_t *) (a + A.meta);
        const float * xd = (const float *) (a + A.d);
        switch (B) {
            case 1: run_k56_nbl<1>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 2: run_k56_nbl<2>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 3: run_k56_nbl<3>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 4: run_k56_nbl<4>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 5: run_k56_nbl<5>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 6: run_k56_nbl<6>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            case 7: run_k56_nbl<7>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
            default: run_k56_nbl<8>(type, nbl, w, L, xc, xbs, xd, y, res, (int) N, nsb, (int) ldy, s); break;
        }
    } else {
        fail("mul_mat: unsupported weight type " + std::to_string(type));
    }
    check_launch("gemv");
}

void launch_isums(int type, const void * wv, int64_t N, int64_t K, const void * act, int64_t B, int32_t * out,
                  hipStream_t s) {
    const uint8_t * w = (const uint8_t *) wv;
    const ActLayout A = act_layout(type, B, K);
    const uint8_t * a = (const uint8_t *) act;
    if (type == T_Q4_0 || type == T_Q8_0) {
        const WeightLayout L = weight_layout(type, N, K);
        const int nb = (int) (K / QK);
        const int64_t n = B * N * nb;
        k_isums_q0<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(type, w + L.qs, (const uint16_t *) (w + L.d),
                                                             (const int8_t *) (a + A.codes),
                                                             (const float2 *) (a + A.meta), out, (int) N, nb, (int) B);
    } else if (type == T_Q4_K) {
        const int nsb = (int) (K / QKK);
        const int64_t n = B * N * nsb;
        k_isums_q4_K<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(w, (const int8_t *) (a + A.codes),
                                                               (const int16_t *) (a + A.meta), out, (int) N, nsb,
                                                               (int) B);
    } else if (type == T_Q5_K) {
        const int nsb = (int) (K / QKK);
        const int64_t n = B * N * nsb;
        k_isums_q5_K<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(w, (const int8_t *) (a + A.codes),
                                                               (const int16_t *) (a + A.meta), out, (int) N, nsb,
                                                               (int) B);
    } else if (type == T_Q6_K) {
        const WeightLayout L = weight_layout(type, N, K);
        const int nsb = (int) (K / QKK);
        const int64_t n = B * N * nsb;
        k_isums_q6_K<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(w + L.qs, (const int8_t *) (a + A.codes),
                                                               (const int16_t *) (a + A.meta), out, (int) N, nsb,
                                                               (int) B);
    } else {
        fail("isums: unsupported type " + std::to_string(type));
    }
    check_launch("isums");
}

}  // namespace gcq
