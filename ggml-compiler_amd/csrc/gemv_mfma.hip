// gemv_mfma.hip - the Q4_0 / Q8_0 mat-vec of 2..16 activation rows on the int8 matrix cores.
//
// y[b][n] = sum_k W[n][k] x[b][k] for a batch of B rows, the ggml_mul_mat of a decode batch
// (runtime/src/ops.cpp:107-119; ggml-cpu's vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0 per block). The
// one-row kernels (rowgemv.hip, gemv.hip) read every activation block once per weight row pair,
// which at B = 8 is 14 times the weight bytes per block from the caches: the batch rows, not HBM,
// bound them. Here one v_mfma_i32_16x16x32_i8 per 32-value block takes 16 weight rows against up
// to 16 activation rows, so each activation block is read once per 16 weight rows:
//
//   A (16 x 32): the activation codes, row b = lane % 16 (rows >= B zero), k = 8 (lane / 16) + j;
//   B (32 x 16): the weight codes of row n = lane % 16 of the tile, k = 8 (lane / 16) + j. Q4_0:
//     the k-th value of a block is the low nibble of byte k (k < 16) or the high nibble of byte
//     k - 16, so lanes l and l + 32 need the same 8 bytes; lanes 0-31 load block 2p, lanes 32-63
//     block 2p + 1 (8 bytes each, the 16 rows x 32 contiguous bytes of the pair, no byte twice),
//     and one v_permlane32_swap gives every lane both blocks' bytes. Q8_0: 8 bytes per block.
//   D (16 x 16): int32 sums; lane l holds batch rows 4 (lane / 16) + i, weight row lane % 16.
//
// Without a residual (y = W x only; the caller adds one with the row kernels). Per block the
// integer sum is scaled as ggml and the row kernels do: s = sum (q - 8) x (the -8
// folded in through the activation's code sum for Q4_0), acc += ((float) s * d_w) * d_x. A
// workgroup of NW wavefronts (8, or 16 when there are fewer tiles than two per CU) owns a tile of
// 16 weight rows at a time (tiles blockIdx.x, + grid); wavefront w takes block pairs w, w + NW,
// ... (together they read adjacent 32-byte pieces of every row), its loads 8 pairs ahead across
// tile boundaries (Q4_0: 512 bytes of weights per pair and wavefront, so 32-64 KB per CU in
// flight); the partial sums are added in LDS in wavefront order. The activation scales and code
// sums of all blocks sit in LDS for the launch.
#include "gcq_common.h"

#include <algorithm>

namespace gcq {

int cu_count();

namespace {

constexpr int kDepth = 8;  // block pairs a wavefront has in flight

typedef int v4i __attribute__((ext_vector_type(4)));

template <int TYPE>
struct PairRegs {
    static constexpr int WD = TYPE == T_Q4_0 ? 2 : 4;  // weight dwords per lane per pair
    uint32_t w[WD];
    uint32_t sc;       // fp16 scales of blocks 2p (low half) and 2p + 1
    uint32_t x[4];     // activation codes of blocks 2p, 2p + 1 (8 bytes each)
};

// LDS workgroup barrier that waits for LDS only (outstanding global loads stay in flight).
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int TYPE, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemv_mfma(const uint8_t * __restrict__ wqs,
                                                           const uint16_t * __restrict__ wd,
                                                           const int8_t * __restrict__ xc,
                                                           const float2 * __restrict__ xm, float * y, int N,
                                                           int nb, int B, int ldy) {
    extern __shared__ float2 s_meta[];  // [nb][16] (d, code sum) of activation row b, zero past B
    __shared__ float s_red[NW][64][4];
    constexpr int CB = TYPE == T_Q4_0 ? 16 : 32;  // bytes per weight block
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = nb * QK;
    for (int i = threadIdx.x; i < nb * 16; i += NW * 64) {
        const int blk = i >> 4, b = i & 15;
        s_meta[i] = b < B ? xm[(size_t) b * nb + blk] : make_float2(0.0f, 0.0f);
    }
    lds_sync();

    const int ntiles = (N + 15) / 16;
    const int npairs = nb / 2;
    const int per_tile = (npairs - wave + NW - 1) / NW;  // this wavefront's pairs per tile
    const int my_tiles = (int) blockIdx.x < ntiles ? (ntiles - (int) blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    const int total = my_tiles * per_tile;
    const int n_l = lane & 15, kq = lane >> 4;
    const int xrow = lane & 15;  // activation row of this lane's A operand
    const bool xlive = xrow < B;

    // Item i of this wavefront: tile blockIdx.x + (i / per_tile) * grid, pair wave + (i % per_tile) * NW.
    // Buffer loads, every one issued whatever the item (an offset past the buffer reads zeros
    // without a memory access: items past the last, activation rows >= B), so the number of loads
    // in flight is the same on every path and each use waits for its own loads only.
    constexpr uint32_t kPast = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wqs), 0, (int) ((uint32_t) N * (uint32_t) nb * CB), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(wd), 0, (int) ((uint32_t) N * (uint32_t) nb * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(xc), 0, (int) ((uint32_t) B * (uint32_t) K), 0x00020000);
    // (k, j): the wavefront's j-th pair of its k-th tile; advanced without divisions.
    auto load = [&](int k, int j, PairRegs<TYPE> & r) {
        const bool live = k < my_tiles;
        const int tile = (int) blockIdx.x + k * (int) gridDim.x;
        const int p = wave + j * NW;
        const int row = min(tile * 16 + n_l, N - 1);
        const uint32_t rb = (uint32_t) row * (uint32_t) nb;
        if constexpr (TYPE == T_Q4_0) {
            const uint32_t blk = 2u * (uint32_t) p + (uint32_t) (lane >> 5);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rw, live ? (rb + blk) * CB + 8u * (kq & 1) : kPast, 0, 2);
            r.w[0] = v[0];
            r.w[1] = v[1];
        } else {
            const auto v0 = __builtin_amdgcn_raw_buffer_load_b64(rw, live ? (rb + 2u * p) * CB + 8u * kq : kPast, 0, 2);
            const auto v1 = __builtin_amdgcn_raw_buffer_load_b64(rw, live ? (rb + 2u * p + 1u) * CB + 8u * kq : kPast, 0, 2);
            r.w[0] = v0[0];
            r.w[1] = v0[1];
            r.w[2] = v1[0];
            r.w[3] = v1[1];
        }
        // nb even: the pair's two fp16 scales are one aligned word
        r.sc = __builtin_amdgcn_raw_buffer_load_b32(rs, live ? (rb + 2u * p) * 2u : kPast, 0, 0);
        const uint32_t xo = (uint32_t) xrow * (uint32_t) K + (uint32_t) (2 * p) * QK + 8u * kq;
        const bool xin = live && xlive;
        const auto a0 = __builtin_amdgcn_raw_buffer_load_b64(rx, xin ? xo : kPast, 0, 0);
        const auto a1 = __builtin_amdgcn_raw_buffer_load_b64(rx, xin ? xo + QK : kPast, 0, 0);
        r.x[0] = a0[0];
        r.x[1] = a0[1];
        r.x[2] = a1[0];
        r.x[3] = a1[1];
    };

    PairRegs<TYPE> buf[kDepth];
    int lk = 0, lj = 0;  // load cursor
    auto advance = [&](int & k, int & j) {
        if (++j == per_tile) {
            j = 0;
            ++k;
        }
    };
#pragma unroll
    for (int d = 0; d < kDepth; d++) {
        load(lk, lj, buf[d]);
        advance(lk, lj);
    }

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // One block: D = A B, then acc[i] += ((float) (D_i - 8 xsum_b) * d_w) * d_x_b.
    auto block = [&](int blk, long a, long bw, uint16_t dbits) {
        v4i c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bw, c, 0, 0, 0);
        const float dw = h2f(dbits);
        const int bm = min(blk, nb - 1) * 16 + 4 * kq;  // items past the last: any block (their sums are 0)
        const float4 m01 = *reinterpret_cast<const float4 *>(&s_meta[bm]);
        const float4 m23 = *reinterpret_cast<const float4 *>(&s_meta[bm + 2]);
        const float dx[4] = {m01.x, m01.z, m23.x, m23.z};
        const int xs[4] = {__float_as_int(m01.y), __float_as_int(m01.w), __float_as_int(m23.y), __float_as_int(m23.w)};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = TYPE == T_Q4_0 ? c[i] - 8 * xs[i] : c[i];
            acc[i] += ((float) s * dw) * dx[i];
        }
    };
    auto pair = [&](int j, const PairRegs<TYPE> & r) {
        const int p = wave + j * NW;
        long b0, b1;
        if constexpr (TYPE == T_Q4_0) {
            // lanes < 32 hold block 2p, lanes >= 32 block 2p + 1: after the swap [0] is block 2p's
            // bytes and [1] block 2p + 1's in every lane; lanes >= 32 take the high nibbles.
            const auto s0 = __builtin_amdgcn_permlane32_swap(r.w[0], r.w[0], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(r.w[1], r.w[1], false, false);
            const uint32_t sh = (uint32_t) (lane >> 5) * 4u;
            const uint32_t lo0 = (s0[0] >> sh) & 0x0F0F0F0Fu, hi0 = (s1[0] >> sh) & 0x0F0F0F0Fu;
            const uint32_t lo1 = (s0[1] >> sh) & 0x0F0F0F0Fu, hi1 = (s1[1] >> sh) & 0x0F0F0F0Fu;
            b0 = (long) (((uint64_t) hi0 << 32) | lo0);
            b1 = (long) (((uint64_t) hi1 << 32) | lo1);
        } else {
            b0 = (long) (((uint64_t) r.w[1] << 32) | r.w[0]);
            b1 = (long) (((uint64_t) r.w[3] << 32) | r.w[2]);
        }
        const long a0 = (long) (((uint64_t) r.x[1] << 32) | r.x[0]);
        const long a1 = (long) (((uint64_t) r.x[3] << 32) | r.x[2]);
        block(2 * p, a0, b0, (uint16_t) (r.sc & 0xffff));
        block(2 * p + 1, a1, b1, (uint16_t) (r.sc >> 16));
    };
    // The tile's sums: the four wavefronts' partials added in wavefront order.
    auto finish = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 4; i++) s_red[wave][lane][i] = acc[i];
        lds_sync();
        // thread t: output (b = t / 16, n = t % 16): lane (b / 4) * 16 + n, register b % 4
        const int t = threadIdx.x, b = t >> 4, n = t & 15;
        if (b < B) {  // b < 16: t < 256
            const int src = (b >> 2) * 16 + n, reg = b & 3;
            float v = s_red[0][src][reg];
#pragma unroll
            for (int w = 1; w < NW; w++) v += s_red[w][src][reg];
            const int row = tile * 16 + n;
            if (row < N) y[(size_t) b * ldy + row] = v;
        }
        lds_sync();
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = 0.0f;
    };

    // Items past the last are computed on the zeros their loads returned (adding nothing), so
    // only the tile ends are conditional.
    int ck = 0, cj = 0;  // compute cursor
    for (int i0 = 0; i0 < total; i0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; d++) {
            pair(cj, buf[d]);
            load(lk, lj, buf[d]);
            advance(lk, lj);
            const bool end = cj == per_tile - 1 && ck < my_tiles;
            if (end) finish((int) blockIdx.x + ck * (int) gridDim.x);
            advance(ck, cj);
        }
    }
    // Every wavefront meets the others in finish once per tile: the host requires nb / 2 >= NW,
    // so each has at least one pair per tile.
}

}  // namespace

// B = 2..16 rows of Q8_0 activations against a packed Q4_0 / Q8_0 weight with nb even and at
// least 32 blocks per row (a pair per wavefront of 16); the activation scales of all blocks fit
// 64 KB of LDS (nb <= 512, K <= 16384).
bool gemv_mfma_fits(int type, int64_t K, int64_t B) {
    const int64_t nb = K / QK;
    return (type == T_Q4_0 || type == T_Q8_0) && K % 64 == 0 && nb >= 32 && nb <= 512 && B >= 2 && B <= 16;
}

void launch_gemv_mfma(int type, const uint8_t * wqs, const uint16_t * wd, const int8_t * xc, const float2 * xm,
                      float * y, int N, int nb, int B, int ldy, hipStream_t s) {
    require(gemv_mfma_fits(type, (int64_t) nb * QK, B), "gemv mfma: shape not supported");
    const int ntiles = (N + 15) / 16;
    const size_t lds = (size_t) nb * 16 * sizeof(float2);
    // Workgroups: as many as give every one the same number of tiles, at most 2 per CU; 16
    // wavefronts each when that leaves less than 2 per CU.
    const int cus = cu_count(), maxg = 2 * cus;
    const int per = (ntiles + maxg - 1) / maxg;
    const unsigned grid = (unsigned) ((ntiles + per - 1) / per);
    const bool wide = (int) grid < maxg;
#define GCQ_GM(T, W) k_gemv_mfma<T, W><<<grid, W * 64, lds, s>>>(wqs, wd, xc, xm, y, N, nb, B, ldy)
    if (type == T_Q4_0) {
        if (wide) GCQ_GM(T_Q4_0, 16);
        else GCQ_GM(T_Q4_0, 8);
    } else {
        if (wide) GCQ_GM(T_Q8_0, 16);
        else GCQ_GM(T_Q8_0, 8);
    }
#undef GCQ_GM
    check_launch("gemv mfma");
}

}  // namespace gcq
