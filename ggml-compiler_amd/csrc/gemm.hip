// gemm.hip - quantized mat-mul for prefill (M > 8 activation rows) on int8 MFMA.
//
// Replaces ggml_mul_mat of a Q8_0 / Q4_0 weight with an f32 src1 of many rows
// (runtime/src/ops.cpp:107-119). As ggml, src1 is quantized to Q8_0 per 32 values (quant.hip);
// then out[m, n] = sum_blk d_x[m, blk] * d_w[n, blk] * isum(m, n, blk) with isum the exact int32
// dot of one 32-value block.
//
// gfx950's v_mfma_i32_32x32x32_i8 has a depth of exactly one quant block, so every MFMA yields
// the 32x32 tile of block sums isum(., ., blk) exactly; the fp16-scale epilogue folds it into fp32
// accumulators (d_w and d_x from LDS). Workgroup tile 128 (m) x 128 (n), 4 wavefronts of 64x64
// (2x2 MFMA tiles); two LDS stages of 2 K-blocks each of A (activation codes) and B (weight codes,
// Q4_0 nibbles expanded to signed int8 q-8), with a 16-byte row pad against bank conflicts. Tiles
// are numbered so that the workgroups sharing one weight tile land on the same XCD (and L2).
//
// The per-block epilogue (3 VALU operations per output element per K-block of 32, against one
// 32-deep MFMA step) bounds this kernel near 1/6 of the int8 MFMA peak: ggml's semantics put a
// scale on every block, so the block sums cannot stay in the int32 accumulator.
#include "gcq_common.h"

namespace gcq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128;  // workgroup tile
constexpr int GKB = 2;               // K-blocks (of 32) per LDS stage
constexpr int GPITCH = GKB * 32 + 16;  // LDS row pitch in bytes (16 B pad against bank conflicts)

__device__ __forceinline__ uint32_t q4_to_s8(uint32_t w) {  // 4 nibbles (0..15) -> 4 int8 (q - 8)
    return (((w & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// One LDS stage's worth of global data held in registers between its load and its LDS store.
// A stage is GKB K-blocks of the workgroup's 128 activation rows and 128 weight rows.
constexpr int GA = GBM * GKB * 2 / 256;  // 16-byte activation chunks per thread (two per row-block)
constexpr int GS = GBM * GKB / 256;      // row-blocks per thread for the scales and Q4_0 nibbles
static_assert(GA >= 1 && GS >= 1, "stage size");

// Native vector types, not HIP's int4 / uint4 structs: struct copies become memcpys through a
// stack object that is not promoted to registers, which puts the staged loads in scratch memory
// and makes every chunk wait for its global loads before computing.
template <int TYPE>
struct GemmStage {
    v4i a[GA];                                // activation codes
    v4i b[TYPE == T_Q8_0 ? GA : GS];          // weight codes: Q8_0 like a, Q4_0 one block's 16 B of nibbles
    float dx[GS];                             // activation scales
    uint32_t dw[GS];                          // weight scales (fp16 bits)
};

// Chunk c (K-blocks kb0 .. kb0 + GKB) of this workgroup's tile: thread t's share. Rows past M or
// N reload the last row; blocks past nb reload the last block (never used).
template <int TYPE>
__device__ __forceinline__ void gemm_load(GemmStage<TYPE> & st, const uint8_t * __restrict__ wqs,
                                          const uint16_t * __restrict__ wd, const int8_t * __restrict__ xc,
                                          const float2 * __restrict__ xm, int m0, int n0, int M, int N, int nb, int kb0) {
    const int t = threadIdx.x;
    const int K = nb * 32;
#pragma unroll
    for (int i = 0; i < GA; i++) {  // A: 128 rows x GKB*32 B in chunks of 16 B
        const int c = t + 256 * i;
        const int row = c / (GKB * 2), part = c % (GKB * 2);
        const int gm = min(m0 + row, M - 1);
        const int kb = min(kb0 + part / 2, nb - 1);
        st.a[i] = *reinterpret_cast<const v4i *>(xc + (size_t) gm * K + (size_t) kb * 32 + (part & 1) * 16);
    }
    if constexpr (TYPE == T_Q8_0) {
#pragma unroll
        for (int i = 0; i < GA; i++) {
            const int c = t + 256 * i;
            const int row = c / (GKB * 2), part = c % (GKB * 2);
            const int gn = min(n0 + row, N - 1);
            const int kb = min(kb0 + part / 2, nb - 1);
            st.b[i] = *reinterpret_cast<const v4i *>(wqs + ((size_t) gn * nb + kb) * 32 + (part & 1) * 16);
        }
    } else {  // 128 rows x GKB blocks of 16 B
#pragma unroll
        for (int i = 0; i < GS; i++) {
            const int c = t + 256 * i;
            const int row = c / GKB, j = c % GKB;
            const int gn = min(n0 + row, N - 1);
            const int kb = min(kb0 + j, nb - 1);
            st.b[i] = *reinterpret_cast<const v4i *>(wqs + ((size_t) gn * nb + kb) * 16);
        }
    }
#pragma unroll
    for (int i = 0; i < GS; i++) {  // scales: 128 rows x GKB blocks each
        const int c = t + 256 * i;
        const int row = c / GKB, j = c % GKB;
        const int kb = min(kb0 + j, nb - 1);
        st.dx[i] = xm[(size_t) min(m0 + row, M - 1) * nb + kb].x;
        st.dw[i] = wd[(size_t) min(n0 + row, N - 1) * nb + kb];
    }
}

template <int TYPE>
__device__ __forceinline__ void gemm_store(const GemmStage<TYPE> & st, int8_t * sA, int8_t * sB, float * sdx,
                                           float * sdw) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < GA; i++) {
        const int c = t + 256 * i;
        const int row = c / (GKB * 2), part = c % (GKB * 2);
        *reinterpret_cast<v4i *>(sA + row * GPITCH + part * 16) = st.a[i];
    }
    if constexpr (TYPE == T_Q8_0) {
#pragma unroll
        for (int i = 0; i < GA; i++) {
            const int c = t + 256 * i;
            const int row = c / (GKB * 2), part = c % (GKB * 2);
            *reinterpret_cast<v4i *>(sB + row * GPITCH + part * 16) = st.b[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < GS; i++) {
            const int c = t + 256 * i;
            const int row = c / GKB, j = c % GKB;
            const v4i w = st.b[i];
            v4i lo, hi;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                lo[e] = (int) q4_to_s8((uint32_t) w[e]);
                hi[e] = (int) q4_to_s8((uint32_t) w[e] >> 4);
            }
            *reinterpret_cast<v4i *>(sB + row * GPITCH + j * 32) = lo;
            *reinterpret_cast<v4i *>(sB + row * GPITCH + j * 32 + 16) = hi;
        }
    }
#pragma unroll
    for (int i = 0; i < GS; i++) {
        const int c = t + 256 * i;
        const int row = c / GKB, j = c % GKB;
        sdx[j * GBM + row] = st.dx[i];
        sdw[j * GBN + row] = h2f((uint16_t) st.dw[i]);
    }
}

// RAW: write the int32 block sums of block `raw_blk` instead of the scaled result.
//
// Pipeline: chunk c + 1's global loads are issued into registers before chunk c is computed from
// LDS, then stored to the other LDS buffer; one barrier per chunk. Per K-block each wavefront
// issues its four 32x32x32 MFMAs, then folds each int32 result into the fp32 accumulators as
// (isum * d_w) * d_x, the scales read from LDS once per block as vectors.
template <int TYPE, bool RAW>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t * __restrict__ wqs, const uint16_t * __restrict__ wd,
                                              const int8_t * __restrict__ xc, const float2 * __restrict__ xm,
                                              float * y, const float * res, int32_t * __restrict__ yraw, int M, int N,
                                              int nb, int ldy, int raw_blk) {
    __shared__ __attribute__((aligned(16))) int8_t sA[2][GBM * GPITCH];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][GBN * GPITCH];
    __shared__ __attribute__((aligned(16))) float sdx[2][GKB * GBM];
    __shared__ __attribute__((aligned(16))) float sdw[2][GKB * GBN];

    // Tile numbering: ids id, id+8, ... run on one XCD; give each XCD a contiguous run of tiles,
    // m-tiles fastest, so the workgroups that read one weight tile share an L2.
    const int mt = (M + GBM - 1) / GBM, nt = (N + GBN - 1) / GBN;
    const int total = mt * nt;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    const int m0 = (id % mt) * GBM, n0 = (id / mt) * GBN;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    float acc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.0f;

    const int kb_begin = RAW ? raw_blk : 0;
    const int kb_end = RAW ? raw_blk + 1 : nb;
    const int nchunk = (kb_end - kb_begin + GKB - 1) / GKB;
    GemmStage<TYPE> st;
    gemm_load<TYPE>(st, wqs, wd, xc, xm, m0, n0, M, N, nb, kb_begin);
    gemm_store<TYPE>(st, sA[0], sB[0], sdx[0], sdw[0]);
    __syncthreads();

    for (int c = 0; c < nchunk; c++) {
        const int buf = c & 1;
        const int kb0 = kb_begin + c * GKB;
        if (c + 1 < nchunk) gemm_load<TYPE>(st, wqs, wd, xc, xm, m0, n0, M, N, nb, kb0 + GKB);
        const int nblk = min(GKB, kb_end - kb0);
#pragma unroll
        for (int j = 0; j < GKB; j++) {
            if (j >= nblk) break;
            v4i af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                af[t] = *reinterpret_cast<const v4i *>(sA[buf] + (wm * 64 + t * 32 + (lane & 31)) * GPITCH + j * 32 +
                                                       16 * (lane >> 5));
                bf[t] = *reinterpret_cast<const v4i *>(sB[buf] + (wn * 64 + t * 32 + (lane & 31)) * GPITCH + j * 32 +
                                                       16 * (lane >> 5));
            }
            v16i cc[2][2];
#pragma unroll
            for (int tm = 0; tm < 2; tm++)
#pragma unroll
                for (int tn = 0; tn < 2; tn++)
                    cc[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bf[tn], v16i{}, 0, 0, 0);
            if constexpr (RAW) {
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
#pragma unroll
                    for (int tn = 0; tn < 2; tn++)
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[tm][tn][r] = __int_as_float(cc[tm][tn][r]);
            } else {
                // d_x of this lane's rows: element r of tile tm is row wm*64 + tm*32 + 8*(r/4) + 4*(lane/32) + r%4
                float4 dx[2][4];
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        dx[tm][q] = *reinterpret_cast<const float4 *>(sdx[buf] + j * GBM + wm * 64 + tm * 32 + q * 8 +
                                                                      (lane >> 5) * 4);
                float dwv[2];
#pragma unroll
                for (int tn = 0; tn < 2; tn++) dwv[tn] = sdw[buf][j * GBN + wn * 64 + tn * 32 + (lane & 31)];
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
#pragma unroll
                    for (int tn = 0; tn < 2; tn++)
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            acc[tm][tn][4 * q + 0] += ((float) cc[tm][tn][4 * q + 0] * dwv[tn]) * dx[tm][q].x;
                            acc[tm][tn][4 * q + 1] += ((float) cc[tm][tn][4 * q + 1] * dwv[tn]) * dx[tm][q].y;
                            acc[tm][tn][4 * q + 2] += ((float) cc[tm][tn][4 * q + 2] * dwv[tn]) * dx[tm][q].z;
                            acc[tm][tn][4 * q + 3] += ((float) cc[tm][tn][4 * q + 3] * dwv[tn]) * dx[tm][q].w;
                        }
            }
        }
        if (c + 1 < nchunk) gemm_store<TYPE>(st, sA[buf ^ 1], sB[buf ^ 1], sdx[buf ^ 1], sdw[buf ^ 1]);
        __syncthreads();
    }

#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int n = n0 + wn * 64 + tn * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (m >= M) continue;
                if constexpr (RAW) yraw[(size_t) m * N + n] = __float_as_int(acc[tm][tn][r]);
                else {
                    const size_t o = (size_t) m * ldy + n;
                    y[o] = res ? acc[tm][tn][r] + res[o] : acc[tm][tn][r];
                }
            }
        }
}

void launch_gemm(int type, const void * wv, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                 hipStream_t s, const float * res) {
    const WeightLayout L = weight_layout(type, N, K);
    const ActLayout A = act_layout(type, M, K);
    const uint8_t * w = (const uint8_t *) wv;
    const uint8_t * a = (const uint8_t *) act;
    const unsigned grid = (unsigned) (((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN));
    const int nb = (int) (K / 32);
    if (type == T_Q8_0)
        k_gemm<T_Q8_0, false><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), (const int8_t *) (a + A.codes),
                                                    (const float2 *) (a + A.meta), y, res, nullptr, (int) M, (int) N, nb,
                                                    (int) ldy, 0);
    else if (type == T_Q4_0)
        k_gemm<T_Q4_0, false><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), (const int8_t *) (a + A.codes),
                                                    (const float2 *) (a + A.meta), y, res, nullptr, (int) M, (int) N, nb,
                                                    (int) ldy, 0);
    else
        fail("gemm: unsupported weight type " + std::to_string(type));
    check_launch("gemm");
}

void launch_gemm_block_isums(int type, const void * wv, int64_t N, int64_t K, const void * act, int64_t M, int blk,
                             int32_t * out, hipStream_t s) {
    const WeightLayout L = weight_layout(type, N, K);
    const ActLayout A = act_layout(type, M, K);
    const uint8_t * w = (const uint8_t *) wv;
    const uint8_t * a = (const uint8_t *) act;
    const unsigned grid = (unsigned) (((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN));
    const int nb = (int) (K / 32);
    if (type == T_Q8_0)
        k_gemm<T_Q8_0, true><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), (const int8_t *) (a + A.codes),
                                                   (const float2 *) (a + A.meta), nullptr, nullptr, out, (int) M, (int) N, nb, 0,
                                                   blk);
    else if (type == T_Q4_0)
        k_gemm<T_Q4_0, true><<<grid, 256, 0, s>>>(w + L.qs, (const uint16_t *) (w + L.d), (const int8_t *) (a + A.codes),
                                                   (const float2 *) (a + A.meta), nullptr, nullptr, out, (int) M, (int) N, nb, 0,
                                                   blk);
    else
        fail("gemm: unsupported weight type " + std::to_string(type));
    check_launch("gemm isums");
}

}  // namespace gcq
