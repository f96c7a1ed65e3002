// matmul_f.hip - ggml_mul_mat of an f32 or f16 first operand (an activation or a KV-cache view)
// by f32 rows: Q·Kᵀ and P·V of eager attention (the attention programs compiled without the
// flash-attention fusion, and the fallback of runtime/include/ggml_compiler_ops.h:140-148), and any
// other activation-by-activation product a program holds (runtime/src/ops.cpp:107-119).
//
// Semantics (ggml_compiler/ir/ops.py:186-214): a [K, N, A2, A3] (ggml ne), b [K, M, B2, B3] with
// A2 | B2 and A3 | B3; out [N, M, B2, B3] f32 contiguous, out[i3][i2][m][n] =
// sum_k a[i3 / (B3/A3)][i2 / (B2/A2)][n][k] * b[i3][i2][m][k] -- a's batch repeat-interleaved over
// b's, which is grouped-query attention's head sharing. As ggml's CPU mul_mat converts src1 to the
// first operand's vec_dot_type, b is rounded to f16 when a is f16; products and sums are f32.
//
// One 256-thread block per 64 x 64 output tile of one batch; K in steps of 16 staged through LDS
// (a tile k-major so the 16 threads of a row read consecutive n), 4 x 4 outputs per thread. Strides
// are arbitrary (element strides of a's rows and batches, b's rows and batches), so permuted views
// multiply without a copy; only a's innermost dim must be contiguous (ggml refuses a transposed
// first operand).
#include "gcq_common.h"

namespace gcq {
namespace {

constexpr int TN = 64, TM = 64, TK = 16;

template <bool AF16>
__global__ __launch_bounds__(256) void k_mul_mat_f(const void * __restrict__ a_, int64_t a1, int64_t a2, int64_t a3,
                                                   const float * __restrict__ b, int64_t b1, int64_t b2, int64_t b3,
                                                   float * __restrict__ out, int K, int N, int M, int B2, int r2, int r3) {
    __shared__ float As[TK][TN + 1];
    __shared__ float Bs[TK][TM + 1];
    const int t = threadIdx.x;
    const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
    const int i2 = blockIdx.z % B2, i3 = blockIdx.z / B2;
    const int64_t abase = (int64_t) (i2 / r2) * a2 + (int64_t) (i3 / r3) * a3;
    const float * bb = b + (int64_t) i2 * b2 + (int64_t) i3 * b3;
    // loader: row lr (0..63) of the tile, k offsets lk .. lk + 3
    const int lr = t >> 2, lk = (t & 3) * 4;
    const int tx = t & 15, ty = t >> 4;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += TK) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = k0 + lk + q;
            const int n = n0 + lr, m = m0 + lr;
            float av = 0.0f, bv = 0.0f;
            if (k < K && n < N) {
                const int64_t off = abase + (int64_t) n * a1 + k;
                av = AF16 ? h2f(static_cast<const uint16_t *>(a_)[off]) : static_cast<const float *>(a_)[off];
            }
            if (k < K && m < M) {
                bv = bb[(int64_t) m * b1 + k];
                if (AF16) bv = h2f(f2h(bv));
            }
            As[lk + q][lr] = av;
            Bs[lk + q][lr] = bv;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < TK; k++) {
            float ar[4], br[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ar[i] = As[k][tx + 16 * i];
                br[i] = Bs[k][ty + 16 * i];
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[j][i] = fmaf(ar[i], br[j], acc[j][i]);
        }
        __syncthreads();
    }
    float * ob = out + (int64_t) blockIdx.z * M * N;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int m = m0 + ty + 16 * j;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + tx + 16 * i;
            if (n < N) ob[(int64_t) m * N + n] = acc[j][i];
        }
    }
}

}  // namespace

void launch_mul_mat_f(bool a_f16, const void * a, const int64_t * ane, const int64_t * anb_el, const float * b,
                      const int64_t * bne, const int64_t * bnb_el, float * out, hipStream_t s) {
    const int64_t K = ane[0], N = ane[1], M = bne[1], B2 = bne[2], B3 = bne[3];
    if (bne[0] != K || ane[2] <= 0 || ane[3] <= 0 || B2 % ane[2] || B3 % ane[3])
        throw std::runtime_error("mul_mat: operand shapes do not line up");
    if (K > INT32_MAX || N > INT32_MAX || M > INT32_MAX || B2 * B3 > INT32_MAX)
        throw std::runtime_error("mul_mat: sizes out of range");
    if (N == 0 || M == 0 || B2 * B3 == 0) return;
    const dim3 grid((unsigned) ((N + TN - 1) / TN), (unsigned) ((M + TM - 1) / TM), (unsigned) (B2 * B3));
    if (grid.y > 65535 || grid.z > 65535) throw std::runtime_error("mul_mat: too many row tiles or batches");
    const int r2 = (int) (B2 / ane[2]), r3 = (int) (B3 / ane[3]);
    if (a_f16)
        k_mul_mat_f<true><<<grid, 256, 0, s>>>(a, anb_el[1], anb_el[2], anb_el[3], b, bnb_el[1], bnb_el[2], bnb_el[3],
                                               out, (int) K, (int) N, (int) M, (int) B2, r2, r3);
    else
        k_mul_mat_f<false><<<grid, 256, 0, s>>>(a, anb_el[1], anb_el[2], anb_el[3], b, bnb_el[1], bnb_el[2], bnb_el[3],
                                                out, (int) K, (int) N, (int) M, (int) B2, r2, r3);
    check_launch("mul_mat (f32 / f16)");
}

}  // namespace gcq
