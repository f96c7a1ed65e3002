// gemm_kq.hip - quantized mat-mul for prefill (M > 8 activation rows) with K-quant weights (Q4_K,
// Q5_K, Q6_K) on int8 MFMA.
//
// Replaces ggml_mul_mat of a K-quant weight with an f32 src1 of many rows
// (runtime/src/ops.cpp:107-119). As ggml (vec_dot_type Q8_K), src1 is quantized to Q8_K per 256
// values (quant.hip); per super-block i and output (m, n) the integer parts of ggml's
// vec_dot_q{4,5,6}_K_q8_K are exact and the float part scales them:
//   Q4_K / Q5_K: I1 = sum_j sc_j(n) isum_j(m, n), I2 = sum_j m_j(n) (bsum_2j + bsum_2j+1)(m) over the
//                8 sub-blocks of 32; y += d_x(m) (d_w(n) I1 - dmin_w(n) I2)
//   Q6_K:        I1 = sum_j sc_j(n) isum_j(m, n) over the 16 sub-blocks of 16 (codes q - 32);
//                y += d_x(m) d_w(n) I1
// isum_j is one MFMA: v_mfma_i32_32x32x32_i8 over a 32-value sub-block, v_mfma_i32_32x32x16_i8 over
// a 16-value one. I1 takes the sub-block's 6-bit / int8 scale on the VALU (one integer
// multiply-add per output and sub-block). I2 is itself a small integer product over the 8
// sub-blocks: the activation's block sums split into bytes (bs = 64 hi + lo, lo in [0, 64)) against
// the weight's 6-bit mins, two MFMAs of K 32 (8 used) per super-block.
//
// Workgroup tile 128 (m) x 128 (n), 8 wavefronts of 64 x 32 (2 MFMA tiles of 32 x 32). The K
// loop steps half a super-block (128 values) at a time: the next half's global loads are issued
// into registers before the current half is computed from LDS, then stored (weights expanded to
// int8 codes, the super-block's scales decoded); activations and weights of a tile are read once
// per workgroup. A wavefront's 64 outputs per lane (f32 sums and the super-block's int32 sums) keep it
// within 256 registers, two wavefronts per SIMD. Tiles are numbered
// so that the workgroups sharing a weight tile land on one XCD.
#include "gcq_common.h"

namespace gcq {

int cu_count();

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int TM = 128;            // workgroup tile rows; its columns TN: 128, or 64 for small grids
constexpr int NT = 512;            // threads: 8 wavefronts of 64 (m) x 32 (n)
constexpr int HV = 128;            // values per K step (half a super-block)
constexpr int KP = HV + 16;        // LDS row pitch of the codes (bytes; 16 B pad against bank conflicts)

template <int TYPE>
struct Kq {
    static constexpr int BB = 128;  // the low bits' bytes per super-block (nibbles / Q6_K's ql)
    static constexpr bool MIN = TYPE != T_Q6_K;  // a min term (Q4_K / Q5_K)
    static constexpr int NSUB = TYPE == T_Q6_K ? 16 : 8;  // scales per super-block
};

// Registers between one K step's global loads and its LDS store (thread t's share).
template <int TYPE>
struct KqStage {
    v4i a[2];          // activation codes: 128 rows x 128 B, 16 B chunks t and t + 512
    v4i b;             // weight bytes: Q4_K / Q5_K 16 B of nibbles; Q6_K (t < 256) ql, first half
    v4i b2;            // Q5_K: 16 B of qh; Q6_K: ql, second half
    v4i b3;            // Q6_K: 16 B of qh
    // first half only: t < 128: e0 = the weight row's 16 B of d / dmin / scales (Q6_K: scales),
    // dw = its fp16 d (Q6_K); t >= 128: e0, e1 = the activation row's 16 block sums (int16), dx
    // its d. (One pair of registers for both: loads into different members on the two sides of
    // a branch became one load into a private-memory slot picked by the branch.)
    v4i e0, e1;
    uint32_t dw;
    float dx;
};

__device__ __forceinline__ uint32_t u32(int x) { return (uint32_t) x; }

// 6-bit (scale, min) of sub-block j from ggml's 12 packed bytes (get_scale_min_k4), the bytes
// held 4 per word in w[0..2] (register values: no byte pointer into them).
__device__ __forceinline__ int sbyte(const uint32_t (&w)[3], int k) { return (int) ((w[k >> 2] >> (8 * (k & 3))) & 0xffu); }
__device__ __forceinline__ void scale_min(const uint32_t (&q)[3], int j, int & sc, int & m) {
    if (j < 4) {
        sc = sbyte(q, j) & 63;
        m = sbyte(q, j + 4) & 63;
    } else {
        sc = (sbyte(q, j + 4) & 0xF) | ((sbyte(q, j - 4) >> 6) << 4);
        m = (sbyte(q, j + 4) >> 4) | ((sbyte(q, j) >> 6) << 4);
    }
}

template <int TYPE>
struct KqArgs {
    const uint8_t * w;      // packed weight's low bits: [N][nsb][128] (nibbles / Q6_K's ql)
    const uint16_t * wd;    // Q6_K: fp16 d [N][nsb]
    const uint8_t * wqh;    // Q5_K: the fifth bits [N][nsb][32]; Q6_K: qh [N][nsb][64]
    const uint8_t * whdr;   // Q4_K / Q5_K: the headers (d, dmin, scales[12]) [N][nsb][16]; Q6_K: scales[16]
    const int8_t * xc;      // Q8_K codes [M][K]
    const int16_t * xbs;    // block sums [M][K / 16]
    const float * xd;       // d [M][K / 256]
    float * y;
    const float * res;
    int32_t * raw;          // RAW: the integer parts of super-block raw_sb, [M][N][2] (Q6_K: [M][N][1]), stored
                            // when its second half is done
    int M, N, nsb, ldy, raw_sb;
};

template <int TYPE, int TN>
__device__ __forceinline__ void kq_load(KqStage<TYPE> & st, const KqArgs<TYPE> & a, int m0, int n0, int step) {
    const int t = threadIdx.x;
    const int sb = step >> 1, h = step & 1;
    const int K = a.nsb * 256;
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int c = t + NT * q, row = c >> 3, part = c & 7;
        const int m = min(m0 + row, a.M - 1);
        st.a[q] = *reinterpret_cast<const v4i *>(a.xc + (size_t) m * K + sb * 256 + h * HV + 16 * part);
    }
    if constexpr (TYPE == T_Q6_K) {
        if (t < 2 * TN) {  // row t / 2, bytes l0 .. l0 + 15 of each 32 of the half
            const int row = t >> 1, l0 = 16 * (t & 1);
            const size_t bi = (size_t) min(n0 + row, a.N - 1) * a.nsb + sb;
            const uint8_t * ql = a.w + bi * 128;
            st.b = *reinterpret_cast<const v4i *>(ql + 64 * h + l0);
            st.b2 = *reinterpret_cast<const v4i *>(ql + 64 * h + 32 + l0);
            st.b3 = *reinterpret_cast<const v4i *>(a.wqh + bi * 64 + 32 * h + l0);
        }
    } else if (t < 4 * TN) {
        // row t / 4, u = t % 4: 16 B of nibbles (and Q5_K the matching 16 B of qh)
        const int row = t >> 2, u = t & 3;
        const size_t bi = (size_t) min(n0 + row, a.N - 1) * a.nsb + sb;
        st.b = *reinterpret_cast<const v4i *>(a.w + bi * 128 + 64 * h + 16 * u);
        if constexpr (TYPE == T_Q5_K) st.b2 = *reinterpret_cast<const v4i *>(a.wqh + bi * 32 + 16 * (u & 1));
    }
    if (h == 0) {
        if (t < TN) {
            const size_t bi = (size_t) min(n0 + t, a.N - 1) * a.nsb + sb;
            st.e0 = *reinterpret_cast<const v4i *>(a.whdr + bi * 16);  // header / Q6_K scales
            if constexpr (TYPE == T_Q6_K) st.dw = a.wd[bi];
        } else if (t < TN + TM) {
            const int m = min(m0 + t - TN, a.M - 1);
            st.dx = a.xd[(size_t) m * a.nsb + sb];
            const v4i * bp = reinterpret_cast<const v4i *>(a.xbs + (size_t) m * (a.nsb * 16) + sb * 16);
            st.e1 = bp[1];
            st.e0 = bp[0];  // last, as on the other side: both sides end with a load into e0
        }
    }
}

// LDS of one K step and of one super-block's scales (one copy: the next super-block's are stored
// after a barrier that follows the last use of these, which keeps a workgroup under 80 KB of LDS,
// two of them per CU).
template <int TN>
struct KqLds {
    int8_t A[TM * KP];
    int8_t B[TN * KP];
};
template <int TYPE, int TN>
struct KqScales {
    int8_t sc[TN][Kq<TYPE>::NSUB];  // Q4_K / Q5_K: the 6-bit sc_j; Q6_K: the 16 int8 scales
    int8_t mn[Kq<TYPE>::MIN ? TN : 1][8];  // Q4_K / Q5_K: m_j
    int8_t bh[Kq<TYPE>::MIN ? TM : 1][8], bl[Kq<TYPE>::MIN ? TM : 1][8];  // block sums of sub-block j: 64 bh + bl
    float dw[TN], dm[Kq<TYPE>::MIN ? TN : 1], dx[TM];
};

// Byte-wise: codes in [0, 64) minus 32 as int8.
__device__ __forceinline__ uint32_t minus32(uint32_t v) { return ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }

template <int TYPE, int TN>
__device__ __forceinline__ void kq_store(const KqStage<TYPE> & st, KqLds<TN> & L, KqScales<TYPE, TN> & S, int step) {
    const int t = threadIdx.x;
    const int h = step & 1;
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int c = t + NT * q, row = c >> 3, part = c & 7;
        *reinterpret_cast<v4i *>(L.A + row * KP + 16 * part) = st.a[q];
    }
    if constexpr (TYPE == T_Q6_K) {
        // value r = 32 p + l of the half: low 4 bits from ql (p even: the first 32 bytes, odd: the
        // second; p < 2 low nibbles, else high), 2 high bits from qh[l] >> 2p
        if (t < 2 * TN) {
            const int row = t >> 1, l0 = 16 * (t & 1);
            v4i o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t x = u32(st.b[e]), y = u32(st.b2[e]), hq = u32(st.b3[e]);
                o[0][e] = (int) minus32((x & 0x0F0F0F0Fu) | ((hq & 0x03030303u) << 4));
                o[1][e] = (int) minus32((y & 0x0F0F0F0Fu) | (((hq >> 2) & 0x03030303u) << 4));
                o[2][e] = (int) minus32(((x >> 4) & 0x0F0F0F0Fu) | (((hq >> 4) & 0x03030303u) << 4));
                o[3][e] = (int) minus32(((y >> 4) & 0x0F0F0F0Fu) | (((hq >> 6) & 0x03030303u) << 4));
            }
#pragma unroll
            for (int p = 0; p < 4; p++) *reinterpret_cast<v4i *>(L.B + row * KP + 32 * p + l0) = o[p];
        }
    } else if (t < 4 * TN) {
        // 16 B of nibbles of chunk c = 2h + u / 2 at bytes l0 = 16 (u % 2): low nibbles are values
        // 64c + l0 + k, high ones 64c + 32 + l0 + k; Q5_K adds 16 times bit 2c / 2c + 1 of qh[l0 + k]
        const int row = t >> 2, u = t & 3;
        const int cc = 2 * h + (u >> 1);
        v4i lo, hi;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t x = u32(st.b[k]);
            uint32_t l = x & 0x0F0F0F0Fu, g = (x >> 4) & 0x0F0F0F0Fu;
            if constexpr (TYPE == T_Q5_K) {
                const uint32_t hq = u32(st.b2[k]);
                l |= ((hq >> (2 * cc)) & 0x01010101u) << 4;
                g |= ((hq >> (2 * cc + 1)) & 0x01010101u) << 4;
            }
            lo[k] = (int) l;
            hi[k] = (int) g;
        }
        *reinterpret_cast<v4i *>(L.B + row * KP + 64 * (u >> 1) + 16 * (u & 1)) = lo;
        *reinterpret_cast<v4i *>(L.B + row * KP + 64 * (u >> 1) + 32 + 16 * (u & 1)) = hi;
    }
    if (h == 0) {
        if (t < TN) {
            if constexpr (TYPE == T_Q6_K) {
                *reinterpret_cast<v4i *>(&S.sc[t][0]) = st.e0;
                S.dw[t] = h2f((uint16_t) st.dw);
            } else {
                S.dw[t] = h2f((uint16_t) (u32(st.e0[0]) & 0xffffu));
                S.dm[t] = h2f((uint16_t) (u32(st.e0[0]) >> 16));
                const uint32_t q3[3] = {u32(st.e0[1]), u32(st.e0[2]), u32(st.e0[3])};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    int sc, m;
                    scale_min(q3, j, sc, m);
                    S.sc[t][j] = (int8_t) sc;
                    S.mn[t][j] = (int8_t) m;
                }
            }
        } else if (t < TN + TM) {
            const int row = t - TN;
            S.dx[row] = st.dx;
            if constexpr (Kq<TYPE>::MIN) {
                const uint32_t bw[8] = {u32(st.e0.x), u32(st.e0.y), u32(st.e0.z), u32(st.e0.w),
                                        u32(st.e1.x), u32(st.e1.y), u32(st.e1.z), u32(st.e1.w)};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    // bsums 2j and 2j + 1: the two int16 halves of word j of the 32 bytes
                    const uint32_t wj = bw[j];
                    const int bs = (int) (int16_t) (wj & 0xffffu) + (int) (int16_t) (wj >> 16);  // |bs| <= 32 * 127
                    S.bh[row][j] = (int8_t) (bs >> 6);
                    S.bl[row][j] = (int8_t) (bs & 63);
                }
            }
        }
    }
}

template <int TYPE, bool RAW, int TN>
__global__ __launch_bounds__(NT) void k_gemm_kq(const KqArgs<TYPE> a) {
    constexpr int WN = TN / 32;         // wavefronts along n, each 32 columns
    constexpr int XT = TM / 32 / (8 / WN);  // 32-row MFMA tiles per wavefront: 2 (TN 128) or 1 (TN 64)
    __shared__ __align__(16) KqLds<TN> L[2];
    __shared__ __align__(16) KqScales<TYPE, TN> S;
    const int mt = (a.M + TM - 1) / TM, nt = (a.N + TN - 1) / TN, total = mt * nt;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;  // XCD x holds a contiguous run of tiles
    const int m0 = (id % mt) * TM, n0 = (id / mt) * TN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;  // this wavefront: rows wm * 32 XT + [0, 32 XT), columns wn * 32 + [0, 32)
    const int lr = lane & 31, lk = lane >> 5;
    const int nc = wn * 32 + lr;  // the tile column of this lane's outputs

    float acc[XT][16];
    int i1[XT][16];
#pragma unroll
    for (int x = 0; x < XT; x++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[x][r] = 0.0f, i1[x][r] = 0;

    const int s_begin = RAW ? 2 * a.raw_sb : 0, s_end = RAW ? 2 * a.raw_sb + 2 : 2 * a.nsb;
    KqStage<TYPE> st;
    kq_load<TYPE, TN>(st, a, m0, n0, s_begin);
    kq_store<TYPE, TN>(st, L[0], S, s_begin);
    __syncthreads();

    for (int step = s_begin; step < s_end; step++) {
        const int buf = (step - s_begin) & 1, h = step & 1;
        if (step + 1 < s_end) kq_load<TYPE, TN>(st, a, m0, n0, step + 1);
        const KqLds<TN> & l = L[buf];
        if constexpr (TYPE == T_Q6_K) {
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {  // sub-blocks of 16: v_mfma_i32_32x32x16_i8
                long af[XT];
#pragma unroll
                for (int x = 0; x < XT; x++)
                    af[x] = *reinterpret_cast<const long *>(l.A + (wm * 32 * XT + x * 32 + lr) * KP + 16 * jj + 8 * lk);
                const long bf = *reinterpret_cast<const long *>(l.B + nc * KP + 16 * jj + 8 * lk);
                const int sc = S.sc[nc][8 * h + jj];
#pragma unroll
                for (int x = 0; x < XT; x++) {
                    const v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(af[x], bf, v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) i1[x][r] += sc * c[r];
                }
            }
        } else {
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {  // sub-blocks of 32: v_mfma_i32_32x32x32_i8
                v4i af[XT];
#pragma unroll
                for (int x = 0; x < XT; x++)
                    af[x] = *reinterpret_cast<const v4i *>(l.A + (wm * 32 * XT + x * 32 + lr) * KP + 32 * jj + 16 * lk);
                const v4i bf = *reinterpret_cast<const v4i *>(l.B + nc * KP + 32 * jj + 16 * lk);
                const int sc = S.sc[nc][4 * h + jj];
#pragma unroll
                for (int x = 0; x < XT; x++) {
                    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[x], bf, v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) i1[x][r] += sc * c[r];
                }
            }
        }
        if (h == 1) {  // the super-block is complete: its integer parts into the f32 sums
            v16i i2[XT];
            if constexpr (Kq<TYPE>::MIN) {
                // I2 = sum_j m_j(n) bs_j(m) = 64 (bh . mn) + (bl . mn), K = 8 of 32 (lanes 32..63 and
                // bytes 8..15 zero)
                const int keep = lk ? 0 : -1;
                const int2 m8 = *reinterpret_cast<const int2 *>(&S.mn[nc][0]);
                const v4i bm = v4i{m8.x & keep, m8.y & keep, 0, 0};
#pragma unroll
                for (int x = 0; x < XT; x++) {
                    const int row = wm * 32 * XT + x * 32 + lr;
                    const int2 h8 = *reinterpret_cast<const int2 *>(&S.bh[row][0]);
                    const int2 l8 = *reinterpret_cast<const int2 *>(&S.bl[row][0]);
                    const v4i ah = v4i{h8.x & keep, h8.y & keep, 0, 0};
                    const v4i al = v4i{l8.x & keep, l8.y & keep, 0, 0};
                    const v16i hh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bm, v16i{}, 0, 0, 0);
                    const v16i ll = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bm, v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) i2[x][r] = 64 * hh[r] + ll[r];
                }
            }
            if constexpr (RAW) {  // the one super-block's integers, stored here
                const int n = n0 + nc;
#pragma unroll
                for (int x = 0; x < XT; x++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = m0 + wm * 32 * XT + x * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                        if (m >= a.M || n >= a.N) continue;
                        int32_t * o = a.raw + ((size_t) m * a.N + n) * (Kq<TYPE>::MIN ? 2 : 1);
                        o[0] = i1[x][r];
                        if constexpr (Kq<TYPE>::MIN) o[1] = i2[x][r];
                    }
            } else {
                const float dw = S.dw[nc], dm = Kq<TYPE>::MIN ? S.dm[nc] : 0.0f;
#pragma unroll
                for (int x = 0; x < XT; x++) {
                    // d_x of this lane's rows: element r is row wm*64 + x*32 + 8 (r / 4) + 4 lk + r % 4
                    float4 dxv[4];
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        dxv[q] = *reinterpret_cast<const float4 *>(&S.dx[wm * 32 * XT + x * 32 + 8 * q + 4 * lk]);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float4 d4 = dxv[r >> 2];
                        const float dx = (r & 3) == 0 ? d4.x : (r & 3) == 1 ? d4.y : (r & 3) == 2 ? d4.z : d4.w;
                        float v = dw * (float) i1[x][r];
                        if constexpr (Kq<TYPE>::MIN) v = fmaf(-dm, (float) i2[x][r], v);
                        acc[x][r] = fmaf(dx, v, acc[x][r]);
                        i1[x][r] = 0;
                    }
                }
            }
        }
        if (step + 1 < s_end) {
            if (h == 1) __syncthreads();  // every wavefront is done with this super-block's scales
            kq_store<TYPE, TN>(st, L[buf ^ 1], S, step + 1);
        }
        __syncthreads();
    }

    if constexpr (!RAW) {
        const int n = n0 + nc;
        if (n >= a.N) return;
#pragma unroll
        for (int x = 0; x < XT; x++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 32 * XT + x * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (m >= a.M) continue;
                const size_t o = (size_t) m * a.ldy + n;
                a.y[o] = a.res ? acc[x][r] + a.res[o] : acc[x][r];
            }
        }
    }
}

template <int TYPE, bool RAW>
void run_kq(const void * wv, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
            const float * res, int32_t * raw, int raw_sb, hipStream_t s) {
    // 64-column tiles when 128-column ones would leave CUs without a workgroup
    const bool narrow = ((M + TM - 1) / TM) * ((N + 127) / 128) <= cu_count();
    const int TN = narrow ? 64 : 128;
    const WeightLayout WL = weight_layout(TYPE, N, K);
    const ActLayout AL = act_layout(TYPE, M, K);
    const uint8_t * w = (const uint8_t *) wv;
    const uint8_t * x = (const uint8_t *) act;
    KqArgs<TYPE> a{};
    a.w = w + WL.qs;
    a.wd = TYPE == T_Q6_K ? (const uint16_t *) (w + WL.d) : nullptr;
    a.wqh = TYPE == T_Q4_K ? nullptr : w + WL.qh;
    a.whdr = TYPE == T_Q6_K ? w + WL.sc : w + WL.d;
    a.xc = (const int8_t *) (x + AL.codes);
    a.xbs = (const int16_t *) (x + AL.meta);
    a.xd = (const float *) (x + AL.d);
    a.y = y;
    a.res = res;
    a.raw = raw;
    a.M = (int) M;
    a.N = (int) N;
    a.nsb = (int) (K / 256);
    a.ldy = (int) ldy;
    a.raw_sb = raw_sb;
    const unsigned grid = (unsigned) (((M + TM - 1) / TM) * ((N + TN - 1) / TN));
    if (narrow) k_gemm_kq<TYPE, RAW, 64><<<grid, NT, 0, s>>>(a);
    else k_gemm_kq<TYPE, RAW, 128><<<grid, NT, 0, s>>>(a);
}

}  // namespace

bool gemm_kq_fits(int type, int64_t K) { return is_kquant(type) && K > 0 && K % 256 == 0; }

// ggml_mul_mat of a packed K-quant weight [N][K] with M > 8 Q8_K activation rows (gcq_act_size's
// layout): y[m * ldy + n] (+ res).
void launch_gemm_kq(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                    hipStream_t s, const float * res) {
    require(gemm_kq_fits(type, K), "gemm kq: K-quant weight and K a multiple of 256");
    require(N > 0 && M > 0 && N < INT32_MAX && M < INT32_MAX && ldy < INT32_MAX, "gemm kq: sizes");
    if (type == T_Q4_K) run_kq<T_Q4_K, false>(w, N, K, act, M, y, ldy, res, nullptr, 0, s);
    else if (type == T_Q5_K) run_kq<T_Q5_K, false>(w, N, K, act, M, y, ldy, res, nullptr, 0, s);
    else run_kq<T_Q6_K, false>(w, N, K, act, M, y, ldy, res, nullptr, 0, s);
    check_launch("gemm kq");
}

// The integer parts of super-block sb: out[(m N + n) 2 + {0, 1}] = {I1, I2} (Q4_K / Q5_K), or
// out[m N + n] = I1 (Q6_K).
void launch_gemm_kq_isums(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, int sb,
                          int32_t * out, hipStream_t s) {
    require(gemm_kq_fits(type, K) && sb >= 0 && sb < K / 256, "gemm kq isums: K-quant weight, super-block in range");
    require(N > 0 && M > 0 && N < INT32_MAX && M < INT32_MAX, "gemm kq isums: sizes");
    if (type == T_Q4_K) run_kq<T_Q4_K, true>(w, N, K, act, M, nullptr, 0, nullptr, out, sb, s);
    else if (type == T_Q5_K) run_kq<T_Q5_K, true>(w, N, K, act, M, nullptr, 0, nullptr, out, sb, s);
    else run_kq<T_Q6_K, true>(w, N, K, act, M, nullptr, 0, nullptr, out, sb, s);
    check_launch("gemm kq isums");
}

}  // namespace gcq
