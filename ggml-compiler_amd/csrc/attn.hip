// attn.hip - ggml_flash_attn_ext over an f16 KV cache (runtime/src/ops.cpp:217-243 ->
// runtime/include/ggml_compiler_ops.h:133-136, GGML_PREC_F32), split-K for decode.
//
// Semantics (ggml-cpu flash_attn_ext_f16): Q is rounded to f16 (K's vec_dot type); a key's score
// is (K.Q)*scale + mask; keys whose f16 mask is -inf are skipped; softmax in f32; out = V-sum / S,
// and 0 when no key is visible. Query head h reads KV head h / (H / Hkv) (GQA).
//
// Layout: q[h][s][d] f32 (strides q_h, q_s); k, v [hk][j][d] f16 (strides k_h, k_j / v_h, v_j: a
// view of the first n_kv rows of a [Hkv][max_context][D] cache); mask [s][j] f16 (row stride
// m_s); out [s][h][Dv] f32, ggml's ne = [Dv, H, Sq].
//
// Attention is HBM-bound by the K/V stream. Both kernels split the keys: grid = (split, KV head
// [, query row]), each workgroup streams one contiguous slice of its KV head's rows once and
// serves all G = H/Hkv query heads that share it. One query row (decode) runs k_attn_decode on the
// matrix cores; prompt rows run k_attn_split (D/8 lanes cover one 2*D-byte row; pass 1 forms the
// scores with v_dot2_f32_f16 into LDS, pass 2 the slice's max and exp-sum, pass 3 P.V). A merge
// (k_attn_merge, or the prologue of the GEMV that reads the attention row) combines the splits'
// (max, sum, partial output) exactly as one online softmax would.
#include "gcq_common.h"
#include "attn_lanes.h"

#include <algorithm>

namespace gcq {

int cu_count();

constexpr int kChunkMax = 1024;  // keys per workgroup slice

template <int D, int G>
__global__ __launch_bounds__(256) void k_attn_split(const float * __restrict__ q, int64_t q_h, int64_t q_s,
                                                    const uint16_t * __restrict__ k, int64_t k_h, int64_t k_j,
                                                    const uint16_t * __restrict__ v, int64_t v_h, int64_t v_j,
                                                    const uint16_t * __restrict__ mask, int64_t m_s, float scale,
                                                    int n_kv, int chunk, const int * __restrict__ n_kv_dev,
                                                    float * __restrict__ part_o, float2 * __restrict__ part_ml, int H,
                                                    int nsplit) {
    constexpr int LPK = D / 8;         // lanes per key row
    constexpr int KPW = 64 / LPK;      // keys per wavefront step
    constexpr int KPB = 4 * KPW;       // keys per workgroup step
    constexpr int NB = 8;              // steps per load batch (8 K rows and 8 V rows per lane)
    __shared__ float sc[G][kChunkMax];
    __shared__ float red[4][G];
    __shared__ float accs[4][G][D];

    if (n_kv_dev) {  // KV length read on the device (a captured decode step): same splits, new chunk
        n_kv = *n_kv_dev;
        chunk = (n_kv + nsplit - 1) / nsplit;
    }
    chunk = min(chunk, kChunkMax);  // the host sizes nsplit so that this never drops a key
    const int split = blockIdx.x, hk = blockIdx.y, s = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane % LPK, slot = lane / LPK;
    const int j0 = split * chunk;
    const int j1 = min(n_kv, j0 + chunk);
    const int len = max(0, j1 - j0);

    // This lane's 8 dims of each of the G query heads, rounded to f16.
    half2_t qh[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float * qp = q + (int64_t) (hk * G + g) * q_h + (int64_t) s * q_s + 8 * sub;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            half2_t t;
            t.x = (_Float16) qp[2 * c];
            t.y = (_Float16) qp[2 * c + 1];
            qh[g][c] = t;
        }
    }

    // Pass 1: scores. Keys go in batches of NB steps with every load of a batch issued before
    // any math; the first batch's V rows are loaded with its K rows (they do not depend on the
    // scores), so a slice of up to NB*KPB keys costs one HBM round trip.
    const uint16_t * kb = k + (int64_t) hk * k_h;
    const uint16_t * vb = v + (int64_t) hk * v_h;
    const uint16_t * mrow = mask ? mask + (int64_t) s * m_s : nullptr;
    uint4 vpre[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int jj = b * KPB + wave * KPW + slot;
        vpre[b] = jj < len ? *reinterpret_cast<const uint4 *>(vb + (int64_t) (j0 + jj) * v_j + 8 * sub)
                           : make_uint4(0, 0, 0, 0);
    }
    for (int base = 0; base < len; base += NB * KPB) {
        uint4 kr[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int jj = base + b * KPB + wave * KPW + slot;
            kr[b] = jj < len ? *reinterpret_cast<const uint4 *>(kb + (int64_t) (j0 + jj) * k_j + 8 * sub)
                             : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int jj = base + b * KPB + wave * KPW + slot;
            float part[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float a = 0.0f;
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].x), qh[g][0], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].y), qh[g][1], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].z), qh[g][2], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].w), qh[g][3], a, false);
                part[g] = a;
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                if constexpr (LPK <= 16) part[g] = group_reduce<LPK, float, op_add<float>>(part[g]);
                else part[g] = wave_sum<LPK>(part[g]);
            }
            if (jj < len && sub == 0) {
                const float mv = mrow ? h2f(mrow[j0 + jj]) : 0.0f;
#pragma unroll
                for (int g = 0; g < G; g++) sc[g][jj] = mv == -INFINITY ? -INFINITY : part[g] * scale + mv;
            }
        }
    }
    __syncthreads();

    // Pass 2: max and sum of exp per head over the slice; scores become weights.
    float mx[G], sum[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = -INFINITY;
        for (int i = threadIdx.x; i < len; i += 256) m = fmaxf(m, sc[g][i]);
        m = wave_max(m);
        if (lane == 0) red[wave][g] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) mx[g] = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float l = 0.0f;
        for (int i = threadIdx.x; i < len; i += 256) {
            const float p = mx[g] == -INFINITY ? 0.0f : __expf(sc[g][i] - mx[g]);
            sc[g][i] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) red[wave][g] = l;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) sum[g] = red[0][g] + red[1][g] + red[2][g] + red[3][g];

    // Pass 3: P.V, this lane's 8 dims of one key per step, batches as in pass 1.
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int c = 0; c < 8; c++) acc[g][c] = 0.0f;
    for (int base = 0; base < len; base += NB * KPB) {
        uint4 vr[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int jj = base + b * KPB + wave * KPW + slot;
            if (base == 0) vr[b] = vpre[b];
            else vr[b] = jj < len ? *reinterpret_cast<const uint4 *>(vb + (int64_t) (j0 + jj) * v_j + 8 * sub)
                                  : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int jj = base + b * KPB + wave * KPW + slot;
            if (jj < len) {
                const uint32_t vw[4] = {vr[b].x, vr[b].y, vr[b].z, vr[b].w};
                float vf[8];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    vf[2 * c] = h2f((uint16_t) (vw[c] & 0xffff));
                    vf[2 * c + 1] = h2f((uint16_t) (vw[c] >> 16));
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[g][jj];
#pragma unroll
                    for (int c = 0; c < 8; c++) acc[g][c] += p * vf[c];
                }
            }
        }
    }
    // Reduce over the key slots of a wavefront, then over the 4 wavefronts.
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int o = LPK; o < 64; o <<= 1) acc[g][c] += __shfl_xor(acc[g][c], o, 64);
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int c = 0; c < 8; c++) accs[wave][g][8 * sub + c] = acc[g][c];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        const float o = accs[0][g][d] + accs[1][g][d] + accs[2][g][d] + accs[3][g][d];
        const int h = hk * G + g;
        part_o[(((int64_t) s * H + h) * nsplit + split) * D + d] = o;
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        const int h = hk * G + g;
        part_ml[((int64_t) s * H + h) * nsplit + split] = make_float2(mx[g], sum[g]);
    }
}

// The lane-group kernel (attn_lanes.h): grid (split, KV head, query-head group); workgroups past
// the splits read ahead for the next launches.
template <int D, int G, int NW, bool MASK>
__global__ __launch_bounds__(NW * 64) void k_attn_lanes(int GT, const float * __restrict__ q, int64_t q_h,
                                                         const uint16_t * __restrict__ k, int64_t k_h, int64_t k_j,
                                                         const uint16_t * __restrict__ v, int64_t v_h, int64_t v_j,
                                                         float scale, int n_kv, const int * __restrict__ n_kv_dev,
                                                         int chunk, int kv_rows, int nsplit, float * __restrict__ out,
                                                         float * __restrict__ part_o, float2 * __restrict__ part_ml,
                                                         const Prefetch pf, const uint16_t * __restrict__ mask) {
    __shared__ float so[NW][G * D];
    __shared__ float2 sml[NW][G];
    if ((int) blockIdx.x >= nsplit) {  // a spare workgroup: read ahead for the next launches
        const int w = ((blockIdx.x - nsplit) * gridDim.y + blockIdx.y) * gridDim.z + blockIdx.z;
        prefetch_share(pf, w, NW * 64);
        return;
    }
    if (n_kv_dev) n_kv = *n_kv_dev;
    const int hk = blockIdx.y;
    const int h0 = hk * GT + blockIdx.z * G;  // this workgroup's first query head (GT per KV head)
    attn_lanes_task<D, G, NW, MASK, false>(q, q_h, k, k_h, k_j, v, v_h, v_j, scale, n_kv, chunk, kv_rows, nsplit,
                                           out, part_o, part_ml, mask, blockIdx.x, hk, h0, so, sml, [] {});
}

// Decode attention on the matrix cores: one query row, grid (split, KV head). A workgroup of NW
// wavefronts takes a contiguous slice of its KV head's keys for all G = H / Hkv query heads that
// share them, so each K and V row is read from HBM once. A wavefront takes 16-key blocks of the
// slice (blocks w, w + NW, ...) and per block:
//   - loads the 16 K rows and 16 V rows: in load step s lane (g, c) = (lane / 16, lane % 16)
//     reads dims 32s + 8g .. +8 of key c (16 B; the four lanes of a key read 64 contiguous bytes
//     of its row), the next block's rows in flight while this one is computed;
//   - scores S[key][head] = K·Qᵀ with v_mfma_f32_16x16x32_f16, one per 32 dims: A = the K rows as
//     loaded (lane (g, c) supplies key c, k-index 8g + j = dim 32s + 8g + j), B = Q rounded to
//     f16 (column c = query head c, zero past G). The result leaves keys 4g + r (r < 4) of head c
//     in lane (g, c);
//   - the online softmax of head c over those scores (the block's maximum through two row swaps),
//     rescaling the accumulators;
//   - Oᵀ[dim][head] += Vᵀ·P with v_mfma_f32_16x16x16_f16 per 16 dims: B = P exactly as the scores
//     lie (keys 4g + r of head c, rounded to f16), A = Vᵀ read from LDS, where the wavefront
//     stored its V rows (lane (g, c) gathers dim 16t + c of keys 4g..4g+3; rows padded to keep
//     the four lane groups on distinct banks).
// The accumulators hold dims 16t + 4g + r of head c in lane (g, c). The wavefronts then merge in
// LDS; one split writes the normalized row out[h][d], several write (max, exp-sum, unnormalized
// output) per split in k_attn_split's partial layout, for the merge (k_attn_merge, or a GEMV
// prologue). Numerics: Q·K products of f16 values are exact in f32 and summed in f32; P enters the
// P·V product as two f16 terms (its rounding and the rounding of the remainder, 2^-22 relative
// together), products exact in f32, sums in f32.
//
// Split and block ranges come from the host's chunk, so the first K / V loads do not wait for a
// KV length read from device state; rows are clamped into the kv_rows that exist and keys at or
// past n_kv are masked. MASK: an f16 mask row (n_kv values) is added to the scaled scores, -inf
// dropping a key. Spare workgroups (blockIdx.x >= nsplit) read ahead for the next launches.
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kDecodeWaves = 4;
__host__ __device__ constexpr int decode_keys(int, int) { return 16 * kDecodeWaves; }

template <int D>
__host__ __device__ constexpr size_t decode_lds_bytes(int NW) {
    // max(V rows: NW x 16 x (D + 4) f16, the merge: NW x 8 heads x D f32)
    return (size_t) NW * 16 * (D + 4) * 2 > (size_t) NW * 8 * D * 4 ? (size_t) NW * 16 * (D + 4) * 2
                                                                      : (size_t) NW * 8 * D * 4;
}

template <int D, int NW, bool MASK>
__global__ __launch_bounds__(NW * 64) void k_attn_decode(int G, const float * __restrict__ q, int64_t q_h,
                                                         const uint16_t * __restrict__ k, int64_t k_h, int64_t k_j,
                                                         const uint16_t * __restrict__ v, int64_t v_h, int64_t v_j,
                                                         float scale, int n_kv, const int * __restrict__ n_kv_dev,
                                                         int chunk, int kv_rows, int nsplit, float * __restrict__ out,
                                                         float * __restrict__ part_o, float2 * __restrict__ part_ml,
                                                         const Prefetch pf, const uint16_t * __restrict__ mask) {
    constexpr int KS = D / 32;   // QK k-steps (8 dims of each lane per step)
    constexpr int DT = D / 16;   // P.V dim tiles
    constexpr int LDV = D + 4;   // LDS row of V, in f16
    __shared__ __align__(16) uint8_t lds[decode_lds_bytes<D>(NW)];
    __shared__ float2 sml[NW][16];

    if ((int) blockIdx.x >= nsplit) {  // a spare workgroup: read ahead for the next launches
        prefetch_share(pf, (blockIdx.x - nsplit) * gridDim.y + blockIdx.y, NW * 64);
        return;
    }
    if (n_kv_dev) n_kv = *n_kv_dev;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int j0 = split * chunk;
    const int len = max(0, min(n_kv - j0, chunk));  // keys of this split below n_kv
    const int nblk = (chunk + 15) / 16;             // blocks of the host's chunk
    const int lblk = (len + 15) / 16;               // blocks holding keys below n_kv

    const uint16_t * kb = k + (int64_t) hk * k_h + 8 * g;
    const uint16_t * vb = v + (int64_t) hk * v_h + 8 * g;
    uint4 kf[KS], vf[KS];
    if (wave < nblk) {
        const int64_t row = min(j0 + 16 * wave + c, kv_rows - 1);
#pragma unroll
        for (int s = 0; s < KS; s++) {
            kf[s] = *reinterpret_cast<const uint4 *>(kb + row * k_j + 32 * s);
            vf[s] = *reinterpret_cast<const uint4 *>(vb + row * v_j + 32 * s);
        }
    }

    // Q as the B operand: column c = query head hk * G + c, this lane's k-slices.
    h8_t qb[KS];
    {
        const bool live = c < G;
        const float * qp = q + (int64_t) (hk * G + (live ? c : 0)) * q_h + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const float4 a = *reinterpret_cast<const float4 *>(qp + 32 * s);
            const float4 b = *reinterpret_cast<const float4 *>(qp + 32 * s + 4);
            const float e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; j++) qb[s][j] = live ? (_Float16) e[j] : (_Float16) 0.0f;
        }
    }

    float m = -INFINITY, l = 0.0f;
    f4_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    _Float16 * vl = reinterpret_cast<_Float16 *>(lds) + (size_t) wave * 16 * LDV;

    for (int blk = wave; blk < lblk; blk += NW) {
        // The next block's rows are loaded into the registers of this one as soon as they are
        // consumed (K after the score MFMAs, V after its LDS store), so they are in flight during
        // the rest of this block's work.
        const bool more = blk + NW < lblk;
        const int64_t nrow = min(j0 + 16 * (blk + NW) + c, kv_rows - 1);
        // scores of keys 4g + r, head c
        f4_t S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; s++) {
            h8_t a;
            __builtin_memcpy(&a, &kf[s], 16);
            S = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[s], S, 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int s = 0; s < KS; s++) kf[s] = *reinterpret_cast<const uint4 *>(kb + nrow * k_j + 32 * s);
        }
        float sc[4];
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int jj = 16 * blk + 4 * g + r;
            float x = jj < len ? S[r] * scale : -INFINITY;
            if constexpr (MASK) {
                if (jj < len) {
                    const float mv = h2f(mask[j0 + jj]);
                    x = mv == -INFINITY ? -INFINITY : x + mv;
                }
            }
            sc[r] = x;
            bm = fmaxf(bm, x);
        }
        bm = row_pair<16>(bm, [](float a, float b) { return fmaxf(a, b); });
        bm = row_pair<32>(bm, [](float a, float b) { return fmaxf(a, b); });
        const float mn = fmaxf(m, bm);
        const float f = mn == -INFINITY ? 1.0f : (m == -INFINITY ? 0.0f : __expf(m - mn));
        h4_t pb, pl;  // P = pb + pl: its f16 rounding and the f16 rounding of the remainder
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = sc[r] == -INFINITY ? 0.0f : __expf(sc[r] - mn);
            ps += p;
            pb[r] = (_Float16) p;
            pl[r] = (_Float16) (p - (float) pb[r]);
        }
        l = l * f + ps;
        m = mn;
        // this block's V rows into LDS, then Vᵀ tiles against P
#pragma unroll
        for (int s = 0; s < KS; s++) {  // 8-byte stores: a padded row is 8-byte aligned only
            uint2 * dst = reinterpret_cast<uint2 *>(vl + c * LDV + 32 * s + 8 * g);
            dst[0] = make_uint2(vf[s].x, vf[s].y);
            dst[1] = make_uint2(vf[s].z, vf[s].w);
        }
        if (more) {
#pragma unroll
            for (int s = 0; s < KS; s++) vf[s] = *reinterpret_cast<const uint4 *>(vb + nrow * v_j + 32 * s);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int t = 0; t < DT; t++) {
            h4_t a;
#pragma unroll
            for (int j = 0; j < 4; j++) a[j] = vl[(4 * g + j) * LDV + 16 * t + c];
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[t] * f, 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pl, o[t], 0, 0, 0);
        }
    }
    // the lane groups' exp-sums of head c; max m is already common to them
    l = row_pair<16>(l, [](float a, float b) { return a + b; });
    l = row_pair<32>(l, [](float a, float b) { return a + b; });
    __syncthreads();  // every wavefront is done with its V rows: the LDS now holds outputs
    float * so = reinterpret_cast<float *>(lds);  // [NW][G][D]
    if (c < G) {
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) so[((size_t) wave * G + c) * D + 16 * t + 4 * g + r] = o[t][r];
        if (g == 0) sml[wave][c] = make_float2(m, l);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += NW * 64) {
        const int gg = i / D, d = i % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sml[w][gg].x);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float2 ml = sml[w][gg];
                if (ml.x == -INFINITY) continue;
                const float f = __expf(ml.x - M);
                L += f * ml.y;
                acc += f * so[((size_t) w * G + gg) * D + d];
            }
        }
        const int h = hk * G + gg;
        if (nsplit == 1) {
            out[h * D + d] = L == 0.0f ? 0.0f : acc / L;
        } else {
            part_o[((int64_t) h * nsplit + split) * D + d] = acc;
            if (d == 0) part_ml[(int64_t) h * nsplit + split] = make_float2(M, L);
        }
    }
}

// Combine the splits of one (query row, head): out = sum_i e^(m_i - M) o_i / sum_i e^(m_i - M) l_i.
// One 256-thread workgroup per (query row, head): thread t takes 4 dims (d4 = t % (D/4)) of the
// splits i = t / (D/4) + NG·j (NG = 256 / (D/4) split groups), every partial it needs loaded before
// any math (up to kMergeLoads in flight per thread), so even 1024 splits cost few round trips;
// the split groups then add up in LDS.
constexpr int kMergeMaxSplit = 1024;
constexpr int kMergeLoads = 16;

template <int D>
__global__ __launch_bounds__(256) void k_attn_merge(const float * __restrict__ part_o, const float2 * __restrict__ part_ml,
                                                    float * __restrict__ out, int nsplit) {
    constexpr int Q = D / 4;        // float4 columns
    constexpr int NG = 256 / Q;     // split groups
    __shared__ float2 sml[kMergeMaxSplit];
    __shared__ float red[4], red_l[4];
    __shared__ float4 acc_s[NG][Q];
    const int64_t sh = blockIdx.x;  // s * H + h
    const int t = threadIdx.x, d4 = t % Q, sg = t / Q;
    const float2 * ml = part_ml + sh * nsplit;
    float M = -INFINITY;
    for (int i = t; i < nsplit; i += 256) {
        const float2 v = ml[i];
        sml[i] = v;
        M = fmaxf(M, v.x);
    }
    M = wave_max(M);
    if ((t & 63) == 0) red[t >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.0f;  // sum_i e^(m_i - M) l_i
    if (M != -INFINITY)
        for (int i = t; i < nsplit; i += 256) {
            const float2 v = sml[i];
            if (v.x != -INFINITY) L += __expf(v.x - M) * v.y;
        }
    L = wave_sum(L);
    if ((t & 63) == 0) red_l[t >> 6] = L;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (M != -INFINITY) {
        const float4 * po = reinterpret_cast<const float4 *>(part_o + sh * nsplit * D) + d4;
        for (int i0 = sg; i0 < nsplit; i0 += NG * kMergeLoads) {
            float4 pv[kMergeLoads];
#pragma unroll
            for (int j = 0; j < kMergeLoads; j++) pv[j] = po[(int64_t) min(i0 + NG * j, nsplit - 1) * Q];
#pragma unroll
            for (int j = 0; j < kMergeLoads; j++) {
                const int i = i0 + NG * j;
                if (i >= nsplit) break;
                const float2 ml_i = sml[i];
                if (ml_i.x == -INFINITY) continue;
                const float w = __expf(ml_i.x - M);
                o.x += w * pv[j].x;
                o.y += w * pv[j].y;
                o.z += w * pv[j].z;
                o.w += w * pv[j].w;
            }
        }
    }
    acc_s[sg][d4] = o;
    __syncthreads();
    if (t < Q) {
        float4 r = acc_s[0][t];
        for (int g = 1; g < NG; g++) {
            const float4 a = acc_s[g][t];
            r.x += a.x;
            r.y += a.y;
            r.z += a.z;
            r.w += a.w;
        }
        const float Lt = red_l[0] + red_l[1] + red_l[2] + red_l[3];
        const float4 y = Lt == 0.0f ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                    : make_float4(r.x / Lt, r.y / Lt, r.z / Lt, r.w / Lt);
        reinterpret_cast<float4 *>(out + sh * D)[t] = y;
    }
}

// ------------------------------------------------------------------------------- dispatch

AttnPlan attn_plan(int Sq, int Hkv, int n_kv) {
    int nsplit = (n_kv + 63) / 64;
    const int target = 1024 / max(1, Hkv * Sq);  // about 4 workgroups per CU in all
    nsplit = max(1, min(nsplit, max(1, target)));
    int chunk = (n_kv + nsplit - 1) / nsplit;
    if (chunk > kChunkMax) {
        nsplit = (n_kv + kChunkMax - 1) / kChunkMax;
        chunk = (n_kv + nsplit - 1) / nsplit;
    }
    return {nsplit, max(chunk, 1)};
}

// Decode attention has two kernels: up to kLanesMaxKv keys the lane-group kernel (k_attn_lanes,
// one query head per workgroup: four times the workgroups of one per KV head, K / V re-read from
// L2), beyond that the matrix-core kernel (k_attn_decode, every query head of a KV head per
// workgroup, each K / V row read once). The planners and the launcher pick by the largest KV
// length a launch may see (max_kv: n_kv, or the cache rows when the length is read on the device).
constexpr int kLanesMaxKv = 2048;
bool decode_lanes(int max_kv) { return max_kv <= kLanesMaxKv; }

// Query heads one decode workgroup takes of its KV head's GT.
int decode_group(int GT, int max_kv) { return decode_lanes(max_kv) ? 1 : GT; }

// The decode split count for n_kv keys and H query heads, at most max_split splits:
//   - lane groups, wide (the decode step's plan: its output projection merges the splits in its
//     prologue, which every workgroup repeats, so fewer splits): one 16-wavefront load batch per
//     split, 16 wavefronts each;
//   - lane groups, not wide (a merge kernel follows): a split per four wavefronts' load batches
//     (64 keys at D = 128), at most 512 / H splits, 4-16 wavefronts each (lanes_nw). Measured on
//     MI355X (32 query heads on 8 KV heads of 128): 512-2048 wavefronts in all end soonest, the
//     first loads of more queue behind the others';
//   - matrix cores: one 16-key block per wavefront of a 4-wavefront workgroup (the wavefronts then
//     take several).
int decode_splits(int D, int H, int G, int n_kv, int max_split, bool wide) {
    int per = decode_keys(D, G);
    if (decode_lanes(n_kv)) {
        if (!wide) {
            per = 4 * lanes_batch(D, 1);
            max_split = std::min(max_split, std::max(1, 512 / std::max(1, H)));
        } else {
            per = lanes_keys(D, 1);
        }
    }
    return std::max(1, std::min(max_split, (n_kv + per - 1) / per));
}

// Decode (one query row, captured once for every KV length up to max_ctx): the wide split count
// for max_ctx keys; the KV length itself is read on the device and each split takes an equal share.
AttnPlan attn_plan_decode(int D, int H, int G, int max_ctx, int max_split) {
    const int nsplit = decode_splits(D, H, decode_group(G, max_ctx), max_ctx, max_split, true);
    return {nsplit, (max_ctx + nsplit - 1) / nsplit};
}

bool attn_decode_fits(int D, int G) { return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 4 || G == 8); }

// out [H*D] (one split) or part_o / part_ml (several), q [H][D] at head stride q_h.
// chunk: keys per split (nsplit * chunk >= n_kv); kv_rows: rows the K and V buffers hold per head;
// GS: query heads per workgroup (decode_group). pf (optional): byte ranges that about as many spare
// workgroups as leave the CUs one each read ahead into the Infinity Cache.
// nw_lanes: wavefronts per lane-group split (4, 8 or 16; 16 for a wide plan), or 0 for lanes_nw's
// choice.
void launch_attn_decode(const float * q, int64_t q_h, const void * k, int64_t k_h, int64_t k_j, const void * v,
                        int64_t v_h, int64_t v_j, int D, int H, int Hkv, int n_kv, const int * n_kv_dev, float scale,
                        int nsplit, int chunk, int kv_rows, int GS, float * out, float * part_o, float2 * part_ml,
                        hipStream_t s, const Prefetch * pf,
                        const void * mask, int nw_lanes) {
    const int G = H / Hkv;
    require(attn_decode_fits(D, G) && H % Hkv == 0, "attn decode: D 64 / 128 and 1, 2, 4 or 8 query heads per KV head");
    const bool lanes = decode_lanes(n_kv_dev ? kv_rows : n_kv);
    require(GS == decode_group(G, n_kv_dev ? kv_rows : n_kv), "attn decode: head group does not match the plan");
    require(kv_rows >= 1 && chunk >= 1 && (int64_t) nsplit * chunk >= (n_kv_dev ? kv_rows : n_kv),
            "attn decode: the splits must cover the keys");
    require(k_j % 8 == 0 && v_j % 8 == 0 && k_h % 8 == 0 && v_h % 8 == 0 && q_h % 4 == 0 &&
                ((uintptr_t) q & 15) == 0 && ((uintptr_t) k & 15) == 0 && ((uintptr_t) v & 15) == 0,
            "attn decode: 16-byte aligned K / V rows and q heads");
    const int per_slot = Hkv * (G / GS);  // workgroups per split
    Prefetch P{};
    int extra = 0;  // spare split slots: extra * per_slot prefetching workgroups
    if (pf && (pf->n[0] || pf->n[1])) {
        require(pf->sink && pf->n[0] % 16 == 0 && pf->n[1] % 16 == 0, "attn decode: prefetch ranges of 16 B");
        const int spare = cu_count() - nsplit * per_slot;
        extra = std::max(0, spare / per_slot);
        P = *pf;
        P.wgs = extra * per_slot;
    }
    const uint16_t *kp = (const uint16_t *) k, *vp = (const uint16_t *) v;
    const uint16_t * mp = (const uint16_t *) mask;
    if (lanes) {
        const dim3 grid((unsigned) (nsplit + extra), (unsigned) Hkv, (unsigned) (G / GS));
        const int nw = nw_lanes ? nw_lanes : lanes_nw(D, 1, chunk);
        require(nw == 4 || nw == 8 || nw == 16, "attn decode: 4, 8 or 16 wavefronts per split");
#define GCQ_AL(DD, NW)                                                                                          \
    if (D == DD && nw == NW) {                                                                                  \
        if (mp)                                                                                                 \
            k_attn_lanes<DD, 1, NW, true><<<grid, NW * 64, 0, s>>>(G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale,   \
                                                               n_kv, n_kv_dev, chunk, kv_rows, nsplit, out,     \
                                                               part_o, part_ml, P, mp);                         \
        else                                                                                                    \
            k_attn_lanes<DD, 1, NW, false><<<grid, NW * 64, 0, s>>>(G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale,  \
                                                                n_kv, n_kv_dev, chunk, kv_rows, nsplit, out,    \
                                                                part_o, part_ml, P, nullptr);                   \
    }
        GCQ_AL(64, 4) GCQ_AL(64, 8) GCQ_AL(64, 16) GCQ_AL(128, 4) GCQ_AL(128, 8) GCQ_AL(128, 16)
#undef GCQ_AL
        check_launch("attn decode");
        return;
    }
    const dim3 grid((unsigned) (nsplit + extra), (unsigned) Hkv);
    // wavefronts: one per 16-key block of a split, 4 to 16
    const int blocks = (chunk + 15) / 16;
    const int nw = blocks <= 4 ? 4 : blocks <= 8 ? 8 : 16;
#define GCQ_AD(DD, NW)                                                                                                 \
    if (D == DD && nw == NW) {                                                                                         \
        if (mp)                                                                                                        \
            k_attn_decode<DD, NW, true><<<grid, NW * 64, 0, s>>>(G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale, n_kv,   \
                                                                 n_kv_dev, chunk, kv_rows, nsplit, out, part_o,      \
                                                                 part_ml, P, mp);                                     \
        else                                                                                                           \
            k_attn_decode<DD, NW, false><<<grid, NW * 64, 0, s>>>(G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale, n_kv,  \
                                                                  n_kv_dev, chunk, kv_rows, nsplit, out, part_o,     \
                                                                  part_ml, P, nullptr);                              \
    }
    GCQ_AD(64, 4) GCQ_AD(128, 4) GCQ_AD(64, 8) GCQ_AD(128, 8) GCQ_AD(64, 16) GCQ_AD(128, 16)
#undef GCQ_AD
    check_launch("attn decode");
}

size_t attn_workspace(int Sq, int H, int Hkv, int Dv, int n_kv) {
    const AttnPlan p = attn_plan(Sq, Hkv, n_kv);
    return align256((size_t) Sq * H * p.nsplit * Dv * sizeof(float)) +
           align256((size_t) Sq * H * p.nsplit * sizeof(float2));
}

template <int D>
static void run_split(int G, const float * q, int64_t q_h, int64_t q_s, const uint16_t * k, int64_t k_h, int64_t k_j,
                      const uint16_t * v, int64_t v_h, int64_t v_j, const uint16_t * mask, int64_t m_s, int Sq, int H,
                      int Hkv, int n_kv, float scale, float * po, float2 * pml, const AttnPlan & p,
                      const int * n_kv_dev, hipStream_t s) {
    const dim3 grid((unsigned) p.nsplit, (unsigned) Hkv, (unsigned) Sq);
#define GCQ_A(GG)                                                                                                  \
    k_attn_split<D, GG><<<grid, 256, 0, s>>>(q, q_h, q_s, k, k_h, k_j, v, v_h, v_j, mask, m_s, scale, n_kv, p.chunk, \
                                             n_kv_dev, po, pml, H, p.nsplit)
    switch (G) {
        case 1: GCQ_A(1); break;
        case 2: GCQ_A(2); break;
        case 3: GCQ_A(3); break;
        case 4: GCQ_A(4); break;
        case 5: GCQ_A(5); break;
        case 6: GCQ_A(6); break;
        case 7: GCQ_A(7); break;
        case 8: GCQ_A(8); break;
        default: fail("flash_attn: at most 8 query heads per KV head are supported");
    }
#undef GCQ_A
    check_launch("flash_attn split");
}

// Split pass only: partials into (po, pml) sized for plan p. With n_kv_dev, the KV length is read
// on the device (n_kv is then the largest it may be, which p was planned for).
void launch_attn_split(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                       const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, int D, int Sq, int H,
                       int Hkv, int n_kv, float scale, float * po, float2 * pml, const AttnPlan & p,
                       const int * n_kv_dev, hipStream_t s) {
    require(D == 64 || D == 128 || D == 256, "flash_attn: head size must be 64, 128 or 256");
    require(H % Hkv == 0, "flash_attn: query heads must be a multiple of KV heads");
    require((int64_t) p.nsplit * kChunkMax >= n_kv, "flash_attn: too few splits for the KV length");
    const int G = H / Hkv;
    const uint16_t * kk = (const uint16_t *) k;
    const uint16_t * vv = (const uint16_t *) v;
    const uint16_t * mm = (const uint16_t *) mask;
    if (D == 64) run_split<64>(G, q, q_h, q_s, kk, k_h, k_j, vv, v_h, v_j, mm, m_s, Sq, H, Hkv, n_kv, scale, po, pml, p, n_kv_dev, s);
    else if (D == 128) run_split<128>(G, q, q_h, q_s, kk, k_h, k_j, vv, v_h, v_j, mm, m_s, Sq, H, Hkv, n_kv, scale, po, pml, p, n_kv_dev, s);
    else run_split<256>(G, q, q_h, q_s, kk, k_h, k_j, vv, v_h, v_j, mm, m_s, Sq, H, Hkv, n_kv, scale, po, pml, p, n_kv_dev, s);
}

void launch_flash_attn(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                       const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, float * out, int D,
                       int Dv, int Sq, int H, int Hkv, int n_kv, float scale, void * ws, size_t ws_size,
                       hipStream_t s) {
    require(D == Dv, "flash_attn: K and V head sizes must match");
    const AttnPlan p = attn_plan(Sq, Hkv, n_kv);
    require(p.nsplit <= kMergeMaxSplit, "flash_attn: n_kv above 1024 * 1024 keys");  // k_attn_merge's LDS
    require(ws_size >= attn_workspace(Sq, H, Hkv, Dv, n_kv), "flash_attn: workspace too small");
    float * po = (float *) ws;
    float2 * pml = (float2 *) ((uint8_t *) ws + align256((size_t) Sq * H * p.nsplit * Dv * sizeof(float)));
    if (Sq == 1 && H % Hkv == 0 && attn_decode_fits(D, H / Hkv)) {
        // One query row (its mask row added to the scores, if any): the one-pass decode kernel
        // (fewer splits than p, so the workspace holds its partials).
        const int GS = decode_group(H / Hkv, n_kv);
        // one 16-key block per wavefront, at most about one workgroup per CU (longer contexts take
        // more blocks per wavefront: fewer partials to merge)
        const int nsplit = decode_splits(D, H, GS, n_kv, std::min(p.nsplit, std::max(1, cu_count() / Hkv)), false);
        launch_attn_decode(q, q_h, k, k_h, k_j, v, v_h, v_j, D, H, Hkv, n_kv, nullptr, scale, nsplit,
                           (n_kv + nsplit - 1) / nsplit, n_kv, GS, out, po, pml, s, nullptr, mask, 0);
        if (nsplit == 1) return;
        if (D == 64) k_attn_merge<64><<<(unsigned) H, 256, 0, s>>>(po, pml, out, nsplit);
        else k_attn_merge<128><<<(unsigned) H, 256, 0, s>>>(po, pml, out, nsplit);
        check_launch("flash_attn merge");
        return;
    }
    launch_attn_split(q, q_h, q_s, k, k_h, k_j, v, v_h, v_j, mask, m_s, D, Sq, H, Hkv, n_kv, scale, po, pml, p,
                      nullptr, s);
    if (D == 64) k_attn_merge<64><<<(unsigned) (Sq * H), 256, 0, s>>>(po, pml, out, p.nsplit);
    else if (D == 128) k_attn_merge<128><<<(unsigned) (Sq * H), 256, 0, s>>>(po, pml, out, p.nsplit);
    else k_attn_merge<256><<<(unsigned) (Sq * H), 256, 0, s>>>(po, pml, out, p.nsplit);
    check_launch("flash_attn merge");
}

}  // namespace gcq
