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
// Decode is HBM-bound by the K/V stream. Grid = (split, KV head, query row): each workgroup
// streams one contiguous slice of its KV head's rows once and serves all G = H/Hkv query heads
// that share it. D/8 lanes cover one 2*D-byte row (16 B per lane, 8 f16), so a wavefront reads
// 64*16 B of consecutive rows per instruction. Pass 1 forms the scores (v_dot2_f32_f16 on f16 Q
// and K) into LDS; pass 2 is the slice's max and exp-sum; pass 3 accumulates P.V. A merge
// kernel combines the splits' (max, sum, partial output) exactly as one online softmax would.
#include "gcq_common.h"

#include <algorithm>

namespace gcq {

int cu_count();

constexpr int kChunkMax = 1024;  // keys per workgroup slice

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t u) {
    half2_t h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

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

// Decode attention: one query row, every key below n_kv visible (no mask), grid (split, KV head),
// NW wavefronts. Each wavefront takes a contiguous run of the split's keys; its lanes work in
// groups of D/8 (8 dims, 16 B of a K or V row each) and every lane group keeps its own online
// softmax per query head (running max m, exp-sum l, P.V accumulator) over load batches of NB
// keys, K and V rows of a batch loaded together, so no reduction crosses lane groups inside the
// loop. The lane groups and then the NW wavefronts are merged at the end (shuffles, LDS). One
// split: the normalized output out[h][d]; several: the split's (max, exp-sum, unnormalized output)
// in k_attn_split's partial layout, for the merge (k_attn_merge, or a GEMV prologue). The host
// sizes splits so that each wavefront's keys are one load batch (decode_keys).
//
// Wavefronts per k_attn_decode workgroup: 16, or 8 for four query heads per KV head (whose
// registers need two wavefronts' share); steps per load batch: 4, or 2 for four query heads (with
// four heads' accumulators per lane the two-step batch measures about 11% faster at 32768 keys and
// the same at 4096 and below); keys one workgroup loads in one batch per wavefront.
__host__ __device__ constexpr int decode_waves(int G) { return G >= 4 ? 8 : 16; }
__host__ __device__ constexpr int decode_nb(int G) { return G >= 4 ? 2 : 4; }
__host__ __device__ constexpr int decode_keys(int D, int G) { return decode_waves(G) * (64 / (D / 8)) * decode_nb(G); }

// f16 value c (0..7) of 8 packed in a uint4, as f32.
__device__ __forceinline__ float half_at(const uint4 & r, int c) {
    const uint32_t w = c < 2 ? r.x : c < 4 ? r.y : c < 6 ? r.z : r.w;
    return h2f((uint16_t) (c & 1 ? w >> 16 : w & 0xffff));
}

// MASK: an f16 mask row (n_kv values, ggml's [n_kv, 1] mask of one query row) is added to the
// scaled scores, -inf dropping a key.
template <int D, int G, int NW, bool MASK>
__global__ __launch_bounds__(NW * 64) void k_attn_decode(int GT, const float * __restrict__ q, int64_t q_h,
                                                         const uint16_t * __restrict__ k, int64_t k_h, int64_t k_j,
                                                         const uint16_t * __restrict__ v, int64_t v_h, int64_t v_j,
                                                         float scale, int n_kv, const int * __restrict__ n_kv_dev,
                                                         int chunk, int kv_rows, int nsplit, float * __restrict__ out,
                                                         float * __restrict__ part_o, float2 * __restrict__ part_ml,
                                                         const Prefetch pf, const uint16_t * __restrict__ mask) {
    constexpr int LPK = D / 8;     // lanes per key row
    constexpr int KPW = 64 / LPK;  // lane groups (keys per step) per wavefront
    constexpr int NB = decode_nb(G);  // steps per load batch
    static_assert(G * D <= NW * 64, "one output per thread in the merge");
    static_assert(NW == decode_waves(G) && NW * KPW * NB == decode_keys(D, G), "decode split size");
    __shared__ float so[NW][G * D];
    __shared__ float2 sml[NW][G];

    // Split and wavefront ranges come from the host's chunk, so the K/V addresses do not wait for
    // the KV length read from the device; rows are clamped into the kv_rows that exist and keys
    // at or past n_kv are masked.
    if ((int) blockIdx.x >= nsplit) {  // a spare workgroup: read ahead for the next launches
        const int w = ((blockIdx.x - nsplit) * gridDim.y + blockIdx.y) * gridDim.z + blockIdx.z;
        prefetch_share(pf, w, NW * 64);
        return;
    }
    if (n_kv_dev) n_kv = *n_kv_dev;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int h0 = hk * GT + blockIdx.z * G;  // this workgroup's first query head (GT per KV head)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane % LPK, slot = lane / LPK;
    const int j0 = split * chunk;
    const int per_wave = (chunk + NW - 1) / NW;
    const int w0 = min(chunk, wave * per_wave), w1 = min(chunk, w0 + per_wave);
    const int len = max(0, min(n_kv - j0, chunk));  // keys of this split below n_kv

    // q, then the first batch of K / V rows, are in flight before q is converted (the K / V
    // loads do not wait for q).
    float4 qf[G][2];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float * qp = q + (int64_t) (h0 + g) * q_h + 8 * sub;
        qf[g][0] = *reinterpret_cast<const float4 *>(qp);
        qf[g][1] = *reinterpret_cast<const float4 *>(qp + 4);
    }
    const uint16_t * kb = k + (int64_t) hk * k_h + 8 * sub;
    const uint16_t * vb = v + (int64_t) hk * v_h + 8 * sub;
    uint4 kr[NB], vr[NB];
    uint16_t mk[NB];
    auto load = [&](int base) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int64_t row = min(j0 + base + b * KPW + slot, kv_rows - 1);
            kr[b] = *reinterpret_cast<const uint4 *>(kb + row * k_j);
            vr[b] = *reinterpret_cast<const uint4 *>(vb + row * v_j);
            if constexpr (MASK) mk[b] = mask[min(j0 + base + b * KPW + slot, n_kv - 1)];
        }
    };
    if (w0 < w1) load(w0);
    __builtin_amdgcn_sched_barrier(0);  // all of the batch's loads issued before any wait
    half2_t qh[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 f = qf[g][c / 2];
            half2_t t;
            t.x = (_Float16) ((c & 1) ? f.z : f.x);
            t.y = (_Float16) ((c & 1) ? f.w : f.y);
            qh[g][c] = t;
        }
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) acc[g][c] = 0.0f;
    }
    for (int base = w0; base < w1; base += NB * KPW) {
        if (base != w0) load(base);
        __builtin_amdgcn_sched_barrier(0);
        float vf[NB][8];  // this lane's 8 dims of each key's V row, converted once for all G heads
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int c = 0; c < 8; c++) vf[b][c] = half_at(vr[b], c);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float sc[NB];
            float bm = -INFINITY;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float a = 0.0f;
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].x), qh[g][0], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].y), qh[g][1], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].z), qh[g][2], a, false);
                a = __builtin_amdgcn_fdot2(as_h2(kr[b].w), qh[g][3], a, false);
                a = group_reduce<LPK, float, op_add<float>>(a);
                const int jj = base + b * KPW + slot;
                if constexpr (MASK) sc[b] = jj < w1 && jj < len ? a * scale + h2f(mk[b]) : -INFINITY;
                else sc[b] = jj < w1 && jj < len ? a * scale : -INFINITY;
                bm = fmaxf(bm, sc[b]);
            }
            const float mn = fmaxf(m[g], bm);
            if (mn == -INFINITY) continue;  // no key of this lane group yet
            const float f = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
            float p[NB];
            float ps = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                p[b] = sc[b] == -INFINITY ? 0.0f : __expf(sc[b] - mn);
                ps += p[b];
            }
            l[g] = l[g] * f + ps;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                float t = acc[g][c] * f;
#pragma unroll
                for (int b = 0; b < NB; b++) t += p[b] * vf[b][c];
                acc[g][c] = t;
            }
            m[g] = mn;
        }
    }
    // Merge the wavefront's lane groups (same sub, slots 0..KPW-1), then the NW wavefronts.
    // Reduction over the slots (lanes sub, sub + LPK, ...): lane ^ 8 for the 8-lane slots of
    // D = 64, then the row swaps.
    auto slots = [&](float v, auto f) {
        if constexpr (LPK == 8) v = f(v, lane_xor8(v));
        v = row_pair<16>(v, f);
        return row_pair<32>(v, f);
    };
    auto fmax2 = [](float a, float b) { return fmaxf(a, b); };
    auto add2 = [](float a, float b) { return a + b; };
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float M = slots(m[g], fmax2);
        const float f = m[g] == -INFINITY ? 0.0f : __expf(m[g] - M);
        l[g] = slots(l[g] * f, add2);
#pragma unroll
        for (int c = 0; c < 8; c++) acc[g][c] = slots(acc[g][c] * f, add2);
        m[g] = M;
    }
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int c = 0; c < 8; c++) so[wave][g * D + 8 * sub + c] = acc[g][c];
    }
    if (lane < G) {
#pragma unroll
        for (int g = 0; g < G; g++)
            if (lane == g) sml[wave][g] = make_float2(m[g], l[g]);
    }
    __syncthreads();
    const int i = threadIdx.x;
    if (i < G * D) {
        const int g = i / D, d = i % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sml[w][g].x);
        float L = 0.0f, o = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float2 ml = sml[w][g];
                if (ml.x == -INFINITY) continue;
                const float f = __expf(ml.x - M);
                L += f * ml.y;
                o += f * so[w][i];
            }
        }
        const int h = h0 + g;
        if (nsplit == 1) {
            out[h * D + d] = L == 0.0f ? 0.0f : o / L;
        } else {
            part_o[((int64_t) h * nsplit + split) * D + d] = o;
            if (d == 0) part_ml[(int64_t) h * nsplit + split] = make_float2(M, L);
        }
    }
}

// Combine the splits of one (query row, head): out = sum_i e^(m_i - M) o_i / sum_i e^(m_i - M) l_i.
// D threads; the (max, sum) pairs go through LDS once, and each thread's partials are loaded 8 at a
// time before any math, so a long context's many splits cost few round trips.
template <int D>
__global__ __launch_bounds__(D) void k_attn_merge(const float * __restrict__ part_o, const float2 * __restrict__ part_ml,
                                                  float * __restrict__ out, int nsplit) {
    constexpr int kMaxSplit = 1024;
    __shared__ float2 sml[kMaxSplit];
    __shared__ float red[D / 64 > 0 ? D / 64 : 1];
    const int64_t sh = blockIdx.x;  // s * H + h
    const int d = threadIdx.x;
    const float2 * ml = part_ml + sh * nsplit;
    float M = -INFINITY;
    for (int i = d; i < nsplit; i += D) {
        const float2 t = ml[i];
        sml[i] = t;
        M = fmaxf(M, t.x);
    }
    M = wave_max<(D < 64 ? D : 64)>(M);
    if constexpr (D > 64) {
        if ((d & 63) == 0) red[d >> 6] = M;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < D / 64; w++) M = fmaxf(M, red[w]);
    }
    __syncthreads();
    float L = 0.0f, o = 0.0f;
    if (M != -INFINITY) {
        const float * po = part_o + sh * nsplit * D + d;
        for (int i0 = 0; i0 < nsplit; i0 += 8) {
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) pv[j] = po[(int64_t) min(i0 + j, nsplit - 1) * D];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (i0 + j >= nsplit) break;
                const float2 t = sml[i0 + j];
                if (t.x == -INFINITY) continue;
                const float w = __expf(t.x - M);
                L += w * t.y;
                o += w * pv[j];
            }
        }
    }
    out[sh * D + d] = L == 0.0f ? 0.0f : o / L;
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

// Query heads one k_attn_decode workgroup takes of its KV head's GT: all of them (each K/V row read
// once) for long contexts, one (4x the workgroups, a quarter of the arithmetic each, K/V re-read
// from L2) up to 4096 keys, where the kernel is bound by latency and arithmetic, not HBM.
int decode_group(int GT, int max_kv) { return max_kv <= 4096 ? 1 : GT; }

// k_attn_decode's split count for n_kv keys: one load batch per wavefront, at most max_split
// splits (the wavefronts then take several batches).
int decode_splits(int D, int G, int n_kv, int max_split) {
    return max(1, min(max_split, (n_kv + decode_keys(D, G) - 1) / decode_keys(D, G)));
}

// Decode (one query row, captured once for every KV length up to max_ctx): the split count for
// max_ctx keys; the KV length itself is read on the device and each split takes an equal share.
AttnPlan attn_plan_decode(int D, int G, int max_ctx, int max_split) {
    const int nsplit = decode_splits(D, decode_group(G, max_ctx), max_ctx, max_split);
    return {nsplit, (max_ctx + nsplit - 1) / nsplit};
}

bool attn_decode_fits(int D, int G) { return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 4); }

// out [H*D] (one split) or part_o / part_ml (several), q [H][D] at head stride q_h.
// chunk: keys per split (nsplit * chunk >= n_kv); kv_rows: rows the K and V buffers hold per head;
// GS: query heads per workgroup (decode_group). pf (optional): byte ranges that about as many spare
// workgroups as leave the CUs one each read ahead into the Infinity Cache.
void launch_attn_decode(const float * q, int64_t q_h, const void * k, int64_t k_h, int64_t k_j, const void * v,
                        int64_t v_h, int64_t v_j, int D, int H, int Hkv, int n_kv, const int * n_kv_dev, float scale,
                        int nsplit, int chunk, int kv_rows, int GS, float * out, float * part_o, float2 * part_ml,
                        hipStream_t s, const Prefetch * pf,
                        const void * mask) {
    const int G = H / Hkv;
    require(attn_decode_fits(D, G) && H % Hkv == 0, "attn decode: D 64 / 128 and 1, 2 or 4 query heads per KV head");
    require(GS >= 1 && G % GS == 0, "attn decode: head group must divide the query heads per KV head");
    require(kv_rows >= 1 && chunk >= 1 && (int64_t) nsplit * chunk >= (n_kv_dev ? kv_rows : n_kv),
            "attn decode: the splits must cover the keys");
    Prefetch P{};
    int extra = 0;  // spare split slots: extra * Hkv * (G / GS) prefetching workgroups
    if (pf && (pf->n[0] || pf->n[1])) {
        require(pf->sink && pf->n[0] % 16 == 0 && pf->n[1] % 16 == 0, "attn decode: prefetch ranges of 16 B");
        const int per_slot = Hkv * (G / GS);
        const int spare = cu_count() - nsplit * per_slot;
        extra = std::max(0, spare / per_slot);
        P = *pf;
        P.wgs = extra * per_slot;
    }
    const dim3 grid((unsigned) (nsplit + extra), (unsigned) Hkv, (unsigned) (G / GS));
    const uint16_t *kp = (const uint16_t *) k, *vp = (const uint16_t *) v;
    const uint16_t * mp = (const uint16_t *) mask;
#define GCQ_AD(DD, GG)                                                                                          \
    if (D == DD && GS == GG) {                                                                                  \
        if (mp)                                                                                                 \
            k_attn_decode<DD, GG, decode_waves(GG), true><<<grid, decode_waves(GG) * 64, 0, s>>>(               \
                G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale, n_kv, n_kv_dev, chunk, kv_rows, nsplit, out, part_o, \
                part_ml, P, mp);                                                                                \
        else                                                                                                    \
            k_attn_decode<DD, GG, decode_waves(GG), false><<<grid, decode_waves(GG) * 64, 0, s>>>(              \
                G, q, q_h, kp, k_h, k_j, vp, v_h, v_j, scale, n_kv, n_kv_dev, chunk, kv_rows, nsplit, out, part_o, \
                part_ml, P, nullptr);                                                                           \
    }
    GCQ_AD(64, 1) GCQ_AD(64, 2) GCQ_AD(64, 4) GCQ_AD(128, 1) GCQ_AD(128, 2) GCQ_AD(128, 4)
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
    require(p.nsplit <= 1024, "flash_attn: n_kv above 1024 * 1024 keys");  // k_attn_merge's LDS
    require(ws_size >= attn_workspace(Sq, H, Hkv, Dv, n_kv), "flash_attn: workspace too small");
    float * po = (float *) ws;
    float2 * pml = (float2 *) ((uint8_t *) ws + align256((size_t) Sq * H * p.nsplit * Dv * sizeof(float)));
    if (Sq == 1 && H % Hkv == 0 && attn_decode_fits(D, H / Hkv)) {
        // One query row (its mask row added to the scores, if any): the one-pass decode kernel
        // (fewer splits than p, so the workspace holds its partials).
        const int GS = decode_group(H / Hkv, n_kv);
        const int nsplit = decode_splits(D, GS, n_kv, p.nsplit);
        launch_attn_decode(q, q_h, k, k_h, k_j, v, v_h, v_j, D, H, Hkv, n_kv, nullptr, scale, nsplit,
                           (n_kv + nsplit - 1) / nsplit, n_kv, GS, out, po, pml, s, nullptr, mask);
        if (nsplit == 1) return;
        if (D == 64) k_attn_merge<64><<<(unsigned) H, 64, 0, s>>>(po, pml, out, nsplit);
        else k_attn_merge<128><<<(unsigned) H, 128, 0, s>>>(po, pml, out, nsplit);
        check_launch("flash_attn merge");
        return;
    }
    launch_attn_split(q, q_h, q_s, k, k_h, k_j, v, v_h, v_j, mask, m_s, D, Sq, H, Hkv, n_kv, scale, po, pml, p,
                      nullptr, s);
    if (D == 64) k_attn_merge<64><<<(unsigned) (Sq * H), 64, 0, s>>>(po, pml, out, p.nsplit);
    else if (D == 128) k_attn_merge<128><<<(unsigned) (Sq * H), 128, 0, s>>>(po, pml, out, p.nsplit);
    else k_attn_merge<256><<<(unsigned) (Sq * H), 256, 0, s>>>(po, pml, out, p.nsplit);
    check_launch("flash_attn merge");
}

}  // namespace gcq
