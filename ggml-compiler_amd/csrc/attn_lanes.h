// attn_lanes.h - the lane-group decode attention (one query row over an f16 KV cache), as a
// device function of attn.hip's k_attn_lanes.
//
// Short contexts (up to kLanesMaxKv keys) are latency-bound, so parallel work beats arithmetic
// efficiency: one query row, one workgroup per (split, KV head, query-head group), NW wavefronts.
// Each wavefront takes a contiguous run of the split's keys; its lanes work in groups of D/8
// (8 dims, 16 B of a K or V row each) and every lane group keeps its own online softmax per query
// head (running max m, exp-sum l, P.V accumulator) over load batches of NB keys, K and V rows of a
// batch loaded together, so no reduction crosses lane groups inside the loop. The lane groups and
// then the NW wavefronts are merged at the end (shuffles, LDS). One split with an output row: the
// normalized output out[h][d]; else the split's (max, exp-sum, unnormalized output) in
// k_attn_split's partial layout, for the merge (k_attn_merge, or a GEMV prologue). The host sizes
// splits and NW so that each wavefront's keys are about one load batch (lanes_nw).
#pragma once

#include "gcq_common.h"

namespace gcq {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t u) {
    half2_t h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

// Steps per load batch: 4, or 2 for four query heads per workgroup (with four heads'
// accumulators per lane the two-step batch measured about 11% faster at 32768 keys and the same at
// 4096 and below); keys one wavefront loads per batch; the legacy workgroup size (16 wavefronts, 8
// for four query heads) and the keys such a workgroup loads in one batch.
__host__ __device__ constexpr int lanes_nb(int G) { return G >= 4 ? 2 : 4; }
__host__ __device__ constexpr int lanes_batch(int D, int G) { return (64 / (D / 8)) * lanes_nb(G); }
__host__ __device__ constexpr int lanes_waves(int G) { return G >= 4 ? 8 : 16; }
__host__ __device__ constexpr int lanes_keys(int D, int G) { return lanes_waves(G) * lanes_batch(D, G); }

// Wavefronts per workgroup for a split of `chunk` keys: about one load batch each, 4, 8 or 16.
// Measured on MI355X (32 query heads on 8 KV heads of 128, one query row): a workgroup's
// wavefronts wait at the merge for the slowest of them, and 16 per workgroup left each of them a
// few keys, so 4-8 wavefronts and more splits end 1.5-2.4 us sooner at 512-1024 keys.
__host__ __device__ constexpr int lanes_nw(int D, int G, int chunk) {
    return (chunk + lanes_batch(D, G) - 1) / lanes_batch(D, G) <= 4   ? 4
           : (chunk + lanes_batch(D, G) - 1) / lanes_batch(D, G) <= 8 ? 8
                                                                       : 16;
}

// f16 value c (0..7) of 8 packed in a uint4, as f32.
__device__ __forceinline__ float half_at(const uint4 & r, int c) {
    const uint32_t w = c < 2 ? r.x : c < 4 ? r.y : c < 6 ? r.z : r.w;
    return h2f((uint16_t) (c & 1 ? w >> 16 : w & 0xffff));
}

// One workgroup's task: split `split` of KV head hk for query heads h0 .. h0 + G - 1. Every
// thread of the workgroup calls it (it ends with a workgroup barrier). so / sml: the workgroup's
// LDS for the wavefront merge. issue(): called by every thread once the first batch of K / V
// loads is issued, before any of them is waited for (the fused launch issues its weight loads
// there). MASK: an f16 mask row (n_kv values, ggml's [n_kv, 1] mask of one query row) is added to
// the scaled scores, -inf dropping a key. CO: the partials are stored device-coherently (read by
// other workgroups later in the same launch). out == nullptr: partials even for one split.
template <int D, int G, int NW, bool MASK, bool CO, class Issue>
__device__ __forceinline__ void attn_lanes_task(const float * __restrict__ q, int64_t q_h,
                                                const uint16_t * __restrict__ k, int64_t k_h, int64_t k_j,
                                                const uint16_t * __restrict__ v, int64_t v_h, int64_t v_j,
                                                float scale, int n_kv, int chunk, int kv_rows, int nsplit,
                                                float * __restrict__ out, float * __restrict__ part_o,
                                                float2 * __restrict__ part_ml, const uint16_t * __restrict__ mask,
                                                int split, int hk, int h0, float (&so)[NW][G * D],
                                                float2 (&sml)[NW][G], Issue && issue) {
    constexpr int LPK = D / 8;     // lanes per key row
    constexpr int KPW = 64 / LPK;  // lane groups (keys per step) per wavefront
    constexpr int NB = lanes_nb(G);  // steps per load batch
    static_assert(G * D <= NW * 64, "one output per thread in the merge");

    // Split and wavefront ranges come from the host's chunk, so the K/V addresses do not wait for
    // the KV length read from device state; rows are clamped into the kv_rows that exist and keys
    // at or past n_kv are masked.
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
    issue();
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
        if (nsplit == 1 && out) {
            out[h * D + d] = L == 0.0f ? 0.0f : o / L;
        } else if constexpr (CO) {
            st_co_f(&part_o[((int64_t) h * nsplit + split) * D + d], o);
            if (d == 0) {
                float2 * ml = &part_ml[(int64_t) h * nsplit + split];
                st_co_f(&ml->x, M);
                st_co_f(&ml->y, L);
            }
        } else {
            part_o[((int64_t) h * nsplit + split) * D + d] = o;
            if (d == 0) part_ml[(int64_t) h * nsplit + split] = make_float2(M, L);
        }
    }
}

}  // namespace gcq
