// attn_oproj.hip - one decode layer's attention and output projection in a single launch:
// ggml_flash_attn_ext over the f16 KV cache (runtime/src/ops.cpp:217-243) for one query row, then
// ggml_mul_mat by the packed Q4_0 / Q8_0 output weight and the residual ggml_add
// (ggml_compiler/llm.py:361-444, the attention half of a decoder layer).
//
// As two launches (the lane-group attention, then the row GEMV with its split-merge prologue) the
// output projection pays a launch boundary and the ramp before its first weight bytes arrive,
// while its weights do not depend on the attention at all. Here one workgroup per CU (all
// resident) runs:
//   1. its attention task, if it has one: split s of the keys for query head h (the lane-group
//      code of attn_lanes.h, one query head per workgroup; the G query heads of a KV head and a
//      split sit on workgroups of one XCD, b % 8 equal, so the shared K / V rows come from that
//      XCD's L2 after the first read). Once its K / V loads are issued, every wavefront issues
//      the loads of its output-projection row (or, without a task, at once), so the weights are
//      in registers long before they are used. The split's partial (max, exp-sum, unnormalized
//      output) is stored device-coherently;
//   2. a grid barrier (grid_sync.h: bounded waits, an error word the host checks);
//   3. every workgroup merges the partials of all heads (k_merge_q8's arithmetic, as the row
//      GEMV's merge prologue) into the attention row's Q8_0 codes in LDS, then each wavefront
//      finishes its row: block dots in the row GEMV's per-lane order, a wavefront sum, + the
//      residual.
// Every value is computed with the same operations in the same order as the two-launch path
// (k_attn_lanes, then k_row_gemv<.., PRO_MERGE, EPI_STORE>), so both give the same row bit for
// bit.
#include "attn_lanes.h"
#include "gcq_common.h"
#include "grid_sync.h"

#include <algorithm>

namespace gcq {

int cu_count();

namespace {

constexpr int kNW = 16;         // wavefronts per workgroup
constexpr int kOMaxK = 4096;    // attention row (H D) the merge prologue takes: 4 values per thread
constexpr int kOMaxSplit = 8;   // splits the merge holds in registers
constexpr uint32_t kPast = 0x80000000u;  // a buffer offset past every buffer: reads zeros

// The attention task of workgroup b: (split, KV head hk, query head h). With xcd, the G query
// heads of one (split, KV head) unit u go to workgroups b = 8 (G (u / 8) + g) + u % 8, which share
// b % 8 and so (workgroups are dispatched to the 8 XCDs in turn) one XCD's L2; else task b is
// (split b / H, head b % H).
__device__ __forceinline__ bool attn_task_of(int b, const AttnOArgs & a, int & split, int & hk, int & h) {
    const int G = a.H / a.Hkv;
    if (a.xcd) {
        const int r = b & 7, qq = b >> 3, g = qq % G, u = (qq / G) * 8 + r;
        if (u >= a.nsplit * a.Hkv) return false;
        split = u / a.Hkv;
        hk = u % a.Hkv;
        h = hk * G + g;
        return true;
    }
    if (b >= a.nsplit * a.H) return false;
    split = b / a.H;
    h = b % a.H;
    hk = h / G;
    return true;
}

template <int TYPE, int D, int NBL>
__global__ __launch_bounds__(kNW * 64) void k_attn_oproj(const AttnOArgs a) {
    constexpr int CV = TYPE == T_Q4_0 ? 1 : 2;  // 16-byte loads per block
    __shared__ float so[kNW][D];
    __shared__ float2 sml[kNW][1];
    __shared__ int4 lc[kOMaxK / 16];
    __shared__ float2 lm[kOMaxK / 32];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = a.nb, K = nb * QK;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.wqs), 0, (int) ((size_t) a.N * nb * CV * 16), 0x00020000);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(a.wd), 0, (int) (((size_t) a.N * nb + 1) / 2 * 4), 0x00020000);

    // Output-projection rows of this wavefront: row0, row0 + stride, ... (one for the decoder's
    // shapes); the first row's weights and residual are loaded with the attention's loads.
    const int stride = gridDim.x * kNW;
    const int row0 = blockIdx.x * kNW + wave;
    uint4 w[NBL][CV];
    uint32_t dw[NBL];
    float res = 0.0f;
    auto load_row = [&](int r) {
        const bool live = r < a.N;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = lane + 64 * i;  // lanes past the row read zeros, unused
            const bool in = live && blk < nb;
            const uint32_t o = (uint32_t) r * (uint32_t) nb + (uint32_t) blk;
#pragma unroll
            for (int c = 0; c < CV; c++) {
                const auto t = __builtin_amdgcn_raw_buffer_load_b128(rq, in ? (o * CV + c) * 16u : kPast, 0, 2);
                w[i][c] = make_uint4(t[0], t[1], t[2], t[3]);
            }
            dw[i] = __builtin_amdgcn_raw_buffer_load_b32(rd, in ? (o >> 1) * 4u : kPast, 0, 0);
        }
        res = lane == 0 && live ? a.x[r] : 0.0f;
    };
    auto issue = [&] { load_row(row0); };

    int split = 0, hk = 0, h = 0;
    if (attn_task_of(blockIdx.x, a, split, hk, h)) {
        const int n_kv = *a.n_kv_dev;
        attn_lanes_task<D, 1, kNW, false, true>(a.q, D, a.kc, a.kv_h, D, a.vc, a.kv_h, D, a.scale, n_kv, a.chunk,
                                                 a.kv_rows, a.nsplit, nullptr, a.part_o, a.part_ml, nullptr, split,
                                                 hk, h, so, sml, issue);
    } else {
        issue();
    }
    bar_arrive(a.bar, 1u);
    bar_wait(a.bar, a.err, 1u);

    // The merged attention row (k_merge_q8's arithmetic: sum_i e^(m_i - M) o_i / sum_i e^(m_i - M)
    // l_i in split order, splits with m_i = -inf left out, 0 if none) as Q8_0 codes in LDS.
    {
        float2 mlv[kOMaxSplit];
        float4 pov[kOMaxSplit];
        const int e0 = min((int) threadIdx.x * 4, K - 4);
        const int hh = e0 / D;
        const float2 * ml = a.part_ml + (int64_t) hh * a.nsplit;
        const float * po = a.part_o + (int64_t) hh * a.nsplit * D + e0 % D;
#pragma unroll
        for (int j = 0; j < kOMaxSplit; j++) {
            if (j < a.nsplit) {
                mlv[j] = ml[j];
                pov[j] = *reinterpret_cast<const float4 *>(po + (int64_t) j * D);
            } else {
                mlv[j] = make_float2(-INFINITY, 0.0f);
            }
        }
        const int e = threadIdx.x * 4;
        if (e < K) {
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < kOMaxSplit; j++) M = fmaxf(M, mlv[j].x);
            float L = 0.0f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            if (M != -INFINITY) {
#pragma unroll
                for (int j = 0; j < kOMaxSplit; j++) {
                    if (mlv[j].x == -INFINITY) continue;
                    const float wj = __expf(mlv[j].x - M);
                    L += wj * mlv[j].y;
                    o.x += wj * pov[j].x;
                    o.y += wj * pov[j].y;
                    o.z += wj * pov[j].z;
                    o.w += wj * pov[j].w;
                }
            }
            o.x = L == 0.0f ? 0.0f : o.x / L;
            o.y = L == 0.0f ? 0.0f : o.y / L;
            o.z = L == 0.0f ? 0.0f : o.z / L;
            o.w = L == 0.0f ? 0.0f : o.w / L;
            q8_block_store(o, reinterpret_cast<int8_t *>(lc) + (e & ~31), lm + e / 32, (e / 4) & 7);
        }
    }
    __syncthreads();

    // The wavefront's rows: block dots against the codes, the row sum, + the residual.
    for (int r = row0; r < a.N; r += stride) {
        if (r != row0) load_row(r);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = lane + 64 * i;
            if (blk >= nb) break;
            const int4 ca = lc[2 * blk], cb = lc[2 * blk + 1];
            const float2 cm = lm[blk];
            int sdot;
            if constexpr (TYPE == T_Q4_0) sdot = dot_blk_q4_0(w[i][0], ca, cb, __float_as_int(cm.y));
            else sdot = dot_blk_q8_0(w[i][0], w[i][CV - 1], ca, cb);
            // scale index r * nb + blk: its parity picks the half (blk's parity is the lane's)
            const uint32_t sh = (uint32_t) (((lane ^ (r & nb)) & 1) << 4);
            acc += ((float) sdot * h2f((uint16_t) (dw[i] >> sh))) * cm.x;
        }
        const float v = wave_sum(acc);
        if (lane == 0) a.x[r] = v + res;
    }
    bar_leave(a.bar);
}

}  // namespace

size_t attn_oproj_bar_bytes() { return kBarWords * sizeof(unsigned); }

// Whether the fused launch runs this configuration: Q4_0 / Q8_0 output weight, head_dim 64 / 128,
// the attention row H D (the weight's K) a multiple of 32 and at most 4096, a lane-group split
// plan of at most 8 splits whose tasks (nsplit H) fit one workgroup per CU.
bool attn_oproj_fits(int type, int H, int Hkv, int D, int nsplit) {
    return (type == T_Q4_0 || type == T_Q8_0) && (D == 64 || D == 128) && Hkv >= 1 && H % Hkv == 0 &&
           H * D <= kOMaxK && (H * D) % QK == 0 && nsplit >= 1 && nsplit <= kOMaxSplit &&
           nsplit * H <= cu_count();
}

void launch_attn_oproj(int type, int D, const AttnOArgs & a0, hipStream_t s) {
    require(attn_oproj_fits(type, a0.H, a0.Hkv, D, a0.nsplit), "attn + output projection: configuration not supported");
    require(a0.nb * QK == a0.H * D, "attn + output projection: the weight's K must be the attention row (H D)");
    require((int64_t) a0.nsplit * a0.chunk >= a0.kv_rows, "attn + output projection: the splits must cover the cache");
    require(a0.N >= 1 && (uint64_t) a0.N * a0.nb * (type == T_Q4_0 ? 16u : 32u) < 0x80000000ull,
            "attn + output projection: weight of 2 GB or more");
    require(((uintptr_t) a0.q & 15) == 0 && ((uintptr_t) a0.kc & 15) == 0 && ((uintptr_t) a0.vc & 15) == 0 &&
                a0.kv_h % 8 == 0,
            "attn + output projection: 16-byte aligned q and K / V rows");
    require(a0.bar && a0.err && a0.n_kv_dev, "attn + output projection: barrier words, error word and KV length");
    AttnOArgs a = a0;
    const unsigned grid = (unsigned) cu_count();
    const int U = a.nsplit * a.Hkv, G = a.H / a.Hkv;
    a.xcd = 8 * G * ((U + 7) / 8) <= (int) grid ? 1 : 0;
    const int nbl = (a.nb + 63) / 64;
#define GCQ_AO(T, DD, NB)                                                                                        \
    if (type == T && D == DD && nbl == NB) {                                                                     \
        int occ = 0;                                                                                             \
        check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(                                                  \
                      &occ, reinterpret_cast<const void *>(&k_attn_oproj<T, DD, NB>), kNW * 64, 0),              \
                  "attn + output projection occupancy");                                                        \
        require(occ >= 1, "attn + output projection: a workgroup does not fit a CU");                            \
        k_attn_oproj<T, DD, NB><<<grid, kNW * 64, 0, s>>>(a);                                                    \
        check_launch("attn + output projection");                                                               \
        return;                                                                                                  \
    }
    GCQ_AO(T_Q4_0, 128, 1) GCQ_AO(T_Q4_0, 128, 2) GCQ_AO(T_Q4_0, 64, 1) GCQ_AO(T_Q4_0, 64, 2)
    GCQ_AO(T_Q8_0, 128, 1) GCQ_AO(T_Q8_0, 128, 2) GCQ_AO(T_Q8_0, 64, 1) GCQ_AO(T_Q8_0, 64, 2)
#undef GCQ_AO
    fail("attn + output projection: configuration not supported");
}

}  // namespace gcq
