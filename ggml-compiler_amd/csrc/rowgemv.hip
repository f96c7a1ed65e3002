// rowgemv.hip - the decode step's projections: one f32 activation row times a packed Q4_0 / Q8_0
// weight, with the graph node before and after each mul_mat done in the same launch.
//
// In ggml-compiler's decoder layer (ggml_compiler/llm.py:361-444 at O3) every mul_mat sits between
// small nodes: rms_norm + mul before QKV and gate/up, flash_attn before the output projection,
// rope + set_rows after QKV, swiglu after gate/up, add after the output and down projections. For
// one token these nodes are latency, not bandwidth, so they move into the GEMV:
//
//   prologue (every workgroup, into LDS)        epilogue (per row pair)
//   PRO_PLAIN  Q8_0 of x                        EPI_STORE    y = W x (+ res)
//   PRO_NORM   Q8_0 of rms_norm(x) * w          EPI_ROPE_KV  NEOX rope of q and k (the step's
//                                                            cos/sin table), q -> f32,
//   PRO_MERGE  Q8_0 of the merged split-K                    k and v -> f16 KV cache at pos
//              attention partials (<= 8)        EPI_SWIGLU   y[j] = silu(g_j) * u_j
//   PRO_SWIGLU Q8_0 of silu(g) * u (two f32 rows)
//
// Every value is computed with the same operations, in the same order, as the separate kernels
// (rmsnorm_q8_row / k_merge_q8 / k_rope_kv / k_swiglu_q8 and the Q8_0 activation quantizer), so
// the fused step equals the unfused one bit for bit.
//
// Layout: one 1024-thread workgroup per CU (persistent). The prologue writes the row's Q8_0 codes
// and (d, code sum) to LDS once per CU; each wavefront then walks row groups g, g + waves, ...
// (R rows each) with the next group's weights loaded before the current group is reduced. Lane l
// takes blocks l, l + 64, ... of its rows, so a load moves 64 x 16 B of one row.
//
// Row pairs: EPI_ROPE_KV expects the QKV weight packed so that group g holds the rotation pair
// (i, i + D/2) of a q or k head, then consecutive v rows; EPI_SWIGLU expects gate row j and up row
// j in group j (llama.hip packs them so; with two weights, group j reads row j of each).
#include "gcq_common.h"

#include <algorithm>

namespace gcq {

constexpr int kRowMaxK = 16384;  // LDS holds the row's codes: K bytes + K/32 float2
constexpr int kMergeMax = 8;     // split-K partials the merge prologue takes (held in registers)

template <int TYPE, int R, int NBL, int PRO, int EPI, int MR>
__global__ __launch_bounds__(1024) void k_row_gemv(const RowArgs a) {
    constexpr int NT = 1024, NWV = NT / 64;
    constexpr int CV = TYPE == T_Q4_0 ? 1 : 2;
    constexpr bool XREG = NBL <= 2;  // activation blocks in registers, else read from LDS per use
    constexpr bool PF = CV * NBL * R <= 8;  // next group's weights prefetched (else: registers spill)
    static_assert(EPI == EPI_STORE || R == 2, "row-pair epilogues take two rows per group");
    __shared__ int4 lc[kRowMaxK / 16];
    __shared__ float2 lm[kRowMaxK / 32];
    __shared__ double red[NWV];

    const int lane = threadIdx.x & 63;
    const int ng = (a.N + R - 1) / R;
    const int nb = a.nb;
    const int K = nb * QK;
    // Weights through buffer loads: an offset past the buffer's end reads zeros without a memory
    // access, so the loads of groups past the last (every wavefront issues the same number of
    // loads, which lets the compiler count them) cost nothing and leave nothing in flight.
    // Codes are streamed (non-temporal); the fp16 scales arrive as the aligned 32-bit word holding
    // them (halves picked where used, so the loads' results need no conversion and no wait until
    // then; the word of the last scale stays inside the scales' 256-byte-aligned region).
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.wqs), 0, MR > 1 ? (int) a.qs_span : (int) ((size_t) a.N * nb * CV * 16), 0x00020000);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(a.wd), 0, MR > 1 ? (int) a.d_span : (int) (((size_t) a.N * nb + 1) / 2 * 4),
        0x00020000);
    // Weight k of row `row` (wave-uniform, kept in scalar registers) and the row's index in it; the
    // per-weight values are picked with constant indices (a dynamic index into the kernel
    // arguments becomes a vector memory load in front of every weight load).
    auto range_of = [&](int row, int & local) -> int {
        row = __builtin_amdgcn_readfirstlane(row);
        const bool k1 = a.nr > 1 && row >= a.r_end[0], k2 = a.nr > 2 && row >= a.r_end[1];
        local = k2 ? row - a.r_end[1] : k1 ? row - a.r_end[0] : row;
        return k2 ? 2 : k1 ? 1 : 0;
    };
    auto pick_u = [](int k, const uint32_t (&v)[3]) { return k == 2 ? v[2] : k == 1 ? v[1] : v[0]; };
    // Row r of group g with several weights: EPI_STORE takes the rows in order; EPI_ROPE_KV takes
    // separate q, k, v weights (ranges 0, 1, 2) in the packed QKV order: group g < (H + Hkv) D/2
    // is the rotation pair (i, i + D/2) of q head h (h < H) or k head h - H, then pairs of v rows;
    // EPI_SWIGLU takes separate gate and up weights (ranges 0, 1): group g is gate row g and up
    // row g, the pair the packed gate/up weight holds in group g.
    // x / (D/2) for the rope epilogue's group indices (x >= 0): the high half of x * hd_magic (a
    // division by a value known only at run time is a chain of some 30 dependent instructions,
    // and a choice between it and a shift a branch, either of which in front of a group's weight
    // loads delays them).
    const int hd = a.D >> 1;
    auto div_hd = [&](int x) -> int { return (int) __umulhi((uint32_t) x, a.hd_magic); };
    auto map_row = [&](int g, int r, int & local) -> int {
        if constexpr (EPI == EPI_SWIGLU) {
            local = min(__builtin_amdgcn_readfirstlane(g), a.r_end[0] - 1);
            return r;
        } else if constexpr (EPI == EPI_ROPE_KV) {
            // both cases computed and one selected: scalar selects, no branch
            g = __builtin_amdgcn_readfirstlane(g);
            const int nq = (a.H + a.Hkv) * hd;
            const int gq = min(g, nq - 1);
            const int h = div_hd(gq), i = gq - h * hd;
            const bool qh = h < a.H, vg = g >= nq;
            local = vg ? min(2 * (g - nq) + r, a.Hkv * a.D - 1) : (qh ? h : h - a.H) * a.D + i + r * hd;
            return vg ? 2 : qh ? 0 : 1;
        } else {
            return range_of(min(g * R + r, a.N - 1), local);
        }
    };
    constexpr uint32_t kPast = 0x80000000u;  // an offset past every buffer (sizes < 2 GB)

    uint4 w[NBL][R][CV];
    uint32_t d[NBL][R];
    auto load = [&](int g, uint4 (&wv)[NBL][R][CV], uint32_t (&dv)[NBL][R]) {
        const bool live = g < ng;
        int rows[R];
        uint32_t qbs[R], dbs[R];  // several weights: each row's index and offsets, once per group
        if constexpr (MR > 1) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                rows[r] = min(g * R + r, a.N - 1);
                const int k = map_row(g, r, rows[r]);
                qbs[r] = pick_u(k, a.r_qs);
                dbs[r] = pick_u(k, a.r_d);
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = lane + 64 * i;  // lanes past the row read zeros, unused
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = MR > 1 ? rows[r] : min(g * R + r, a.N - 1);
                const uint32_t qb = MR > 1 ? qbs[r] : 0u, db = MR > 1 ? dbs[r] : 0u;
                const uint32_t o = (uint32_t) row * (uint32_t) nb + (uint32_t) blk;
                const bool in = live && blk < nb;
#pragma unroll
                for (int c = 0; c < CV; c++) {
                    const uint32_t off = in ? qb + (o * CV + c) * 16u : kPast;
                    const auto t = __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 2);  // 2: nt
                    wv[i][r][c] = make_uint4(t[0], t[1], t[2], t[3]);
                }
                dv[i][r] = __builtin_amdgcn_raw_buffer_load_b32(rd, in ? db + (o >> 1) * 4u : kPast, 0, 0);
            }
        }
    };

    // Wavefronts. PLAIN / NORM: the first XW ("x waves") only turn the activation row into Q8_0
    // codes in LDS; the other CW = 16 - XW walk the row groups. A CU's vector memory requests
    // queue in issue order and a wavefront's loads complete in order, so the x waves issue their
    // loads first and the workgroup meets before any weight load is issued: the activation row
    // is not queued behind the CU's weight stream, and the compute waves start that stream at
    // once. The compute waves take the codes through an LDS counter, not a workgroup barrier
    // (which would also wait for wavefronts stalled on issuing loads into a full memory queue).
    // MERGE: every wavefront merges 4 values (K <= 4096) and then walks row groups; its weights
    // are issued before the prologue. With few groups per wavefront (long rows, or groups that
    // all 16 wavefronts of every CU take in one round) the x waves take row groups too, the last
    // ones of the workgroup, loaded once their prologue is done (a.xc, chosen by the dispatch).
    //
    // x thread t (of 64 XW) takes half blocks t, t + 64 XW, ... (16 values each), so the
    // prologue's arithmetic sits on a few wavefronts. Weight loads are unconditional (addresses
    // clamped into range, values past the end discarded), so the compiler knows how many are in
    // flight and waits for the oldest only.
    constexpr bool MERGE = PRO == PRO_MERGE;
    constexpr bool TWO = PRO == PRO_NORM || PRO == PRO_SWIGLU;  // the x waves read two rows
    constexpr int XWMAX = (TWO && NBL > 4) ? 8 : 4;  // x waves at most
    constexpr int RMAX = MERGE ? 1 : (2 * NBL + XWMAX - 1) / XWMAX;  // half blocks per x thread at most
    const int wave = threadIdx.x >> 6;
    const int XW = MERGE ? NWV : min(XWMAX, (K + 1023) / 1024);
    const int rounds = MERGE ? 1 : (K + XW * 1024 - 1) / (XW * 1024);
    const bool XC = !MERGE && a.xc != 0;  // x waves compute too
    const int CW = (MERGE || XC) ? NWV : NWV - XW;  // compute waves (host: run_row_r's cw)
    const bool xw = !MERGE && wave < XW;  // an x wave of PLAIN / NORM
    int g = blockIdx.x * CW + (MERGE ? wave : XC ? (wave + NWV - XW) % NWV : max(wave - XW, 0));
    const int nw = gridDim.x * CW;

    __shared__ unsigned int s_flag[2];  // x waves done with: [0] their norm partial, [1] their codes
    if (threadIdx.x == 0) {
        s_flag[0] = 0u;
        s_flag[1] = 0u;
    }
    const int p_tok = EPI == EPI_ROPE_KV ? *a.pos : 0;
    const int half = a.D / 2;
    const int nqk = (a.H + a.Hkv) * half;  // row-pair groups of q and k (rotated)
    float2 cs_first = make_float2(0.0f, 0.0f);  // the rotation of this wave's first group
    uint4 wn[NBL][R][CV];
    uint32_t dn[NBL][R];

    if constexpr (!MERGE) {
        // The x waves' path ends in this block (their loads never meet the compute waves' code,
        // whose waits would otherwise count them).
        if (xw) {
            float4 xv[RMAX][4], nv[TWO ? RMAX : 1][4];
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r < rounds) {
                    const int e = min(((int) threadIdx.x + r * XW * 64) * 16, K - 16);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        xv[r][c] = *reinterpret_cast<const float4 *>(a.x + e + 4 * c);
                        if constexpr (PRO == PRO_NORM)
                            nv[r][c] = *reinterpret_cast<const float4 *>(a.norm_w + e + 4 * c);
                        if constexpr (PRO == PRO_SWIGLU)
                            nv[r][c] = *reinterpret_cast<const float4 *>(a.up + e + 4 * c);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();  // the x waves' loads are issued before any weight load
            __builtin_amdgcn_sched_barrier(0);
            const int t = threadIdx.x;
            float v[RMAX][16];
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                const bool act = r < rounds && (t + r * XW * 64) * 16 < K;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    v[r][4 * c] = act ? xv[r][c].x : 0.0f;
                    v[r][4 * c + 1] = act ? xv[r][c].y : 0.0f;
                    v[r][4 * c + 2] = act ? xv[r][c].z : 0.0f;
                    v[r][4 * c + 3] = act ? xv[r][c].w : 0.0f;
                }
            }
            if constexpr (PRO == PRO_NORM) {
                // ggml_rms_norm: squares rounded to f32, summed in double, the mean rounded to f32
                double ss = 0.0;
#pragma unroll
                for (int r = 0; r < RMAX; r++)
#pragma unroll
                    for (int j = 0; j < 16; j++) ss += (double) (v[r][j] * v[r][j]);
                ss = wave_sum_d(ss);
                if (lane == 0) {
                    red[wave] = ss;
                    lds_signal(&s_flag[0]);
                }
                lds_wait(&s_flag[0], XW);
                double tot = 0.0;
#pragma unroll
                for (int i = 0; i < XWMAX; i++)
                    if (i < XW) tot += red[i];
                const float scale = 1.0f / sqrtf((float) (tot / (double) K) + a.eps);
#pragma unroll
                for (int r = 0; r < RMAX; r++)
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        v[r][4 * c] = (v[r][4 * c] * scale) * nv[r][c].x;
                        v[r][4 * c + 1] = (v[r][4 * c + 1] * scale) * nv[r][c].y;
                        v[r][4 * c + 2] = (v[r][4 * c + 2] * scale) * nv[r][c].z;
                        v[r][4 * c + 3] = (v[r][4 * c + 3] * scale) * nv[r][c].w;
                    }
            }
            if constexpr (PRO == PRO_SWIGLU) {
                // k_swiglu_q8's arithmetic: g / (1 + e^-g) * u
#pragma unroll
                for (int r = 0; r < RMAX; r++)
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        v[r][4 * c] = v[r][4 * c] / (1.0f + expf(-v[r][4 * c])) * nv[r][c].x;
                        v[r][4 * c + 1] = v[r][4 * c + 1] / (1.0f + expf(-v[r][4 * c + 1])) * nv[r][c].y;
                        v[r][4 * c + 2] = v[r][4 * c + 2] / (1.0f + expf(-v[r][4 * c + 2])) * nv[r][c].z;
                        v[r][4 * c + 3] = v[r][4 * c + 3] / (1.0f + expf(-v[r][4 * c + 3])) * nv[r][c].w;
                    }
            }
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                const int hb = t + r * XW * 64;  // half block; its pair is in the neighbouring lane
                if (r < rounds && hb * 16 < K)
                    q8_half_block_store(v[r], reinterpret_cast<int8_t *>(lc) + (hb / 2) * 32, lm + hb / 2, hb & 1);
            }
            if (lane == 0) lds_signal(&s_flag[1]);
            if (!XC) return;
        } else {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (EPI == EPI_ROPE_KV) {
            const int gq = min(g, nqk - 1);
            cs_first = a.rope_cs[gq - div_hd(gq) * half];
        }
        load(g, w, d);
    } else {
        float2 mlv[kMergeMax];
        float4 pov[kMergeMax];
        const int e0 = min((int) threadIdx.x * 4, K - 4);
        const int h = e0 / a.D;
        const float2 * ml = a.part_ml + (int64_t) h * a.nsplit;
        const float * po = a.part_o + (int64_t) h * a.nsplit * a.D + e0 % a.D;
#pragma unroll
        for (int j = 0; j < kMergeMax; j++) {
            if (j < a.nsplit) {
                mlv[j] = ml[j];
                pov[j] = *reinterpret_cast<const float4 *>(po + (int64_t) j * a.D);
            } else {
                mlv[j] = make_float2(-INFINITY, 0.0f);  // splits past the last: none
            }
        }
        if constexpr (EPI == EPI_ROPE_KV) {
            const int gq = min(g, nqk - 1);
            cs_first = a.rope_cs[gq - div_hd(gq) * half];
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();  // the partials' loads are issued before any weight load
        __builtin_amdgcn_sched_barrier(0);
        load(g, w, d);
        // The merged attention output (k_merge_q8's arithmetic): sum_i e^(m_i - M) o_i /
        // sum_i e^(m_i - M) l_i in split order, splits with m_i = -inf left out, 0 if none.
        const int e = threadIdx.x * 4;
        if (e < K) {
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < kMergeMax; j++) M = fmaxf(M, mlv[j].x);
            float L = 0.0f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            if (M != -INFINITY) {
#pragma unroll
                for (int j = 0; j < kMergeMax; j++) {
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
        if (lane == 0) lds_signal(&s_flag[1]);
    }
    lds_wait(&s_flag[1], XW);
    if constexpr (PF) load(g + nw, wn, dn);

    int4 xa[XREG ? NBL : 1], xb[XREG ? NBL : 1];
    float2 xm[XREG ? NBL : 1];
    if constexpr (XREG) {
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = lane + 64 * i;
            if (blk < nb) {
                xa[i] = lc[2 * blk];
                xb[i] = lc[2 * blk + 1];
                xm[i] = lm[blk];
            }
        }
    }
    const int g_first = g;

    // One row group: block dots, the row sums, the epilogue.
    auto group = [&](int gg, const uint4 (&wv)[NBL][R][CV], const uint32_t (&dv)[NBL][R]) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        int prow[R];  // several weights: each row's index within its weight, once per group
        if constexpr (MR > 1) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                prow[r] = min(gg * R + r, a.N - 1);
                (void) map_row(gg, r, prow[r]);
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int blk = lane + 64 * i;
            if (blk >= nb) break;
            int4 ca, cb;
            float2 cm;
            if constexpr (XREG) {
                ca = xa[i];
                cb = xb[i];
                cm = xm[i];
            } else {
                ca = lc[2 * blk];
                cb = lc[2 * blk + 1];
                cm = lm[blk];
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                int sdot;
                if constexpr (TYPE == T_Q4_0) sdot = dot_blk_q4_0(wv[i][r][0], ca, cb, __float_as_int(cm.y));
                else sdot = dot_blk_q8_0(wv[i][r][0], wv[i][r][CV - 1], ca, cb);
                // scale index row * nb + blk: its parity picks the half (blk's parity is the lane's)
                const int row = MR > 1 ? prow[r] : min(gg * R + r, a.N - 1);
                const uint32_t sh = (uint32_t) (((lane ^ (row & nb)) & 1) << 4);
                acc[r] += ((float) sdot * h2f((uint16_t) (dv[i][r] >> sh))) * cm.x;
            }
        }
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = wave_sum(acc[r]);
        if constexpr (EPI == EPI_STORE && MR > 1) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                int row = gg * R + r;
                if (lane == r && row < a.N) {
                    const int k = range_of(row, row);
                    float * y = k == 2 ? a.r_y[2] : k == 1 ? a.r_y[1] : a.r_y[0];
                    y[row] = v[r];
                }
            }
        } else if constexpr (EPI == EPI_STORE) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = gg * R + r;
                if (lane == r && row < a.N) a.y[row] = a.res ? v[r] + a.res[row] : v[r];
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            if (lane == 0) a.y[gg] = v[0] / (1.0f + expf(-v[0])) * v[1];
        } else {  // EPI_ROPE_KV
            if (lane == 0 && p_tok >= 0 && p_tok < a.ctx) {
                if (gg < nqk) {
                    const int h = div_hd(gg), i = gg - h * half;
                    const float2 cs = gg == g_first ? cs_first : a.rope_cs[i];
                    const float2 yr = rope_pair(v[0], v[1], cs);
                    const float y0 = yr.x, y1 = yr.y;
                    if (h < a.H) {
                        a.y[h * a.D + i] = y0;
                        a.y[h * a.D + i + half] = y1;
                    } else {
                        uint16_t * kr = a.kc + ((int64_t) (h - a.H) * a.ctx + p_tok) * a.D;
                        kr[i] = f2h(y0);
                        kr[i + half] = f2h(y1);
                    }
                } else {
                    const int e = 2 * (gg - nqk);  // v value index over [Hkv][D]
                    const int hv = div_hd(e) >> 1, dd = e - hv * a.D;
                    const uint32_t pair = f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
                    *reinterpret_cast<uint32_t *>(a.vc + ((int64_t) hv * a.ctx + p_tok) * a.D + dd) = pair;
                }
            }
        }
    };

    if constexpr (PF) {
        // Two buffers in turn (w: groups g, g + 2 waves, ...; wn: the ones between), so a group's
        // weights are loaded two groups ahead and never copied between registers.
        while (g < ng) {
            group(g, w, d);
            load(g + 2 * nw, w, d);
            g += nw;
            if (g >= ng) break;
            group(g, wn, dn);
            load(g + 2 * nw, wn, dn);
            g += nw;
        }
    } else {
        while (g < ng) {
            group(g, w, d);
            g += nw;
            if (g < ng) load(g, w, d);
        }
    }
}

// ------------------------------------------------------------------------------ dispatch

int cu_count();

namespace {

template <int TYPE, int R, int NBL, int PRO, int EPI>
void go(const RowArgs & a, unsigned grid, hipStream_t s) {
    if constexpr ((EPI == EPI_STORE || ((EPI == EPI_ROPE_KV || EPI == EPI_SWIGLU) && R == 2)) && PRO == PRO_NORM) {
        if (a.nr > 1) {
            k_row_gemv<TYPE, R, NBL, PRO, EPI, 3><<<grid, 1024, 0, s>>>(a);
            return;
        }
    }
    k_row_gemv<TYPE, R, NBL, PRO, EPI, 1><<<grid, 1024, 0, s>>>(a);
}

// Two rows per group when there are enough groups to give every compute wavefront of the grid
// one and their weights fit the registers (K <= 4096), else one row per group; the row-pair
// epilogues always take two. Long rows (K > 4096): lanes hold up to 8 blocks of a row.
// x waves of a workgroup (the kernel's XW): none for MERGE, else up to 4 (8 for long NORM rows).
int row_gemv_x_waves(int pro, int nb) {
    if (pro == PRO_MERGE) return 0;
    const int nbl = (nb + 63) / 64, K = nb * QK;
    const int xwmax = ((pro == PRO_NORM || pro == PRO_SWIGLU) && nbl > 4) ? 8 : 4;
    return std::min(xwmax, (K + 1023) / 1024);
}

template <int TYPE, int PRO, int EPI>
void run_row_r(const RowArgs & a0, hipStream_t s) {
    RowArgs a = a0;
    const int nbl = (a.nb + 63) / 64;
    const int cus = cu_count();
    const int xw = row_gemv_x_waves(PRO, a.nb);
    const int R = EPI != EPI_STORE || (nbl <= 2 && a.N / 2 >= cus * (16 - xw)) ? 2 : 1;
    const int ng = (a.N + R - 1) / R;
    // The x waves compute too for long rows and when all 16 wavefronts of every CU take the
    // groups in one round but the compute waves alone would need two.
    a.xc = PRO != PRO_MERGE && (nbl > 4 || (ng <= 16 * cus && ng > (16 - xw) * cus));
    if constexpr (EPI == EPI_ROPE_KV) {
        const uint64_t hd = (uint64_t) (a.D / 2);
        require(hd > 0 && (uint64_t) a.N * hd < (1ull << 32), "row gemv: rope epilogue indices past 2^32 / (D/2)");
        a.hd_magic = (uint32_t) ((1ull << 32) / hd + 1);
    }
    const int cw = (PRO == PRO_MERGE || a.xc) ? 16 : 16 - xw;  // the kernel's CW
    const int waves = cus * cw;
    // As many workgroups as give every compute wavefront the same whole number of groups (no
    // wavefront left with one more at the end), at most one per CU.
    const int per_wave = (ng + waves - 1) / waves;
    const unsigned grid = (unsigned) std::max(1, (ng + cw * per_wave - 1) / (cw * per_wave));
    if (R == 2) {
        if (nbl == 1) return go<TYPE, 2, 1, PRO, EPI>(a, grid, s);
        if (nbl == 2) return go<TYPE, 2, 2, PRO, EPI>(a, grid, s);
    } else if constexpr (EPI == EPI_STORE && PRO == PRO_MERGE) {
        if (nbl == 1) return go<TYPE, 1, 1, PRO, EPI>(a, grid, s);
        if (nbl == 2) return go<TYPE, 1, 2, PRO, EPI>(a, grid, s);
    } else if constexpr (EPI == EPI_STORE) {
        switch (nbl) {
            case 1: return go<TYPE, 1, 1, PRO, EPI>(a, grid, s);
            case 2: return go<TYPE, 1, 2, PRO, EPI>(a, grid, s);
            case 3: return go<TYPE, 1, 3, PRO, EPI>(a, grid, s);
            case 4: return go<TYPE, 1, 4, PRO, EPI>(a, grid, s);
            case 5: return go<TYPE, 1, 5, PRO, EPI>(a, grid, s);
            case 6: return go<TYPE, 1, 6, PRO, EPI>(a, grid, s);
            case 7: return go<TYPE, 1, 7, PRO, EPI>(a, grid, s);
            case 8: return go<TYPE, 1, 8, PRO, EPI>(a, grid, s);
            default: break;
        }
    }
    fail("row gemv: K = " + std::to_string(a.nb * QK) + " not supported by this epilogue");
}

template <int TYPE>
void run_row_t(int pro, int epi, const RowArgs & a, hipStream_t s) {
#define GCQ_PE(P, E)                                  \
    if (pro == P && epi == E) return run_row_r<TYPE, P, E>(a, s);
    GCQ_PE(PRO_PLAIN, EPI_STORE) GCQ_PE(PRO_NORM, EPI_STORE) GCQ_PE(PRO_MERGE, EPI_STORE)
    GCQ_PE(PRO_NORM, EPI_ROPE_KV) GCQ_PE(PRO_NORM, EPI_SWIGLU) GCQ_PE(PRO_SWIGLU, EPI_STORE)
#undef GCQ_PE
    fail("row gemv: unsupported prologue / epilogue pair");
}

}  // namespace

bool row_gemv_fits(int type, int64_t K) {
    return (type == T_Q4_0 || type == T_Q8_0) && K % QK == 0 && K > 0 && K <= kRowMaxK;
}

// The weight's codes must stay below 2 GB (32-bit buffer offsets).
static bool row_gemv_rows_fit(int type, int64_t N, int nb) {
    return N > 0 && (uint64_t) N * (uint64_t) nb * (type == T_Q4_0 ? 16u : 32u) < 0x80000000ull;
}

int row_gemv_merge_max() { return kMergeMax; }

bool row_gemv_ranges(int type, int n, const uint8_t * const * w, const int64_t * N, int64_t K, RowArgs & a) {
    if (n < 1 || n > 3 || !row_gemv_fits(type, K)) return false;
    const uint8_t *qs[3], *d[3];
    uintptr_t qlo = UINTPTR_MAX, dlo = UINTPTR_MAX;
    int64_t total = 0;
    for (int k = 0; k < n; k++) {
        const WeightLayout L = weight_layout(type, N[k], K);
        qs[k] = w[k] + L.qs;
        d[k] = w[k] + L.d;
        qlo = std::min(qlo, (uintptr_t) qs[k]);
        dlo = std::min(dlo, (uintptr_t) d[k]);
        total += N[k];
    }
    const uint64_t cb = type == T_Q4_0 ? 16u : 32u, nb = (uint64_t) (K / QK);
    uint64_t qspan = 0, dspan = 0;
    for (int k = 0; k < n; k++) {
        a.r_qs[k] = (uint32_t) ((uintptr_t) qs[k] - qlo);
        a.r_d[k] = (uint32_t) ((uintptr_t) d[k] - dlo);
        qspan = std::max(qspan, (uint64_t) ((uintptr_t) qs[k] - qlo) + (uint64_t) N[k] * nb * cb);
        dspan = std::max(dspan, (uint64_t) ((uintptr_t) d[k] - dlo) + ((uint64_t) N[k] * nb + 1) / 2 * 4);
        a.r_end[k] = (int) ((k ? a.r_end[k - 1] : 0) + N[k]);
    }
    if (qspan >= 0x80000000ull || dspan >= 0x80000000ull || total > INT32_MAX) return false;
    a.nr = n;
    a.wqs = (const uint8_t *) qlo;
    a.wd = (const uint16_t *) dlo;
    a.N = (int) total;
    a.nb = (int) nb;
    a.qs_span = (uint32_t) qspan;
    a.d_span = (uint32_t) dspan;
    return true;
}

void launch_row_gemv(int type, int pro, int epi, const RowArgs & a, hipStream_t s) {
    require(row_gemv_fits(type, (int64_t) a.nb * QK), "row gemv: weight type or K not supported");
    require(row_gemv_rows_fit(type, a.N, a.nb), "row gemv: weight of 2 GB or more");
    require(epi == EPI_STORE || a.N % 2 == 0, "row gemv: row-pair epilogue needs an even row count");
    require(a.nr <= 1 || epi == EPI_STORE ||
                (epi == EPI_ROPE_KV && a.nr == 3 && a.D % 2 == 0 && a.r_end[0] == a.H * a.D &&
                 a.r_end[1] == (a.H + a.Hkv) * a.D && a.r_end[2] == (a.H + 2 * a.Hkv) * a.D) ||
                (epi == EPI_SWIGLU && a.nr == 2 && a.r_end[1] == 2 * a.r_end[0]),
            "row gemv: separate q / k / v weights of H*D, Hkv*D, Hkv*D rows, or gate / up weights of equal rows");
    require(a.nr <= 1 || pro == PRO_NORM, "row gemv: several weights take the rms_norm prologue");
    require(pro != PRO_MERGE || (a.nsplit >= 1 && a.nsplit <= kMergeMax && a.D % 4 == 0 && a.nb * QK <= 4096),
            "row gemv: merge of 1.." + std::to_string(kMergeMax) + " splits, K <= 4096");
    if (type == T_Q4_0) run_row_t<T_Q4_0>(pro, epi, a, s);
    else run_row_t<T_Q8_0>(pro, epi, a, s);
    check_launch("row gemv");
}

}  // namespace gcq
