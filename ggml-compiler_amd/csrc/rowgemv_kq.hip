// rowgemv_kq.hip - ggml_mul_mat of a Q4_K / Q5_K weight with one f32 activation row, in one
// launch (runtime/src/ops.cpp:107-119 -> runtime/include/ggml_compiler_ops.h:116-122).
//
// ggml-cpu quantizes the row to Q8_K (quantize_row_q8_K) and takes vec_dot_q{4,5}_K_q8_K per
// super-block. Here one workgroup of 1024 threads per CU:
//   - its first XW wavefronts ("x waves") turn the row into Q8_K in LDS, a thread per 16 values
//     (one bsum): the super-block's signed maximum of |x| (first one on ties) over its 16 lanes,
//     iscale = -127 / max, q = min(127, rint(iscale x)), d = 1 / iscale, the thread's own bsum;
//   - the other wavefronts meanwhile stream their first weight rows: the x waves issue their row
//     loads first and the workgroup meets before any weight load is issued (a CU's loads complete
//     in issue order), and the compute wavefronts take the codes through an LDS counter;
//   - every wavefront walks groups of R whole weight rows (g, g + waves, ...), lane l taking the
//     row's 32-value tasks l, l + 64, ... (task t: super-block t / 8, chunk c = (t / 2) % 4, half
//     h = t % 2: 16 nibble bytes, whose low nibbles are values 16h.. of sub-block 2c and high
//     nibbles those of 2c + 1), so that a load moves consecutive 16-byte pieces of the packed
//     nibbles (1 KiB per instruction); each quad's four lanes load one 32-bit word each of their
//     super-block's 16-byte header (d / dmin, scales), passed around the quad by DPP; a wavefront
//     sum finishes each output. With long rows (or one group too many for the compute
//     wavefronts) the x waves take row groups too, once their prologue is done.
// Per task: (sc0 s0 + sc1 s1) d d_x - dmin (m0 bs0 + m1 bs1) d_x, s0 / s1 the exact int32 dots of
// the task's 16 values of sub-blocks 2c / 2c + 1 with their Q8_K codes and bs0 / bs1 those 16s'
// Q8_K block sums (ggml's vec_dot_q{4,5}_K_q8_K terms); the weight's bytes are read once, as
// buffer loads (an offset past the weight reads zeros).
#include "gcq_common.h"

#include <algorithm>
#include <type_traits>

namespace gcq {

int cu_count();

namespace {

constexpr int kRowKqMaxK = 16384;  // LDS holds the row's Q8_K codes, bsums and d
constexpr uint32_t kKqPast = 0x80000000u;  // a buffer offset past every weight (sizes < 2 GB)

template <int TYPE, int R, int NBL, int PRO, int EPI, int MR>
__global__ __launch_bounds__(1024) void k_row_gemv_kq(const RowKqArgs a) {
#pragma clang fp contract(off)
    static_assert(EPI == EPI_STORE || R == 2, "row-pair epilogues take two rows per group");
    constexpr bool NORM = PRO == PRO_NORM, MERGE = PRO == PRO_MERGE;
    static_assert(!MERGE || NBL <= 2, "the merge prologue takes rows of at most 4096 values");
    constexpr int NWV = 16;
    constexpr bool Q6 = TYPE == T_Q6_K;
    // 16-byte loads per task: the low bits (nibbles / Q6_K's ql), Q5_K's fifth bits / Q6_K's qh
    constexpr int WV = TYPE == T_Q4_K ? 1 : 2;
    constexpr bool XREG = NBL <= 2;                // the task activations in registers
    constexpr bool PF = WV * NBL * R <= 4;         // the next group's weights prefetched
    // x waves: at most 4 (8 for rows past 8192 values); rounds of 16 values per x thread: K / 16
    // groups over 64 XW threads (a row of NBL * 64 tasks of 32)
    constexpr int XWMAX = NBL > 4 ? 8 : 4, RMAX = NBL > 4 ? (NBL + 3) / 4 : (NBL + 1) / 2;
    // codes, 16 per entry: task t's 16 values of sub-block 2c at t, of 2c + 1 at ntask + t, so that
    // a wavefront's lanes (consecutive tasks) read consecutive entries (no bank conflicts)
    __shared__ int4 lc[kRowKqMaxK / 16];
    __shared__ uint32_t lbp[kRowKqMaxK / 32];      // per task: the two 16s' bsums (int16 each)
    __shared__ float ld[kRowKqMaxK / 256];         // d per super-block
    __shared__ unsigned int s_flag, s_norm;        // x waves done with: their codes; their norm partials
    __shared__ double red[XWMAX];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntask = a.ntask;
    const int K = ntask * 32, ngrp = K / 16;       // 16-value groups of the row
    const int nsb = ntask / 8;                     // super-blocks per row
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(a.w), 0, (int) a.span, 0x00020000);
    const int ng = (a.N + R - 1) / R;
    // MERGE: no x waves; every wavefront merges and quantizes 4 values per lane, then computes
    const int XW = MERGE ? 0 : min(XWMAX, (K + 1023) / 1024);
    const int rounds = MERGE ? 0 : (ngrp + 64 * XW - 1) / (64 * XW);
    const bool XC = MERGE || a.xc != 0;
    const int CW = XC ? NWV : NWV - XW;
    const bool xw = wave < XW;
    int g = blockIdx.x * CW + (XC ? (wave + NWV - XW) % NWV : max(wave - XW, 0));
    const int nw = gridDim.x * CW;

    if (threadIdx.x == 0) {
        s_flag = 0u;
        s_norm = 0u;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the count is zero before the workgroup meets
    }

    // Row r of group gg (wave-uniform, in scalar registers): its weight k (returned) and its index
    // there. One weight (EPI_STORE): rows in order. Several: EPI_STORE takes them in order over the
    // ranges; EPI_ROPE_KV takes separate q, k, v weights, group g < (H + Hkv) D/2 being the rotation
    // pair (i, i + D/2) of q head h (h < H) or k head h - H, then pairs of v rows; EPI_SWIGLU takes
    // gate row g and up row g. Values per weight are picked with constant indices (a dynamic index
    // into the kernel arguments becomes a memory load).
    const int hd = a.D >> 1;
    auto div_hd = [&](int x) -> int { return (int) __umulhi((uint32_t) x, a.hd_magic); };
    auto range_of = [&](int row, int & local) -> int {
        const bool k1 = a.nr > 1 && row >= a.r_end[0], k2 = a.nr > 2 && row >= a.r_end[1];
        local = k2 ? row - a.r_end[1] : k1 ? row - a.r_end[0] : row;
        return k2 ? 2 : k1 ? 1 : 0;
    };
    auto map_row = [&](int gg, int r, int & local) -> int {
        gg = __builtin_amdgcn_readfirstlane(gg);
        if constexpr (EPI == EPI_SWIGLU) {
            local = min(gg, a.r_end[0] - 1);
            return r;
        } else if constexpr (EPI == EPI_V_CACHE) {
            local = min(2 * gg + r, a.N - 1);
            return 0;
        } else if constexpr (EPI == EPI_ROPE_KV) {
            const int nq = (a.H + a.Hkv) * hd;
            const int gq = min(gg, nq - 1);
            const int h = div_hd(gq), i = gq - h * hd;
            const bool qh = h < a.H, vg = gg >= nq;
            local = vg ? min(2 * (gg - nq) + r, a.Hkv * a.D - 1) : (qh ? h : h - a.H) * a.D + i + r * hd;
            return vg ? 2 : qh ? 0 : 1;
        } else if constexpr (MR > 1) {
            return range_of(min(gg * R + r, a.N - 1), local);
        } else {
            local = min(gg * R + r, a.N - 1);
            return 0;
        }
    };
    // the weights' offsets as values (a choice between kernel-argument loads would become one
    // dynamically indexed load from a private copy of the arguments)
    auto rfl = [](uint32_t v) { return (uint32_t) __builtin_amdgcn_readfirstlane((int) v); };
    const uint32_t oq0 = rfl(a.r_qs[0]), oq1 = rfl(a.r_qs[1]), oq2 = rfl(a.r_qs[2]);
    const uint32_t oh0 = rfl(a.r_hdr[0]), oh1 = rfl(a.r_hdr[1]), oh2 = rfl(a.r_hdr[2]);
    const uint32_t ob0 = rfl(a.r_qh[0]), ob1 = rfl(a.r_qh[1]), ob2 = rfl(a.r_qh[2]);
    const uint32_t od0 = rfl(a.r_d[0]), od1 = rfl(a.r_d[1]), od2 = rfl(a.r_d[2]);
    auto pick_u = [](int k, uint32_t v0, uint32_t v1, uint32_t v2) { return k == 2 ? v2 : k == 1 ? v1 : v0; };

    // Per task and row (Q4_K / Q5_K): the 16 nibble bytes (Q5_K: and the half's 16 qh bytes) and
    // word t % 4 of the super-block's 16-byte header, the quad's four lanes holding the whole
    // header. Q6_K: the 16 ql bytes, the 16 qh bytes of its half, its 8 scale bytes, the 32-bit
    // word holding its super-block's fp16 d.
    struct Buf {
        uint4 q[NBL][R][WV];
        uint32_t h[NBL][R];
        uint2 s[Q6 ? NBL : 1][Q6 ? R : 1];
    };
    Buf wa, wb;
    auto load = [&](int gg, Buf & b) {
        const bool live = gg < ng;
        // each row's fields: byte offsets (Q6_K: r_hdr holds the scales, r_d the d values)
        uint32_t rq0[R], rh0[R], rqh0[R], rd0[R];
        bool rin[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int local;
            const int k = map_row(gg, r, local);
            rq0[r] = pick_u(k, oq0, oq1, oq2) + (uint32_t) local * (uint32_t) ntask * 16u;
            rh0[r] = pick_u(k, oh0, oh1, oh2) + (uint32_t) local * (uint32_t) nsb * 16u;
            rqh0[r] = pick_u(k, ob0, ob1, ob2) + (uint32_t) local * (uint32_t) nsb * (Q6 ? 64u : 32u);
            rd0[r] = pick_u(k, od0, od1, od2) + (uint32_t) local * (uint32_t) nsb * 2u;
            rin[r] = live && (EPI != EPI_STORE || gg * R + r < a.N);
        }
        // long rows: the tasks' offsets recomputed per group from an opaque lane index (held
        // across the groups they would spill)
        int ln = lane;
        if constexpr (!XREG) asm volatile("" : "+v"(ln));
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int t = ln + 64 * i;
            const uint32_t sb = (uint32_t) (t >> 3);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const bool in = rin[r] && t < ntask;
                if constexpr (Q6) {
                    // task t: super-block t / 8, half n = (t / 4) % 2, ql part (t / 2) % 2, l half t % 2
                    const uint32_t n = (uint32_t) ((t >> 2) & 1);
                    const uint32_t dof = rd0[r] + 2u * sb;  // the fp16 d: its aligned word
                    b.h[i][r] = __builtin_amdgcn_raw_buffer_load_b32(rq, in ? dof & ~3u : kKqPast, 0, 0);
                    const auto sc = __builtin_amdgcn_raw_buffer_load_b64(rq, in ? rh0[r] + 16u * sb + 8u * n : kKqPast, 0, 0);
                    b.s[i][r] = make_uint2(sc[0], sc[1]);
                } else {
                    b.h[i][r] = __builtin_amdgcn_raw_buffer_load_b32(
                        rq, in ? rh0[r] + 16u * sb + 4u * (uint32_t) (t & 3) : kKqPast, 0, 0);
                }
                // the low bits streamed (nt); the high bits, read by two (Q6_K) or four lanes, cached
                const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, in ? rq0[r] + 16u * (uint32_t) t : kKqPast, 0, 2);
                b.q[i][r][0] = make_uint4(q[0], q[1], q[2], q[3]);
                if constexpr (TYPE == T_Q5_K) {
                    const auto qh = __builtin_amdgcn_raw_buffer_load_b128(
                        rq, in ? rqh0[r] + 32u * sb + 16u * (uint32_t) (t & 1) : kKqPast, 0, 0);
                    b.q[i][r][1] = make_uint4(qh[0], qh[1], qh[2], qh[3]);
                }
                if constexpr (Q6) {
                    const uint32_t n = (uint32_t) ((t >> 2) & 1);
                    const auto qh = __builtin_amdgcn_raw_buffer_load_b128(
                        rq, in ? rqh0[r] + 64u * sb + 32u * n + 16u * (uint32_t) (t & 1) : kKqPast, 0, 0);
                    b.q[i][r][1] = make_uint4(qh[0], qh[1], qh[2], qh[3]);
                }
            }
        }
    };
    // word k of the header from lane k of the quad
    auto hword = [](uint32_t v, auto KI) -> uint32_t {
        constexpr int k = decltype(KI)::value;
        return (uint32_t) __builtin_amdgcn_mov_dpp((int) v, k | (k << 2) | (k << 4) | (k << 6), 0xF, 0xF, false);
    };

    // The task holding 16-value group gi of the row and which of its two 16s it is (sel). Q4_K /
    // Q5_K: group 4c + 2 sel + h of a super-block is sub-block 2c + sel, values 16h..; Q6_K: group
    // 8n + 4 sel + 2jj + h is half n, ql part jj, the low (sel 0) or high (1) nibbles, l half h.
    auto task_of = [](int gi, int & sel) -> int {
        const int gg = gi & 15;
        if constexpr (Q6) {
            sel = (gg >> 2) & 1;
            return 8 * (gi >> 4) + 4 * (gg >> 3) + (gg & 3);
        } else {
            sel = (gg >> 1) & 1;
            return 8 * (gi >> 4) + 2 * (gg >> 2) + (gg & 1);
        }
    };

    if constexpr (MERGE) {
        // The attention row merged from its split partials (the arithmetic of the decode-row
        // GEMV's merge prologue: sum_j e^(m_j - M) o_j / sum_j e^(m_j - M) l_j in split order,
        // splits with m_j = -inf left out, 0 if none), 4 values e = 4 t per thread; the partials'
        // loads are issued before any weight load.
        constexpr int KM = 8;  // splits at most (the launch checks)
        float2 mlv[KM];
        float4 pov[KM];
        const int e0 = min((int) threadIdx.x * 4, K - 4);
        const int hh = e0 / a.D;
        const float2 * ml = a.part_ml + (int64_t) hh * a.nsplit;
        const float * po = a.part_o + (int64_t) hh * a.nsplit * a.D + (e0 - hh * a.D);
#pragma unroll
        for (int j = 0; j < KM; j++) {
            if (j < a.nsplit) {
                mlv[j] = ml[j];
                pov[j] = *reinterpret_cast<const float4 *>(po + (int64_t) j * a.D);
            } else {
                mlv[j] = make_float2(-INFINITY, 0.0f);
                pov[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        load(g, wa);
        const int e = (int) threadIdx.x * 4;
        float vv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e < K) {
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < KM; j++) M = fmaxf(M, mlv[j].x);
            float L = 0.0f;
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (M != -INFINITY) {
#pragma unroll
                for (int j = 0; j < KM; j++) {
                    if (mlv[j].x == -INFINITY) continue;
                    const float wj = __expf(mlv[j].x - M);
                    L += wj * mlv[j].y;
                    o.x += wj * pov[j].x;
                    o.y += wj * pov[j].y;
                    o.z += wj * pov[j].z;
                    o.w += wj * pov[j].w;
                }
            }
            vv[0] = L == 0.0f ? 0.0f : o.x / L;
            vv[1] = L == 0.0f ? 0.0f : o.y / L;
            vv[2] = L == 0.0f ? 0.0f : o.z / L;
            vv[3] = L == 0.0f ? 0.0f : o.w / L;
        }
        // Q8_K of the wavefront's super-block (its 64 lanes' 256 values): the first largest |x|
        float ax = 0.0f, mx = 0.0f;
        int idx = 1 << 30;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (fabsf(vv[j]) > ax) {
                ax = fabsf(vv[j]);
                mx = vv[j];
                idx = e + j;
            }
        }
        auto take = [&](float ax2, float mx2, int idx2) {
            if (ax2 > ax || (ax2 == ax && idx2 < idx)) {
                ax = ax2;
                mx = mx2;
                idx = idx2;
            }
        };
        take(lane_pair<1>(ax), lane_pair<1>(mx), lane_pair_i<1>(idx));
        take(lane_pair<2>(ax), lane_pair<2>(mx), lane_pair_i<2>(idx));
        take(lane_pair<4>(ax), lane_pair<4>(mx), lane_pair_i<4>(idx));
        take(lane_pair<8>(ax), lane_pair<8>(mx), lane_pair_i<8>(idx));
        take(__shfl_xor(ax, 16), __shfl_xor(mx, 16), __shfl_xor(idx, 16));
        take(__shfl_xor(ax, 32), __shfl_xor(mx, 32), __shfl_xor(idx, 32));
        int q[4] = {0, 0, 0, 0};
        float d = 0.0f;
        if (ax != 0.0f) {
            const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int rr = (int) __builtin_rintf(iscale * vv[j]);
                q[j] = rr < 127 ? rr : 127;
            }
            d = __fdiv_rn(1.0f, iscale);
        }
        const int word = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
        int s4 = q[0] + q[1] + q[2] + q[3];
        s4 += lane_pair_i<1>(s4);
        s4 += lane_pair_i<2>(s4);  // the 16-value group's bsum (its 4 lanes)
        if (e < K) {
            const int gi = (int) threadIdx.x >> 2;
            int sel;
            const int t = task_of(gi, sel);
            reinterpret_cast<int *>(lc + sel * ntask + t)[threadIdx.x & 3] = word;
            if ((threadIdx.x & 3) == 0) reinterpret_cast<int16_t *>(lbp)[2 * t + sel] = (int16_t) s4;
            if (lane == 0) ld[wave] = d;  // the wavefront's 256 values are super-block `wave`
        }
        if (lane == 0) lds_signal(&s_flag);
    } else if (xw) {
        // the row's loads first, then the workgroup meets (no weight load is ahead of them)
        float4 xv[RMAX][4], nv[NORM ? RMAX : 1][4];
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            const int gi = (int) threadIdx.x + r * XW * 64;
            if (r < rounds && gi < ngrp) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    xv[r][k] = *reinterpret_cast<const float4 *>(a.x + gi * 16 + 4 * k);
                    if constexpr (NORM) {  // the norm weight at any 4-byte alignment
                        const float * wp = a.norm_w + gi * 16 + 4 * k;
                        nv[r][k] = make_float4(wp[0], wp[1], wp[2], wp[3]);
                    }
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    xv[r][k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if constexpr (NORM) nv[r][k] = xv[r][k];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        float scale = 1.0f;
        if constexpr (NORM) {
            // ggml_rms_norm: squares rounded to f32, summed in double, the mean rounded to f32
            double ss = 0.0;
#pragma unroll
            for (int r = 0; r < RMAX; r++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    ss += (double) (xv[r][k].x * xv[r][k].x);
                    ss += (double) (xv[r][k].y * xv[r][k].y);
                    ss += (double) (xv[r][k].z * xv[r][k].z);
                    ss += (double) (xv[r][k].w * xv[r][k].w);
                }
            ss = wave_sum_d(ss);
            if (lane == 0) {
                red[wave] = ss;
                lds_signal(&s_norm);
            }
            lds_wait(&s_norm, XW);
            double tot = 0.0;
#pragma unroll
            for (int i = 0; i < XWMAX; i++)
                if (i < XW) tot += red[i];
            scale = 1.0f / sqrtf((float) (tot / (double) K) + a.eps);
        }
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            const int gi = (int) threadIdx.x + r * XW * 64;
            if (r >= rounds) break;
            float v[16] = {xv[r][0].x, xv[r][0].y, xv[r][0].z, xv[r][0].w, xv[r][1].x, xv[r][1].y,
                           xv[r][1].z, xv[r][1].w, xv[r][2].x, xv[r][2].y, xv[r][2].z, xv[r][2].w,
                           xv[r][3].x, xv[r][3].y, xv[r][3].z, xv[r][3].w};
            if constexpr (NORM) {
                const float w16[16] = {nv[r][0].x, nv[r][0].y, nv[r][0].z, nv[r][0].w, nv[r][1].x, nv[r][1].y,
                                       nv[r][1].z, nv[r][1].w, nv[r][2].x, nv[r][2].y, nv[r][2].z, nv[r][2].w,
                                       nv[r][3].x, nv[r][3].y, nv[r][3].z, nv[r][3].w};
#pragma unroll
                for (int j = 0; j < 16; j++) v[j] = (v[j] * scale) * w16[j];
            }
            // the super-block's first largest |x| (its 16 groups are 16 consecutive lanes)
            float ax = 0.0f, mx = 0.0f;
            int idx = 1 << 30;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (fabsf(v[j]) > ax) {
                    ax = fabsf(v[j]);
                    mx = v[j];
                    idx = (lane & 15) * 16 + j;
                }
            }
            auto take = [&](float ax2, float mx2, int idx2) {
                if (ax2 > ax || (ax2 == ax && idx2 < idx)) {
                    ax = ax2;
                    mx = mx2;
                    idx = idx2;
                }
            };
            take(lane_pair<1>(ax), lane_pair<1>(mx), lane_pair_i<1>(idx));
            take(lane_pair<2>(ax), lane_pair<2>(mx), lane_pair_i<2>(idx));
            take(lane_pair<4>(ax), lane_pair<4>(mx), lane_pair_i<4>(idx));
            take(lane_pair<8>(ax), lane_pair<8>(mx), lane_pair_i<8>(idx));
            int q[16];
            float d = 0.0f;
            if (ax != 0.0f) {
                const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int rr = (int) __builtin_rintf(iscale * v[j]);
                    q[j] = rr < 127 ? rr : 127;
                }
                d = __fdiv_rn(1.0f, iscale);
            } else {
#pragma unroll
                for (int j = 0; j < 16; j++) q[j] = 0;
            }
            if (gi < ngrp) {
                int pk[4], s = 0;
#pragma unroll
                for (int k = 0; k < 4; k++)
                    pk[k] = (q[4 * k] & 0xff) | ((q[4 * k + 1] & 0xff) << 8) | ((q[4 * k + 2] & 0xff) << 16) |
                            ((q[4 * k + 3] & 0xff) << 24);
#pragma unroll
                for (int j = 0; j < 16; j++) s += q[j];
                int sel;
                const int t = task_of(gi, sel);
                lc[sel * ntask + t] = make_int4(pk[0], pk[1], pk[2], pk[3]);
                reinterpret_cast<int16_t *>(lbp)[2 * t + sel] = (int16_t) s;
                if ((lane & 15) == 0) ld[gi >> 4] = d;
            }
            __builtin_amdgcn_sched_barrier(0);  // one round at a time (its codes are 16 registers)
        }
        if (lane == 0) lds_signal(&s_flag);
        if (!XC) return;
        load(g, wa);
    } else {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        load(g, wa);
    }
    lds_wait(&s_flag, MERGE ? NWV : XW);
    if constexpr (PF) load(g + nw, wb);

    // The lane's task activations: the 16 codes of sub-block 2c, of 2c + 1, d_x, bs0 d_x, bs1 d_x.
    int4 xa[XREG ? NBL : 1], xb[XREG ? NBL : 1];
    float xs[XREG ? NBL : 1], xo[XREG ? NBL : 1], xo2[XREG ? NBL : 1];
    auto act = [&](int i, int4 & ca, int4 & cb, float & ds, float & o1, float & o2) {
        int t = lane + 64 * i;
        // read from LDS once per group: an opaque index keeps the compiler from holding every
        // task's activations in registers across the groups (they would spill)
        if constexpr (!XREG) {
            asm volatile("" : "+v"(t));
            // past the row: a task of the row read instead, whose products with the zero weights
            // (and zero header: d = dmin = 0) add exact zeros
            t = min(t, ntask - 1);
        }
        if (!XREG || t < ntask) {
            ca = lc[t];
            cb = lc[ntask + t];
            ds = ld[t >> 3];
            const uint32_t bp = lbp[t];
            if constexpr (Q6) {  // -32 bsum of each 16 (Q6_K's offset), as integers in float registers
                o1 = __int_as_float(-32 * (int) (int16_t) (bp & 0xffffu));
                o2 = __int_as_float(-32 * (int) (int16_t) (bp >> 16));
            } else {
                o1 = (float) (int) (int16_t) (bp & 0xffffu) * ds;
                o2 = (float) (int) (int16_t) (bp >> 16) * ds;
            }
        } else {
            ca = make_int4(0, 0, 0, 0);
            cb = ca;
            ds = 0.0f;
            o1 = 0.0f;
            o2 = 0.0f;
        }
    };
    if constexpr (XREG) {
#pragma unroll
        for (int i = 0; i < NBL; i++) act(i, xa[i], xb[i], xs[i], xo[i], xo2[i]);
    }
    auto dot16 = [](const int (&q)[4], const int4 x) {
        int s = __builtin_amdgcn_sdot4(q[0], x.x, 0, true);
        s = sdot4(q[1], x.y, s);
        s = sdot4(q[2], x.z, s);
        return sdot4(q[3], x.w, s);
    };
    // the lane's chunk within the super-block (the same for all its tasks: 64 tasks are 8 super-blocks)
    const int c = (lane >> 1) & 3;
    const uint32_t csh = 16u * (uint32_t) (c & 1);
    const uint32_t chim = c >= 2 ? 0xFFFFFFFFu : 0u;

    // Q6_K: the task's ql part (t / 2) % 2 picks the qh bit pairs; byte t % 4 of its scale words;
    // the half of the d word its super-block's parity picks (rows of an odd number of super-blocks
    // alternate it per row)
    const uint32_t sh6 = 2u * (uint32_t) ((lane >> 1) & 1);
    const uint32_t bsel = 8u * (uint32_t) (lane & 3);
    const int sbp = (lane >> 3) & 1;

    auto group = [&](int gg, const Buf & b) {
        float acc[R];
        int dsh[R];  // Q6_K: each row's d half
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] = 0.0f;
            int local = 0;
            if constexpr (Q6) (void) map_row(gg, r, local);
            dsh[r] = 16 * ((local & nsb & 1) ^ sbp);
        }
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            int4 ca, cb;
            float ds, o1, o2;
            if constexpr (XREG) {
                ca = xa[i];
                cb = xb[i];
                ds = xs[i];
                o1 = xo[i];
                o2 = xo2[i];
            } else {
                act(i, ca, cb, ds, o1, o2);  // zeros past the row, as its weights
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                if constexpr (Q6) {
                    // the task's 16 values of its first 16-group (low nibbles of ql, qh bits 2jj) and
                    // of the group 64 values on (high nibbles, qh bits 2jj + 4): 6-bit codes q, the
                    // products sum sc (q - 32) x
                    int lo6[4], hi6[4];
                    const uint4 ql = b.q[i][r][0], qh = b.q[i][r][1];
                    const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w}, hw6[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        lo6[j] = (int) ((lw[j] & 0x0F0F0F0Fu) | (((hw6[j] >> sh6) & 0x03030303u) << 4));
                        hi6[j] = (int) (((lw[j] >> 4) & 0x0F0F0F0Fu) | (((hw6[j] >> (sh6 + 4)) & 0x03030303u) << 4));
                    }
                    const int sc1 = (int) (int8_t) (b.s[i][r].x >> bsel), sc2 = (int) (int8_t) (b.s[i][r].y >> bsel);
                    const int isum = sc1 * (dot16(lo6, ca) + __float_as_int(o1)) + sc2 * (dot16(hi6, cb) + __float_as_int(o2));
                    const float dd = h2f((uint16_t) (b.h[i][r] >> dsh[r]));
                    acc[r] += ((float) isum * dd) * ds;
                    continue;
                }
                // the task's 16 values of sub-block 2c (low nibbles) and of 2c + 1 (high nibbles)
                int lo[4], hi[4];
                const uint4 q = b.q[i][r][0];
                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo[j] = (int) (qw[j] & 0x0F0F0F0Fu);
                    hi[j] = (int) ((qw[j] >> 4) & 0x0F0F0F0Fu);
                }
                if constexpr (TYPE == T_Q5_K) {  // the fifth bits: bit 2c of qh[l] (sub-block 2c), 2c + 1
                    const uint4 qh = b.q[i][r][1];
                    const uint32_t hb[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        lo[j] |= (int) (((hb[j] >> (2 * c)) & 0x01010101u) << 4);
                        hi[j] |= (int) (((hb[j] >> (2 * c + 1)) & 0x01010101u) << 4);
                    }
                }
                // the 6-bit scales and mins of sub-blocks 2c and 2c + 1 (ggml's get_scale_min_k4)
                using I = int;
                const uint32_t h0 = hword(b.h[i][r], std::integral_constant<I, 0>{});
                const uint32_t A = hword(b.h[i][r], std::integral_constant<I, 1>{}) >> csh;
                const uint32_t M = hword(b.h[i][r], std::integral_constant<I, 2>{}) >> csh;
                const uint32_t H = hword(b.h[i][r], std::integral_constant<I, 3>{}) >> csh;
                // chunks 2, 3 take the high form; chosen by a mask (a select here became a branch)
                const uint32_t scp = (chim & ((H & 0x0F0Fu) | ((A >> 2) & 0x3030u))) | (~chim & (A & 0x3F3Fu));
                const uint32_t mp = (chim & (((H >> 4) & 0x0F0Fu) | ((M >> 2) & 0x3030u))) | (~chim & (M & 0x3F3Fu));
                const int sc0 = (int) (scp & 0xFFu), sc1 = (int) ((scp >> 8) & 0xFFu);
                const int m0 = (int) (mp & 0xFFu), m1 = (int) ((mp >> 8) & 0xFFu);
                const float dd = h2f((uint16_t) (h0 & 0xffff)), dmin = h2f((uint16_t) (h0 >> 16));
                const float fm0 = (float) m0 * dmin, fm1 = (float) m1 * dmin;
                const int isc = sc0 * dot16(lo, ca) + sc1 * dot16(hi, cb);
                const float fmin = __builtin_fmaf(fm0, o1, fm1 * o2);
                acc[r] += __builtin_fmaf((float) isc * dd, ds, -fmin);
            }
            // one task's activations in registers at a time
            if constexpr (!XREG) __builtin_amdgcn_sched_barrier(0);
        }
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = wave_sum(acc[r]);
        // What the epilogues read (residual, position, rotation) comes through the scalar unit
        // (constant-space pointers): a vector load here would wait for every weight load issued
        // before it (the next groups'), as loads complete in order.
        typedef const float __attribute__((address_space(4))) cfloat_t;
        gg = __builtin_amdgcn_readfirstlane(gg);
        if constexpr (EPI == EPI_STORE && MR > 1) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = gg * R + r;
                if (lane == r && row < a.N) {
                    int local;
                    const int k = range_of(row, local);
                    float * y = k == 2 ? a.r_y[2] : k == 1 ? a.r_y[1] : a.r_y[0];
                    y[local] = v[r];
                }
            }
        } else if constexpr (EPI == EPI_STORE) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = gg * R + r;
                // each residual value is read before its own output is written and never after
                // another output (res may be y itself)
                const float rv = a.res && row < a.N ? ((cfloat_t *) a.res)[row] : 0.0f;
                if (lane == r && row < a.N) a.y[row] = a.res ? v[r] + rv : v[r];
            }
        } else if constexpr (EPI == EPI_SWIGLU) {  // k_swiglu's arithmetic: g / (1 + e^-g) * u
            if (lane == 0) a.y[gg] = v[0] / (1.0f + expf(-v[0])) * v[1];
        } else if constexpr (EPI == EPI_V_CACHE) {  // the v pair to the f16 v cache at the position
            typedef const int __attribute__((address_space(4))) cint_t;
            const int p = ((cint_t *) a.pos)[0];
            if (p >= 0 && p < a.ctx && lane == 0) {
                const int e = 2 * gg;  // v value index over [Hkv][D]
                const int hv = div_hd(e) >> 1, dd = e - hv * a.D;
                const uint32_t pair = f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
                *reinterpret_cast<uint32_t *>(a.vc + ((int64_t) hv * a.ctx + p) * a.D + dd) = pair;
            }
        } else {  // EPI_ROPE_KV: q roped to y, k roped and v to the f16 caches at the position
            typedef const int __attribute__((address_space(4))) cint_t;
            const int p = ((cint_t *) a.pos)[0];
            const int nqk = (a.H + a.Hkv) * hd;
            if (p >= 0 && p < a.ctx) {
                if (gg < nqk) {
                    const int h = div_hd(gg), i = gg - h * hd;
                    const cfloat_t * cs = (cfloat_t *) a.rope_cs + 2 * i;
                    const float2 yr = rope_pair(v[0], v[1], make_float2(cs[0], cs[1]));
                    if (lane == 0) {
                        if (h < a.H) {
                            a.y[h * a.D + i] = yr.x;
                            a.y[h * a.D + i + hd] = yr.y;
                        } else {
                            uint16_t * kr = a.kc + ((int64_t) (h - a.H) * a.ctx + p) * a.D;
                            kr[i] = f2h(yr.x);
                            kr[i + hd] = f2h(yr.y);
                        }
                    }
                } else if (lane == 0) {
                    const int e = 2 * (gg - nqk);  // v value index over [Hkv][D]
                    const int hv = div_hd(e) >> 1, dd = e - hv * a.D;
                    const uint32_t pair = f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
                    *reinterpret_cast<uint32_t *>(a.vc + ((int64_t) hv * a.ctx + p) * a.D + dd) = pair;
                }
            }
        }
    };

    if constexpr (PF) {
        // two buffers in turn: a group's weights are loaded two groups ahead
        while (g < ng) {
            group(g, wa);
            load(g + 2 * nw, wa);
            g += nw;
            if (g >= ng) break;
            group(g, wb);
            load(g + 2 * nw, wb);
            g += nw;
        }
    } else {
        while (g < ng) {
            group(g, wa);
            g += nw;
            if (g < ng) load(g, wa);
        }
    }
}

template <int TYPE, int PRO, int EPI, int MR>
void go_kq(int R, int nbl, const RowKqArgs & a, int grid, hipStream_t s) {
#define GCQ_KQ(RR, NB)                                                          \
    if (R == RR && nbl == NB) {                                                 \
        k_row_gemv_kq<TYPE, RR, NB, PRO, EPI, MR><<<grid, 1024, 0, s>>>(a);     \
        return;                                                                 \
    }
    GCQ_KQ(2, 1)
    GCQ_KQ(2, 2)
    if constexpr (PRO == PRO_MERGE) {
        GCQ_KQ(1, 1)
        GCQ_KQ(1, 2)
    } else if constexpr (EPI == EPI_STORE) {
        GCQ_KQ(1, 1)
        GCQ_KQ(1, 2)
        GCQ_KQ(1, 3)
        GCQ_KQ(1, 4)
        if constexpr (MR == 1) {  // rows past 8192 values: one weight
            GCQ_KQ(1, 5)
            GCQ_KQ(1, 6)
            GCQ_KQ(1, 7)
            GCQ_KQ(1, 8)
        }
    }
#undef GCQ_KQ
    fail("row gemv kq: no kernel for " + std::to_string(R) + " rows of " + std::to_string(nbl) + " tasks per lane");
}

template <int TYPE>
void go_kq_t(int pro, int epi, bool multi, int R, int nbl, const RowKqArgs & a, int grid, hipStream_t s) {
    if (epi == EPI_ROPE_KV) return go_kq<TYPE, PRO_NORM, EPI_ROPE_KV, 3>(R, nbl, a, grid, s);
    if (epi == EPI_SWIGLU) return go_kq<TYPE, PRO_NORM, EPI_SWIGLU, 3>(R, nbl, a, grid, s);
    if (epi == EPI_V_CACHE) return go_kq<TYPE, PRO_NORM, EPI_V_CACHE, 1>(R, nbl, a, grid, s);
    if (multi) return go_kq<TYPE, PRO_NORM, EPI_STORE, 3>(R, nbl, a, grid, s);
    if (pro == PRO_NORM) return go_kq<TYPE, PRO_NORM, EPI_STORE, 1>(R, nbl, a, grid, s);
    if (pro == PRO_MERGE) return go_kq<TYPE, PRO_MERGE, EPI_STORE, 1>(R, nbl, a, grid, s);
    go_kq<TYPE, PRO_PLAIN, EPI_STORE, 1>(R, nbl, a, grid, s);
}

bool kq_rows_fit(int type, int64_t K) {
    // rows up to 16384 values (the LDS row)
    return (type == T_Q4_K || type == T_Q5_K || type == T_Q6_K) && K > 0 && K % QKK == 0 && K <= kRowKqMaxK;
}

}  // namespace

bool row_gemv_kq_fits(int type, int64_t N, int64_t K) {
    // more rows stream faster through the batched kernel after a separate quantization
    return kq_rows_fit(type, K) && N > 0 && N <= 8192 && weight_layout(type, N, K).total < 0x80000000ull;
}

// With the rms_norm prologue (a normalized row read by several projections, each normalizing it
// itself): up to 16384 rows, where it also saves the norm's and the quantization's launches.
bool row_gemv_kq_norm_fits(int type, int64_t N, int64_t K) {
    return kq_rows_fit(type, K) && N > 0 && N <= 16384 && weight_layout(type, N, K).total < 0x80000000ull;
}

bool row_gemv_kq_epi_fits(int type, int epi, int64_t K) {
    return kq_rows_fit(type, K) && (epi == EPI_STORE || K <= 4096);
}

bool row_gemv_kq_ranges(int type, int n, const uint8_t * const * w, const int64_t * N, int64_t K, RowKqArgs & a) {
    if (n < 1 || n > 3 || !kq_rows_fit(type, K) || K > 8192) return false;  // several weights: rows of 8192 at most
    uintptr_t lo = UINTPTR_MAX;
    int64_t total = 0;
    for (int k = 0; k < n; k++) {
        if (N[k] <= 0) return false;
        lo = std::min(lo, (uintptr_t) w[k]);
        total += N[k];
    }
    uint64_t span = 0;
    for (int k = 0; k < n; k++) {
        const uint64_t o = (uint64_t) ((uintptr_t) w[k] - lo);
        const WeightLayout L = weight_layout(type, N[k], K);
        span = std::max(span, o + L.total);
        if (span >= 0x80000000ull) return false;
        a.r_qs[k] = (uint32_t) (o + L.qs);
        a.r_qh[k] = (uint32_t) (o + L.qh);
        a.r_hdr[k] = (uint32_t) (o + (type == T_Q6_K ? L.sc : L.d));
        a.r_d[k] = (uint32_t) (o + L.d);
        a.r_end[k] = (int) ((k ? a.r_end[k - 1] : 0) + N[k]);
    }
    if (total > INT32_MAX) return false;
    a.nr = n;
    a.w = (const uint8_t *) lo;
    a.N = (int) total;
    a.ntask = (int) (K / 32);
    a.span = (uint32_t) span;
    return true;
}

// The launch behind every K-quant row GEMV: one weight (EPI_STORE, optional residual, optional
// norm) or several of one row length read by the one normalized row (EPI_STORE to r_y, or the
// row-pair epilogues).
void launch_row_gemv_kq_epi(int type, int pro, int epi, const RowKqArgs & a0, hipStream_t s) {
    RowKqArgs a = a0;
    require((pro == PRO_PLAIN || pro == PRO_NORM || pro == PRO_MERGE) && (pro == PRO_NORM) == (a.norm_w != nullptr),
            "row gemv kq: plain, norm (with norm_w) or merge prologue");
    require(pro != PRO_MERGE || (epi == EPI_STORE && a.nr <= 1 && a.ntask * 32 <= 4096 && a.nsplit >= 1 &&
                                 a.nsplit <= 8 && a.D > 0 && a.D % 4 == 0 && (a.ntask * 32) % a.D == 0),
            "row gemv kq: merge of 1..8 splits of D-value heads (D a multiple of 4), K <= 4096, one weight");
    const int64_t K = (int64_t) a.ntask * 32;
    require(row_gemv_kq_epi_fits(type, epi, K),
            "row gemv kq: Q4_K / Q5_K / Q6_K, K a multiple of 256 up to 16384 (8192 for several weights, 4096 for the row-pair epilogues)");
    const bool multi = a.nr > 1;
    require(a.N > 0 && (uint64_t) a.span < 0x80000000ull && (!multi || a.r_end[a.nr - 1] == a.N),
            "row gemv kq: weights of 2 GB or more");
    require(!multi || a.norm_w, "row gemv kq: several weights take the rms_norm prologue");
    require(!multi || K <= 8192, "row gemv kq: several weights take rows of at most 8192 values");
    require(epi == EPI_STORE || a.N % 2 == 0, "row gemv kq: row-pair epilogue needs an even row count");
    require(epi == EPI_STORE ||
                (epi == EPI_ROPE_KV && a.D % 2 == 0 && a.D > 0 && a.r_end[0] == a.H * a.D &&
                 a.r_end[1] == (a.H + a.Hkv) * a.D && (a.nr == 2 || (a.nr == 3 && a.r_end[2] == (a.H + 2 * a.Hkv) * a.D))) ||
                (epi == EPI_SWIGLU && a.nr == 2 && a.r_end[1] == 2 * a.r_end[0]) ||
                (epi == EPI_V_CACHE && a.nr <= 1 && a.D % 2 == 0 && a.D > 0 && a.N == a.Hkv * a.D && a.norm_w),
            "row gemv kq: separate q / k [/ v] weights of H*D, Hkv*D [, Hkv*D] rows, gate / up weights of equal rows, "
            "or a v weight of Hkv*D rows");
    require(!multi || !a.res, "row gemv kq: several weights take no residual");
    if (epi == EPI_ROPE_KV || epi == EPI_V_CACHE) {
        const uint64_t hd = (uint64_t) (a.D / 2);
        require((uint64_t) a.N * hd < (1ull << 32), "row gemv kq: rope epilogue indices past 2^32 / (D/2)");
        a.hd_magic = (uint32_t) ((1ull << 32) / hd + 1);
    }
    const int nbl = (a.ntask + 63) / 64;
    const int cus = cu_count();
    const int xw = pro == PRO_MERGE ? 0 : std::min(nbl > 4 ? 8 : 4, (int) ((K + 1023) / 1024));  // the kernel's XW
    // two rows per group when every compute wavefront of the grid gets one and the rows are short
    // (Q5_K's tasks hold twice the registers: one row, whose next group's weights are prefetched);
    // the row-pair epilogues always take two
    const int R = epi != EPI_STORE || (type == T_Q4_K && nbl <= 2 && a.N / 2 >= (int64_t) cus * (16 - xw)) ? 2 : 1;
    // (Q5_K / Q6_K: one row, as their tasks hold twice the weight registers)
    const int64_t ng = (a.N + R - 1) / R;
    // the x waves take groups too when the compute wavefronts alone would need one more round
    a.xc = pro == PRO_MERGE || (ng <= 16LL * cus && ng > (int64_t) (16 - xw) * cus);
    const int cw = a.xc ? 16 : 16 - xw;
    const int grid = (int) std::max<int64_t>(1, std::min<int64_t>(cus, (ng + cw - 1) / cw));
    if (type == T_Q4_K) go_kq_t<T_Q4_K>(pro, epi, multi, R, nbl, a, grid, s);
    else if (type == T_Q5_K) go_kq_t<T_Q5_K>(pro, epi, multi, R, nbl, a, grid, s);
    else go_kq_t<T_Q6_K>(pro, epi, multi, R, nbl, a, grid, s);
    check_launch("row gemv kq");
}

// One packed weight of N rows of K as RowKqArgs' weight fields.
void row_gemv_kq_one(int type, const void * w, int64_t N, int64_t K, RowKqArgs & a) {
    const WeightLayout L = weight_layout(type, N, K);
    a.w = (const uint8_t *) w;
    a.r_qs[0] = (uint32_t) L.qs;
    a.r_qh[0] = (uint32_t) L.qh;
    a.r_hdr[0] = (uint32_t) (type == T_Q6_K ? L.sc : L.d);
    a.r_d[0] = (uint32_t) L.d;
    a.span = (uint32_t) L.total;
    a.N = (int) N;
    a.ntask = (int) (K / 32);
}

// y[n] (+ res[n]) = sum_k W[n, k] x'[k] for a packed Q4_K / Q5_K / Q6_K weight, x' = x or, with
// norm_w, ggml_mul(ggml_rms_norm(x, eps), norm_w).
void launch_row_gemv_kq(int type, const void * w, int64_t N, int64_t K, const float * x, const float * norm_w, float eps,
                        float * y, const float * res, hipStream_t s) {
    require(norm_w ? row_gemv_kq_norm_fits(type, N, K) : row_gemv_kq_fits(type, N, K),
            "row gemv kq: Q4_K / Q5_K / Q6_K, K a multiple of 256 up to 16384, up to 8192 rows (16384 with the norm)");
    RowKqArgs a{};
    row_gemv_kq_one(type, w, N, K, a);
    a.x = x;
    a.y = y;
    a.res = res;
    a.norm_w = norm_w;
    a.eps = eps;
    launch_row_gemv_kq_epi(type, norm_w ? PRO_NORM : PRO_PLAIN, EPI_STORE, a, s);
}

}  // namespace gcq
