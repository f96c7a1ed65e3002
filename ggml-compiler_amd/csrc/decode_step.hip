// decode_step.hip - every layer of one decode step in a single persistent launch.
//
// The layer-by-layer decode (llama.hip's decode_layer: five launches per layer, the row GEMVs of
// rowgemv.hip and the lane-group attention of attn.hip) pays, per launch, the ramp before the
// first weight bytes arrive and the drain after the last, with HBM idle in between. Here one
// workgroup per CU runs all layers, the phases of a layer
//
//   QKV   rms_norm(x) * attn_norm -> Q8_0 -> packed QKV rows -> rope q, k; k, v into the cache
//   ATT   split-K attention of each query head over the cache (the step's pos visible)
//   O     merge of the splits -> Q8_0 -> output projection + x -> x
//   GU    rms_norm(x) * ffn_norm -> Q8_0 -> gate/up row pairs -> silu(g) * u -> h
//   DOWN  Q8_0 of h -> down projection + x -> x
//
// separated by grid barriers. Within a phase the row GEMV's order is kept: the x waves issue the
// activation loads, the workgroup meets, the other wavefronts start the weight stream, then the x
// waves convert.
//
// Measured on MI355X (8B-shaped Q4_0 decoder, 512-token context; the per-phase clock of
// gcq_llama_step_trace): 1.1-1.3 us from the last workgroup's arrival to the barrier's release,
// and phases as long as the matching standalone launches or longer (QKV 9.7 us, attention 6.8,
// output projection 9.2, gate/up 18.5, down 10.6 per layer), 570 tok/s against 736 for the
// per-layer launches. Issuing the next phase's weight loads before the barrier (tried) does not
// help: a CU's vector memory requests issue and return in order, so the phase's activation loads,
// which can only be issued after the barrier, queue behind them, and with the queue full even the
// issue of other vector memory instructions waits. The path is therefore not the default.
//
// The arithmetic is the layer-by-layer path's, operation for operation: the same prologue
// partitions (norm sums over the same x waves, the same Q8_0 conversions), per-lane block order
// and wavefront reductions in the GEMVs, the lane-group attention of k_attn_lanes<D, 1, 16> with
// the host's split plan, and the merge of k_merge_q8 / the GEMV merge prologue. The two paths give
// the same logits bit for bit.
//
// Memory between phases: the eight XCDs' L2 caches are not coherent with each other within a
// launch. Data one phase writes and another reads (x, q, h, the attention partials, the step's
// K / V row) is stored with sc1 (write-through to the device-coherent level), each at an address
// written once per launch (x, q, h and the partials in rings: one slot per layer and write, every
// slot starting on its own 256-byte boundary so that no cache line holds two slots), so a plain
// load in another XCD misses its L2 and reads the new value, and the XCD's other readers then hit
// its L2. The barrier: each workgroup's stores complete (s_waitcnt), then one thread per
// workgroup adds to its arrival group's counter (8 groups); the last of a group adds to the group
// counter, the last group raises the 8 group flags to the barrier's number; a workgroup waits on
// its group's flag (2.3 us per barrier over 256 idle workgroups in isolation; one counter for all:
// 4.4 us). Every wait gives up after a bounded spin and raises an error word the host checks,
// so a barrier that cannot complete ends the kernel instead of hanging it; the counters return to
// zero at the end of each launch (the last workgroup to leave clears them).
#include "gcq_common.h"
#include "grid_sync.h"

#include <algorithm>

namespace gcq {

int cu_count();

namespace {

constexpr int kThreads = 1024, kWaves = 16;
constexpr int kMaxK = 16384;       // LDS holds one activation row: K codes + K/32 (d, sum)
constexpr int kMaxSplit = 8;       // attention splits the O prologue merges
constexpr uint32_t kPast = 0x80000000u;    // a buffer offset past every buffer: reads zeros
constexpr int kCohere = 16;                // buffer cache policy: sc1 (device-coherent)

// Workgroup barrier for LDS data only: waits for this wavefront's LDS operations, not for its
// global loads (a __syncthreads may wait for every outstanding load, prefetched weights included).
__device__ __forceinline__ void wg_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}


__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void * p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int) bytes, 0x00020000);
}
// Reads of data written earlier in the launch: plain (L2-cached) loads, which is correct because
// every such buffer is written once per launch at an address no workgroup read before in it (the
// rings of StepArgs), so no L2 holds an older copy; within an XCD the readers after the first then
// hit its L2 instead of all 256 CUs fetching the same lines from memory.
__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_float4(__uint_as_float(t[0]), __uint_as_float(t[1]), __uint_as_float(t[2]), __uint_as_float(t[3]));
}
__device__ __forceinline__ float2 ld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_float2(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void st1_co(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kCohere);
}
__device__ __forceinline__ void st_u32_co(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kCohere);
}
__device__ __forceinline__ void st_u16_co(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kCohere);
}

// ------------------------------------------------------------------- weight stream

// One packed weight (N rows of nb blocks): its buffer descriptors and grouping. A wavefront's
// work is a list of steps: row group g (R rows), chunk c of 128 blocks; in a step lane l holds
// blocks 128c + l and 128c + 64 + l of each row (16 B of codes per block and row for Q4_0, 32 B
// for Q8_0, plus the 32-bit word holding the block's fp16 scale).
struct WSrc {
    __amdgpu_buffer_rsrc_t rq, rd;
    int N, nb, ng, nchunk;
};

template <int TYPE>
__device__ __forceinline__ WSrc wsrc(const uint8_t * qs, const uint16_t * d, int N, int nb, int R) {
    constexpr uint32_t CB = TYPE == T_Q4_0 ? 16u : 32u;
    WSrc s;
    s.rq = rsrc(qs, (uint32_t) N * (uint32_t) nb * CB);
    s.rd = rsrc(d, (((uint32_t) N * (uint32_t) nb + 1u) / 2u) * 4u);
    s.N = N;
    s.nb = nb;
    s.ng = (N + R - 1) / R;
    s.nchunk = (nb + 127) / 128;
    return s;
}

template <int TYPE, int R>
struct WStep {
    static constexpr int CV = TYPE == T_Q4_0 ? 1 : 2;
    uint4 w[2][R][CV];
    uint32_t d[2][R];
};

// Loads of step (g, c) into b (zeros, with no memory access, past the weight's end).
template <int TYPE, int R>
__device__ __forceinline__ void load_step(const WSrc & s, int g, int c, WStep<TYPE, R> & b, int lane) {
    constexpr int CV = WStep<TYPE, R>::CV;
    const bool live = g < s.ng;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int blk = 128 * c + lane + 64 * i;
        const bool in = live && blk < s.nb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(g * R + r, s.N - 1);
            const uint32_t o = (uint32_t) row * (uint32_t) s.nb + (uint32_t) blk;
#pragma unroll
            for (int cc = 0; cc < CV; cc++) {
                const auto t = __builtin_amdgcn_raw_buffer_load_b128(s.rq, in ? (o * CV + cc) * 16u : kPast, 0, 2);
                b.w[i][r][cc] = make_uint4(t[0], t[1], t[2], t[3]);
            }
            b.d[i][r] = __builtin_amdgcn_raw_buffer_load_b32(s.rd, in ? (o >> 1) * 4u : kPast, 0, 0);
        }
    }
}

template <int TYPE, int R>
__device__ __forceinline__ void zero(WStep<TYPE, R> & b) {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int c = 0; c < WStep<TYPE, R>::CV; c++) b.w[i][r][c] = make_uint4(0u, 0u, 0u, 0u);
            b.d[i][r] = 0u;
        }
}

// Block dots of step (g, c) against the activation codes in LDS, added to acc in block order.
template <int TYPE, int R>
__device__ __forceinline__ void dot_step(const WSrc & s, int g, int c, const WStep<TYPE, R> & b, const int4 * lc,
                                         const float2 * lm, float (&acc)[R], int lane) {
    constexpr int CV = WStep<TYPE, R>::CV;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int blk = 128 * c + lane + 64 * i;
        if (blk >= s.nb) break;
        const int4 ca = lc[2 * blk], cb = lc[2 * blk + 1];
        const float2 cm = lm[blk];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int sdot;
            if constexpr (TYPE == T_Q4_0) sdot = dot_blk_q4_0(b.w[i][r][0], ca, cb, __float_as_int(cm.y));
            else sdot = dot_blk_q8_0(b.w[i][r][0], b.w[i][r][CV - 1], ca, cb);
            const int row = min(g * R + r, s.N - 1);
            const uint32_t sh = (uint32_t) (((lane ^ (row & s.nb)) & 1) << 4);
            acc[r] += ((float) sdot * h2f((uint16_t) (b.d[i][r] >> sh))) * cm.x;
        }
    }
}

// The wavefront's steps of one projection: groups g0, g0 + nw, ..., each in nchunk steps. On
// entry A holds step 0 when pre >= 1 and B step 1 when pre == 2 (loaded before the barrier that
// precedes this phase); the others are loaded here. Loads run two steps ahead. epi(g, v) gets
// each group's R row sums.
template <int TYPE, int R, class Epi>
__device__ __forceinline__ void run_steps(const WSrc & s, int g0, int nw, WStep<TYPE, R> & A, WStep<TYPE, R> & B,
                                          int pre, const int4 * lc, const float2 * lm, int lane, Epi && epi) {
    const int C = s.nchunk;
    const int mine = g0 < s.ng ? (s.ng - g0 + nw - 1) / nw : 0;
    const int S = mine * C;
    // A step past the wavefront's last zeroes the buffer instead of loading (so no buffer keeps an
    // older value alive, and no vector memory instruction is issued: with the CU's memory queue
    // full, even a load that reads nothing waits to issue).
    auto at = [&](int st, WStep<TYPE, R> & buf) {
        if (st < S) load_step<TYPE, R>(s, g0 + (st / C) * nw, st % C, buf, lane);
        else zero(buf);
    };
    if (pre < 1) at(0, A);
    if (pre < 2) at(1, B);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    auto step = [&](int st, const WStep<TYPE, R> & buf) {
        const int g = g0 + (st / C) * nw, c = st % C;
        dot_step<TYPE, R>(s, g, c, buf, lc, lm, acc, lane);
        if (c == C - 1) {
            float v[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                v[r] = wave_sum(acc[r]);
                acc[r] = 0.0f;
            }
            epi(g, v);
        }
    };
    for (int st = 0; st < S; st += 2) {
        step(st, A);
        at(st + 2, A);
        if (st + 1 >= S) break;
        step(st + 1, B);
        at(st + 3, B);
    }
}

// Steps 0 (and 1 when n == 2) of a wavefront's list into A (and B); live = false: zeros. When
// `now` is false the registers are only zeroed (a wavefront that loads its first steps in the
// phase itself): every buffer is then defined on every path, and none keeps an older value alive.
template <int TYPE, int R>
__device__ __forceinline__ void preload(const WSrc & s, int g0, int nw, int n, bool live, WStep<TYPE, R> & A,
                                        WStep<TYPE, R> & B, int lane, bool now = true) {
    if (!now) {
        zero(A);
        if (n > 1) zero(B);
        return;
    }
    const int C = s.nchunk;
    load_step<TYPE, R>(s, live ? g0 : s.ng, 0, A, lane);
    if (n > 1) load_step<TYPE, R>(s, live ? (C > 1 ? g0 : g0 + nw) : s.ng, C > 1 ? 1 : 0, B, lane);
}

// The lane index as a value the compiler cannot see through, taken afresh in every phase: the
// per-lane addresses of a phase's loads are then computed in the phase instead of being hoisted
// out of the layer loop (where, live across all of it, they would spill).
__device__ __forceinline__ int opaque_lane() {
    int l = (int) (threadIdx.x & 63);
    asm volatile("" : "+v"(l));
    return l;
}
__device__ __forceinline__ int opaque_tid() {
    int t = (int) threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// ------------------------------------------------------------------------ prologues

struct LdsAct {
    int4 * lc;
    float2 * lm;
    double * red;
    unsigned * flag;  // [0]: norm partials, [1]: codes; counts only grow within a launch
};

// Q8_0 codes of x (K values; rms_norm(x) * nw first when NORM) into LDS by the first pro_waves
// wavefronts (thread t: half blocks t, t + 64 XW, ...). NORM: the x waves of the row GEMV's norm
// prologue (4, or 8 past K = 8192), so the sum of squares is added in the same order; without the
// norm every block is converted on its own, by up to 8 wavefronts. Counts flag[1] (and flag[0])
// up by the x waves; the caller waits for its count + pro_waves.
__host__ __device__ inline int pro_waves(bool norm, int K) {
    const int xwmax = !norm || (K + 2047) / 2048 > 4 ? 8 : 4;
    return xwmax < (K + 1023) / 1024 ? xwmax : (K + 1023) / 1024;
}
// Workgroup barrier with no memory wait: orders the wavefronts' instruction issue only.
__device__ __forceinline__ void issue_sync() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// The x waves issue their activation (and norm weight) loads, then every wavefront calls
// mid(is_x_wave) - which meets the others (issue_sync) so the activation row is ahead of the CU's
// weight loads in its memory queue, and lets the other wavefronts issue their first weight steps -
// then the x waves convert. A CU's vector memory requests queue in issue order: loads issued
// behind the weight stream would wait for it.
template <bool NORM, int RMAX, class Mid>
__device__ __forceinline__ void pro_quant(__amdgpu_buffer_rsrc_t rx, const float * nw, int K, float eps,
                                          const LdsAct & L, unsigned base0, int tid, Mid && mid) {
    // RMAX: rounds of 16 values per x thread, (K + 1024 XW - 1) / (1024 XW) at most
    const int XW = pro_waves(NORM, K);
    const int wave = tid >> 6, lane = tid & 63;
    const bool xw = wave < XW;
    const int rounds = (K + XW * 1024 - 1) / (XW * 1024);
    const int t = tid;
    float4 xv[RMAX][4];
    if (xw) {
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            const int e = min((t + r * XW * 64) * 16, K - 16);
#pragma unroll
            for (int c = 0; c < 4; c++)
                xv[r][c] = r < rounds ? ld4(rx, (uint32_t) (e + 4 * c) * 4u) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    mid(xw);
    if (!xw) return;
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
    if constexpr (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int r = 0; r < RMAX; r++)
#pragma unroll
            for (int j = 0; j < 16; j++) ss += (double) (v[r][j] * v[r][j]);
        ss = wave_sum_d(ss);
        if (lane == 0) {
            L.red[wave] = ss;
            lds_signal(&L.flag[0]);
        }
        lds_wait(&L.flag[0], base0 + XW);
        double tot = 0.0;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (i < XW) tot += L.red[i];
        const float scale = 1.0f / sqrtf((float) (tot / (double) K) + eps);
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            if (r >= rounds) continue;
            const int e = min((t + r * XW * 64) * 16, K - 16);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 w = *reinterpret_cast<const float4 *>(nw + e + 4 * c);
                v[r][4 * c] = (v[r][4 * c] * scale) * w.x;
                v[r][4 * c + 1] = (v[r][4 * c + 1] * scale) * w.y;
                v[r][4 * c + 2] = (v[r][4 * c + 2] * scale) * w.z;
                v[r][4 * c + 3] = (v[r][4 * c + 3] * scale) * w.w;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RMAX; r++) {
        const int hb = t + r * XW * 64;
        if (r < rounds && hb * 16 < K)
            q8_half_block_store(v[r], reinterpret_cast<int8_t *>(L.lc) + (hb / 2) * 32, L.lm + hb / 2, hb & 1);
    }
    if (lane == 0) lds_signal(&L.flag[1]);
}

// Q8_0 codes of the merged attention row (H heads of D, split partials) into LDS, by all 16
// wavefronts (thread t: values 4t .. 4t + 3, K = H D <= 4096): sum_i e^(m_i - M) o_i /
// sum_i e^(m_i - M) l_i in split order, splits with m_i = -inf left out, 0 if none.
template <int MS, class Mid>
__device__ __forceinline__ void pro_merge(__amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml, int nsplit, int D,
                                          int K, const LdsAct & L, int tid, Mid && mid) {
    const int e = tid * 4;
    const bool in = e < K;
    const int h = e / D;
    float2 mlv[MS];
    float4 pov[MS];
#pragma unroll
    for (int j = 0; j < MS; j++) {
        if (in && j < nsplit) {
            mlv[j] = ld2(rml, (uint32_t) (h * nsplit + j) * 8u);
            pov[j] = ld4(ro, (uint32_t) ((h * nsplit + j) * D + e % D) * 4u);
        } else {
            mlv[j] = make_float2(-INFINITY, 0.0f);
            pov[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    mid();
    if (in) {
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < MS; j++) M = fmaxf(M, mlv[j].x);
        float Lsum = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        if (M != -INFINITY) {
#pragma unroll
            for (int j = 0; j < MS; j++) {
                if (mlv[j].x == -INFINITY) continue;
                const float wj = __expf(mlv[j].x - M);
                Lsum += wj * mlv[j].y;
                o.x += wj * pov[j].x;
                o.y += wj * pov[j].y;
                o.z += wj * pov[j].z;
                o.w += wj * pov[j].w;
            }
        }
        o.x = Lsum == 0.0f ? 0.0f : o.x / Lsum;
        o.y = Lsum == 0.0f ? 0.0f : o.y / Lsum;
        o.z = Lsum == 0.0f ? 0.0f : o.z / Lsum;
        o.w = Lsum == 0.0f ? 0.0f : o.w / Lsum;
        q8_block_store(o, reinterpret_cast<int8_t *>(L.lc) + (e & ~31), L.lm + e / 32, (e / 4) & 7);
    }
    if ((tid & 63) == 0) lds_signal(&L.flag[1]);
}

// ------------------------------------------------------------------------ attention

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float half_at(const uint4 & r, int c) {
    const uint32_t w = c < 2 ? r.x : c < 4 ? r.y : c < 6 ? r.z : r.w;
    return h2f((uint16_t) (c & 1 ? w >> 16 : w & 0xffff));
}
__device__ __forceinline__ half2_t as_h2(uint32_t u) {
    half2_t h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

// One (split, query head) item of the decode attention, k_attn_lanes<D, 1, 16, false>'s
// arithmetic: 16 wavefronts, D/8 lanes per key, load batches of 4 steps, online softmax per lane
// group, lane groups then wavefronts merged, the split's (max, exp-sum, unnormalized output)
// stored to the partials.
template <int D>
__device__ __forceinline__ void attn_item(int split, int h, int hk, __amdgpu_buffer_rsrc_t rq, const uint16_t * kc,
                                          const uint16_t * vc, int64_t ctx, float scale, int n_kv, int chunk,
                                          int nsplit, __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml,
                                          float (*so)[D], float2 * sml, int tid) {
    constexpr int NW = kWaves, LPK = D / 8, KPW = 64 / LPK, NB = 4;
    const int wave = tid >> 6, lane = tid & 63;
    const int sub = lane % LPK, slot = lane / LPK;
    const int j0 = split * chunk;
    const int per_wave = (chunk + NW - 1) / NW;
    const int w0 = min(chunk, wave * per_wave), w1 = min(chunk, w0 + per_wave);
    const int len = max(0, min(n_kv - j0, chunk));
    const int kv_rows = (int) ctx;

    const float4 q0 = ld4(rq, (uint32_t) (h * D + 8 * sub) * 4u);
    const float4 q1 = ld4(rq, (uint32_t) (h * D + 8 * sub + 4) * 4u);
    const uint16_t * kb = kc + (int64_t) hk * ctx * D + 8 * sub;
    const uint16_t * vb = vc + (int64_t) hk * ctx * D + 8 * sub;
    uint4 kr[NB], vr[NB];
    auto load = [&](int base) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int64_t row = min(j0 + base + b * KPW + slot, kv_rows - 1);
            kr[b] = *reinterpret_cast<const uint4 *>(kb + row * D);
            vr[b] = *reinterpret_cast<const uint4 *>(vb + row * D);
        }
    };
    if (w0 < w1) load(w0);
    __builtin_amdgcn_sched_barrier(0);
    half2_t qh[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float4 f = c < 2 ? q0 : q1;
        half2_t t;
        t.x = (_Float16) ((c & 1) ? f.z : f.x);
        t.y = (_Float16) ((c & 1) ? f.w : f.y);
        qh[c] = t;
    }
    float m = -INFINITY, l = 0.0f, acc[8];
#pragma unroll
    for (int c = 0; c < 8; c++) acc[c] = 0.0f;
    for (int base = w0; base < w1; base += NB * KPW) {
        if (base != w0) load(base);
        __builtin_amdgcn_sched_barrier(0);
        float vf[NB][8];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int c = 0; c < 8; c++) vf[b][c] = half_at(vr[b], c);
        float sc[NB];
        float bm = -INFINITY;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float a = 0.0f;
            a = __builtin_amdgcn_fdot2(as_h2(kr[b].x), qh[0], a, false);
            a = __builtin_amdgcn_fdot2(as_h2(kr[b].y), qh[1], a, false);
            a = __builtin_amdgcn_fdot2(as_h2(kr[b].z), qh[2], a, false);
            a = __builtin_amdgcn_fdot2(as_h2(kr[b].w), qh[3], a, false);
            a = group_reduce<LPK, float, op_add<float>>(a);
            const int jj = base + b * KPW + slot;
            sc[b] = jj < w1 && jj < len ? a * scale : -INFINITY;
            bm = fmaxf(bm, sc[b]);
        }
        const float mn = fmaxf(m, bm);
        if (mn == -INFINITY) continue;
        const float f = m == -INFINITY ? 0.0f : __expf(m - mn);
        float p[NB];
        float ps = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            p[b] = sc[b] == -INFINITY ? 0.0f : __expf(sc[b] - mn);
            ps += p[b];
        }
        l = l * f + ps;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            float t = acc[c] * f;
#pragma unroll
            for (int b = 0; b < NB; b++) t += p[b] * vf[b][c];
            acc[c] = t;
        }
        m = mn;
    }
    auto slots = [&](float v, auto f) {
        if constexpr (LPK == 8) v = f(v, lane_xor8(v));
        v = row_pair<16>(v, f);
        return row_pair<32>(v, f);
    };
    auto fmax2 = [](float a, float b) { return fmaxf(a, b); };
    auto add2 = [](float a, float b) { return a + b; };
    {
        const float M = slots(m, fmax2);
        const float f = m == -INFINITY ? 0.0f : __expf(m - M);
        l = slots(l * f, add2);
#pragma unroll
        for (int c = 0; c < 8; c++) acc[c] = slots(acc[c] * f, add2);
        m = M;
    }
    if (slot == 0) {
#pragma unroll
        for (int c = 0; c < 8; c++) so[wave][8 * sub + c] = acc[c];
    }
    if (lane == 0) sml[wave] = make_float2(m, l);
    wg_sync();
    const int i = tid;
    if (i < D) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sml[w].x);
        float L = 0.0f, o = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float2 ml = sml[w];
                if (ml.x == -INFINITY) continue;
                const float f = __expf(ml.x - M);
                L += f * ml.y;
                o += f * so[w][i];
            }
        }
        st1_co(ro, (uint32_t) ((h * nsplit + split) * D + i) * 4u, o);
        if (i == 0) {
            st1_co(rml, (uint32_t) (h * nsplit + split) * 8u, M);
            st1_co(rml, (uint32_t) (h * nsplit + split) * 8u + 4u, L);
        }
    }
    wg_sync();  // so / sml are reused by the next item
}

}  // namespace

// ---------------------------------------------------------------------------- kernel

namespace {

// RE: rounds of the rms_norm prologue (1: n_embd <= 4096 over its 4 x waves, 2: up to 8192);
// MS: attention splits held in registers by the merge (4 or 8).
template <int TYPE, int D, int RE, int MS>
__global__ __launch_bounds__(kThreads, 1) void k_decode_step(const StepArgs a) {
    __shared__ int4 lc[kMaxK / 16];
    __shared__ float2 lm[kMaxK / 32];
    __shared__ double red[8];
    __shared__ unsigned s_flag[2];
    __shared__ float so[kWaves][D];
    __shared__ float2 sml[kWaves];
    if (threadIdx.x == 0) {
        s_flag[0] = 0u;
        s_flag[1] = 0u;
    }
    wg_sync();
    const LdsAct L{lc, lm, red, s_flag};
    unsigned t_norm = 0, t_codes = 0;  // LDS counts reached so far
    unsigned nbar = 0;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = gridDim.x * kWaves, g0 = blockIdx.x * kWaves + wave;
    const int H = a.H, Hkv = a.Hkv, G = H / Hkv, half = D / 2;
    const int nqk = (H + Hkv) * half;
    const int p_tok = *a.pos, n_kv = *a.n_kv;
    const int E = a.n_embd, F = a.n_ff, AD = H * D;
    const uint32_t qkv_rows = (uint32_t) (H + 2 * Hkv) * D;
    // x slot k (k = 2 l: layer l's input, 2 l + 1: after its attention): the caller's row for the
    // first and last, the ring between
    auto xslot = [&](int k) {
        float * p = k == 0 || k == 2 * a.n_layer ? a.x : a.x_ring + (size_t) (k - 1) * step_ring_stride(E);
        return rsrc(p, (uint32_t) E * 4u);
    };
    const bool tr = a.trace != nullptr && *a.trace_on != 0u;
    const int n_ev = step_trace_events(a.n_layer);
    auto stamp = [&](int e) {
        if (tr && threadIdx.x == 0) a.trace[(size_t) blockIdx.x * n_ev + e] = __builtin_amdgcn_s_memrealtime();
    };
    auto stamp_ptr = [&](int e) { return tr ? a.trace + (size_t) blockIdx.x * n_ev + e : nullptr; };
    stamp(0);
    auto barrier = [&] {
        stamp(3 * (int) nbar + 1);
        bar_arrive(a.bar, nbar + 1, stamp_ptr(3 * (int) nbar + 2));
        ++nbar;
        bar_wait(a.bar, a.err, nbar);
        stamp(3 * (int) nbar);
    };
    const int xw_norm = pro_waves(true, E), xw_plain = pro_waves(false, F);
    // Attention items (split, query head) go to workgroups 0 .. att_wgs - 1; the output projection
    // runs on the others when they have a wavefront for each of its row groups.
    const int items = a.nsplit * H;
    const int att_wgs = min(items, (int) gridDim.x);
    const int o_ng = (E + 1) / 2;
    const int o_wg0 = ((int) gridDim.x - att_wgs) * kWaves >= o_ng ? att_wgs : 0;
    const bool o_here = (int) blockIdx.x >= o_wg0;
    const int o_g0 = ((int) blockIdx.x - o_wg0) * kWaves + wave, o_nw = ((int) gridDim.x - o_wg0) * kWaves;

    for (int l = 0; l < a.n_layer; l++) {
        const StepLayer & Ly = a.layers[l];
        const __amdgpu_buffer_rsrc_t rk = rsrc(Ly.kc, (uint32_t) (Hkv * a.ctx * D) * 2u),
                                     rv = rsrc(Ly.vc, (uint32_t) (Hkv * a.ctx * D) * 2u);
        const __amdgpu_buffer_rsrc_t rx = xslot(2 * l), rxm = xslot(2 * l + 1), rxo = xslot(2 * l + 2),
                                     rq = rsrc(a.q + (size_t) l * step_ring_stride(AD), (uint32_t) AD * 4u),
                                     rh = rsrc(a.h + (size_t) l * step_ring_stride(F), (uint32_t) F * 4u),
                                     ro = rsrc(a.part_o + (size_t) l * step_ring_stride(AD * a.nsplit),
                                               (uint32_t) (AD * a.nsplit) * 4u),
                                     rml = rsrc(a.part_ml + (size_t) l * step_ring_stride(2 * H * a.nsplit) / 2,
                                                (uint32_t) (H * a.nsplit) * 8u);
        // ---- QKV: rms_norm prologue, rope + K / V cache epilogue
        {
            const WSrc s = wsrc<TYPE>(Ly.qkv_qs, Ly.qkv_d, (int) qkv_rows, E / QK, 2);
            WStep<TYPE, 2> A, B;
            pro_quant<true, RE>(rx, Ly.attn_norm, E, a.eps, L, t_norm, opaque_tid(), [&](bool xw) {
                issue_sync();
                preload<TYPE, 2>(s, g0, nw, 2, true, A, B, opaque_lane(), !xw);
            });
            t_norm += xw_norm;
            t_codes += xw_norm;
            lds_wait(&s_flag[1], t_codes);
            run_steps<TYPE, 2>(s, g0, nw, A, B, wave < xw_norm ? 0 : 2, lc, lm, opaque_lane(), [&](int g, const float (&v)[2]) {
                if (lane != 0 || p_tok < 0 || p_tok >= a.ctx) return;
                if (g < nqk) {
                    const int hh = g / half, i = g % half;
                    const float2 cs = a.rope_cs[i];
                    const float y0 = v[0] * cs.x - v[1] * cs.y, y1 = v[0] * cs.y + v[1] * cs.x;
                    if (hh < H) {
                        st1_co(rq, (uint32_t) (hh * D + i) * 4u, y0);
                        st1_co(rq, (uint32_t) (hh * D + i + half) * 4u, y1);
                    } else {
                        const uint32_t row = (uint32_t) (((int64_t) (hh - H) * a.ctx + p_tok) * D);
                        st_u16_co(rk, (row + i) * 2u, f2h(y0));
                        st_u16_co(rk, (row + i + half) * 2u, f2h(y1));
                    }
                } else if (g < (int) qkv_rows / 2) {
                    const int e = 2 * (g - nqk);
                    const int hv = e / D, dd = e % D;
                    const uint32_t pair = f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
                    st_u32_co(rv, (uint32_t) (((int64_t) hv * a.ctx + p_tok) * D + dd) * 2u, pair);
                }
            });
            barrier();
        }
        // ---- attention
        {
            for (int it = blockIdx.x; it < items; it += gridDim.x) {
                const int split = it % a.nsplit, hq = it / a.nsplit;
                attn_item<D>(split, hq, hq / G, rq, Ly.kc, Ly.vc, a.ctx, a.scale, n_kv, a.chunk, a.nsplit, ro, rml,
                             so, sml, opaque_tid());
            }
            barrier();
        }
        // ---- O: merge prologue, residual epilogue
        if (o_here) {
            const WSrc s = wsrc<TYPE>(Ly.o_qs, Ly.o_d, E, AD / QK, 2);
            WStep<TYPE, 2> A, B;
            float res = 0.0f;  // x of row 2 o_g0 + lane (lanes 0, 1)
            if (lane < 2 && 2 * o_g0 + lane < E) res = ld1(rx, (uint32_t) (2 * o_g0 + lane) * 4u);
            pro_merge<MS>(ro, rml, a.nsplit, D, AD, L, opaque_tid(), [&] {
                issue_sync();
                preload<TYPE, 2>(s, o_g0, o_nw, 2, true, A, B, opaque_lane());
            });
            t_codes += kWaves;
            lds_wait(&s_flag[1], t_codes);
            run_steps<TYPE, 2>(s, o_g0, o_nw, A, B, 2, lc, lm, opaque_lane(), [&](int g, const float (&v)[2]) {
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int row = g * 2 + r;
                    if (lane == r && row < E) {
                        const float x0 = g == o_g0 ? res : ld1(rx, (uint32_t) row * 4u);
                        st1_co(rxm, (uint32_t) row * 4u, v[r] + x0);
                    }
                }
            });
        }
        barrier();
        // ---- gate / up: rms_norm prologue, swiglu epilogue
        {
            const WSrc s = wsrc<TYPE>(Ly.gu_qs, Ly.gu_d, 2 * F, E / QK, 2);
            WStep<TYPE, 2> A, B;
            pro_quant<true, RE>(rxm, Ly.ffn_norm, E, a.eps, L, t_norm, opaque_tid(), [&](bool xw) {
                issue_sync();
                preload<TYPE, 2>(s, g0, nw, 2, true, A, B, opaque_lane(), !xw);
            });
            t_norm += xw_norm;
            t_codes += xw_norm;
            lds_wait(&s_flag[1], t_codes);
            run_steps<TYPE, 2>(s, g0, nw, A, B, wave < xw_norm ? 0 : 2, lc, lm, opaque_lane(), [&](int g, const float (&v)[2]) {
                if (lane == 0 && g < F) st1_co(rh, (uint32_t) g * 4u, v[0] / (1.0f + expf(-v[0])) * v[1]);
            });
            barrier();
        }
        // ---- down: Q8_0 prologue, residual epilogue
        {
            const WSrc s = wsrc<TYPE>(Ly.dn_qs, Ly.dn_d, E, F / QK, 1);
            WStep<TYPE, 1> A, B;
            float res = 0.0f;  // x of row g0 (lane 0)
            if (lane == 0 && g0 < E) res = ld1(rxm, (uint32_t) g0 * 4u);
            pro_quant<false, 2>(rh, nullptr, F, 0.0f, L, t_norm, opaque_tid(), [&](bool xw) {
                issue_sync();
                preload<TYPE, 1>(s, g0, nw, 2, true, A, B, opaque_lane(), !xw);
            });
            t_codes += xw_plain;
            lds_wait(&s_flag[1], t_codes);
            run_steps<TYPE, 1>(s, g0, nw, A, B, wave < xw_plain ? 0 : 2, lc, lm, opaque_lane(), [&](int g, const float (&v)[1]) {
                if (lane == 0 && g < E) st1_co(rxo, (uint32_t) g * 4u, v[0] + (g == g0 ? res : ld1(rxm, (uint32_t) g * 4u)));
            });
            barrier();
        }
    }
    stamp(n_ev - 1);
    // The last workgroup to leave clears the barrier words for the next launch (every other
    // workgroup has passed its last wait).
    bar_leave(a.bar);
}

}  // namespace

// ------------------------------------------------------------------------------ host

size_t decode_step_bar_bytes() { return kBarWords * sizeof(unsigned); }

// Whether the persistent step runs this configuration: Q4_0 / Q8_0 weights, head_dim 64 / 128,
// K of every projection a multiple of 32 and at most 16384, the attention row (H D) at most 4096
// and at most 8 splits of the lane-group plan, and one 1024-thread workgroup resident per CU.
bool decode_step_fits(int type, int n_embd, int n_ff, int H, int Hkv, int D, int nsplit) {
    return (type == T_Q4_0 || type == T_Q8_0) && (D == 64 || D == 128) && H % Hkv == 0 && n_embd % QK == 0 &&
           n_ff % QK == 0 && n_embd <= 8192 && n_ff <= kMaxK && H * D <= 4096 && (H * D) % QK == 0 &&
           nsplit >= 1 && nsplit <= kMaxSplit;
}

void launch_decode_step(int type, int D, const StepArgs & a, hipStream_t s) {
    require(decode_step_fits(type, a.n_embd, a.n_ff, a.H, a.Hkv, D, a.nsplit), "decode step: configuration not supported");
    require((int64_t) a.nsplit * a.chunk >= a.ctx, "decode step: the splits must cover the cache");
    require((uint64_t) a.Hkv * a.ctx * D * 2 < 0x80000000ull, "decode step: K / V cache of a layer of 2 GB or more");
    const unsigned grid = (unsigned) cu_count();
    const int re = a.n_embd <= 4096 ? 1 : 2, ms = a.nsplit <= 4 ? 4 : 8;
#define GCQ_DS(T, DD, RE, MS)                                                                         \
    if (type == T && D == DD && re == RE && ms == MS) {                                               \
        int occ = 0;                                                                                  \
        check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(                                       \
                      &occ, reinterpret_cast<const void *>(&k_decode_step<T, DD, RE, MS>), kThreads, 0), \
                  "decode step occupancy");                                                           \
        require(occ >= 1, "decode step: a workgroup does not fit a CU");                              \
        k_decode_step<T, DD, RE, MS><<<grid, kThreads, 0, s>>>(a);                                    \
        check_launch("decode step");                                                                  \
        return;                                                                                       \
    }
#define GCQ_DS2(T, DD) GCQ_DS(T, DD, 1, 4) GCQ_DS(T, DD, 1, 8) GCQ_DS(T, DD, 2, 4) GCQ_DS(T, DD, 2, 8)
    GCQ_DS2(T_Q4_0, 64) GCQ_DS2(T_Q4_0, 128) GCQ_DS2(T_Q8_0, 64) GCQ_DS2(T_Q8_0, 128)
#undef GCQ_DS2
#undef GCQ_DS
    fail("decode step: configuration not supported");
}

}  // namespace gcq
