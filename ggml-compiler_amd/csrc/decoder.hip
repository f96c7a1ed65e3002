// decoder.hip - fused kernels of a Llama-style decoder step, each one launch where the ggml graph
// the reference builds for the same step (runtime/src/ops.cpp op table, node order of
// ggml_compiler/llm.py's causal_lm at O3: rms_norm, mul, mul_mat, rope, set_rows, flash_attn,
// swiglu, add) has two to four nodes:
//
//  rmsnorm_q8   ggml_rms_norm + ggml_mul (norm weight) + the Q8_0 conversion the next mul_mat
//               makes of its src1. The f32 values are those of k_rms_norm, and the codes those of
//               k_act_q8_0 on them, bit for bit.
//  rope_kv      ggml_rope_ext (NEOX) on the q and k heads of a fused QKV row, q in place, and the
//               ggml_set_rows of the roped k and of v into an f16 KV cache.
//  swiglu_q8    ggml_swiglu_split + the Q8_0 conversion of the down projection's src1.
//  merge_q8     the split-K attention merge + the Q8_0 conversion of the output projection's src1.
//  causal_mask  the additive f16 mask of ggml_compiler/llm.py:355-358 for a prompt chunk.
//  step_end     ggml_argmax of the logits plus the generate loop's bookkeeping
//               (runtime/src/ggml_compiler_rt.cpp:402-439): the next token, position and KV length.
#include "gcq_common.h"

#include <algorithm>

namespace gcq {

constexpr int kStepEndBlocks = 256;

// Decoder-step state on the device, read by the captured decode graph.
struct StepState {
    int pos;    // position of the token being decoded
    int n_kv;   // keys visible to it (pos + 1)
    int token;  // token fed at this step
    int step;   // tokens generated so far
};

// One 256-thread block per row; n a multiple of 32.
__global__ __launch_bounds__(256) void k_rmsnorm_q8(const float * __restrict__ x, int64_t ldx,
                                                    const float * __restrict__ w, float eps, int n,
                                                    int8_t * __restrict__ codes, float2 * __restrict__ meta) {
    const int row = blockIdx.x;
    rmsnorm_q8_row(x + row * ldx, n, w, eps, codes + (int64_t) row * n, meta + (int64_t) row * (n / 32));
}

// silu(g) * u over rows of n (g, u at row strides), quantized to Q8_0.
__global__ void k_swiglu_q8(const float * __restrict__ g, const float * __restrict__ u, int64_t ld, int n, int rows,
                            int8_t * __restrict__ codes, float2 * __restrict__ meta) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int per = n / 4;
    if (t >= (int64_t) rows * per) return;  // whole 8-lane groups
    const int row = (int) (t / per);
    const int e = (int) (t % per) * 4;
    const float4 a = *reinterpret_cast<const float4 *>(g + row * ld + e);
    const float4 b = *reinterpret_cast<const float4 *>(u + row * ld + e);
    float4 v;
    v.x = a.x / (1.0f + expf(-a.x)) * b.x;
    v.y = a.y / (1.0f + expf(-a.y)) * b.y;
    v.z = a.z / (1.0f + expf(-a.z)) * b.z;
    v.w = a.w / (1.0f + expf(-a.w)) * b.w;
    q8_block_store(v, codes + (int64_t) row * n + (e & ~31), meta + (int64_t) row * (n / 32) + e / 32, (e / 4) & 7);
}

// NEOX rope (n_dims = D) of the H q heads and Hkv k heads of each fused QKV row [q | k | v], q in
// place, roped k and v written as f16 into the cache rows pos[s]: cache [2*Hkv][ctx][D], K heads
// first. One thread per rotation pair (q and k) or per value pair (v).
__global__ void k_rope_kv(float * __restrict__ qkv, int64_t ld, const int32_t * __restrict__ pos, int S, int H,
                          int Hkv, int D, float theta_scale, uint16_t * __restrict__ cache, int64_t ctx) {
    const int half = D / 2;
    const int per_s = (H + 2 * Hkv) * half;
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) S * per_s) return;
    const int s = (int) (t / per_s);
    const int r = (int) (t % per_s);
    const int h = r / half, i = r % half;
    const int p = pos[s];
    if (p < 0 || p >= ctx) return;
    float * row = qkv + s * ld;
    if (h < H + Hkv) {
        float theta = (float) p;
        for (int k = 0; k < i; k++) theta *= theta_scale;
        const float c = cosf(theta), sn = sinf(theta);
        float * xr = row + h * D;
        const float x0 = xr[i], x1 = xr[i + half];
        const float y0 = x0 * c - x1 * sn, y1 = x0 * sn + x1 * c;
        if (h < H) {
            xr[i] = y0;
            xr[i + half] = y1;
        } else {
            uint16_t * kr = cache + ((int64_t) (h - H) * ctx + p) * D;
            kr[i] = f2h(y0);
            kr[i + half] = f2h(y1);
        }
    } else {  // v head hv: values 2i, 2i+1
        const int hv = h - H - Hkv;
        const float * vr = row + (H + Hkv + hv) * D;
        uint16_t * dr = cache + ((int64_t) (Hkv + hv) * ctx + p) * D;
        const uint32_t pair = f2h(vr[2 * i]) | ((uint32_t) f2h(vr[2 * i + 1]) << 16);
        *reinterpret_cast<uint32_t *>(dr + 2 * i) = pair;
    }
}

// Attention merge of nsplit partials for each (query row, head), then the Q8_0 conversion of the
// [Sq][H*D] result (each block of 32 dims is 8 lanes x 4 dims). D threads x 1 head per block.
template <int D>
__global__ __launch_bounds__(D / 4) void k_merge_q8(const float * __restrict__ part_o, const float2 * __restrict__ part_ml,
                                                    int nsplit, int H, float * __restrict__ out,
                                                    int8_t * __restrict__ codes, float2 * __restrict__ meta) {
    const int64_t sh = blockIdx.x;  // s * H + h
    const int d0 = threadIdx.x * 4;
    const float2 * ml = part_ml + sh * nsplit;
    float M = -INFINITY;
    for (int i = 0; i < nsplit; i++) M = fmaxf(M, ml[i].x);
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (M != -INFINITY) {
        for (int i = 0; i < nsplit; i++) {
            if (ml[i].x == -INFINITY) continue;
            const float w = __expf(ml[i].x - M);
            L += w * ml[i].y;
            const float4 p = *reinterpret_cast<const float4 *>(part_o + (sh * nsplit + i) * D + d0);
            o.x += w * p.x;
            o.y += w * p.y;
            o.z += w * p.z;
            o.w += w * p.w;
        }
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    o.x = L == 0.0f ? 0.0f : o.x / L;
    o.y = L == 0.0f ? 0.0f : o.y / L;
    o.z = L == 0.0f ? 0.0f : o.z / L;
    o.w = L == 0.0f ? 0.0f : o.w / L;
    (void) inv;
    if (out) *reinterpret_cast<float4 *>(out + sh * D + d0) = o;
    const int64_t s = sh / H;
    const int h = (int) (sh % H);
    const int n = H * D;
    const int e = h * D + d0;
    q8_block_store(o, codes + s * n + (e & ~31), meta + s * (n / 32) + e / 32, (d0 / 4) & 7);
}

// The decode step's first launch: ggml_get_rows of the token's embedding row into x, and the NEOX
// rotation table of the token's position, cs[i] = (cos theta_i, sin theta_i) for i < half with
// theta_i = pos * theta_scale^i by repeated f32 multiplication (k_rope_kv's arithmetic), which
// every layer's QKV projection applies in its epilogue.
__global__ void k_embed_rope(int type, const uint8_t * __restrict__ tab, int64_t nrows, int D,
                             const int32_t * __restrict__ idx, float * __restrict__ x, const int32_t * __restrict__ pos,
                             int half, float theta_scale, float2 * __restrict__ cs) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < D) x[t] = table_value(type, tab, nrows, D, idx[0], t);
    if (t < half) {
        float theta = (float) pos[0];
        for (int k = 0; k < t; k++) theta *= theta_scale;
        cs[t] = make_float2(cosf(theta), sinf(theta));
    }
}

// dst[r][map[c]] = src[r][c] for S rows of n columns: a mul_mat result whose weight rows were
// packed in another order, back in the weight's own row order.
__global__ void k_scatter_cols(const float * __restrict__ src, int64_t lds, float * __restrict__ dst, int64_t ldd,
                               const int32_t * __restrict__ map, int S, int n) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) S * n) return;
    const int64_t r = t / n;
    const int c = (int) (t % n);
    dst[r * ldd + map[c]] = src[r * lds + c];
}

// mask[s][j] = 0 for j <= pos0 + s, -inf after (f16), j < n_kv.
__global__ void k_causal_mask(uint16_t * __restrict__ mask, int S, int n_kv, int pos0) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) S * n_kv) return;
    const int s = (int) (t / n_kv), j = (int) (t % n_kv);
    mask[t] = j <= pos0 + s ? (uint16_t) 0 : (uint16_t) 0xfc00;
}

// argmax of the logits (first index of the maximum) and the generate loop's step: record the
// token, advance position and KV length. Every workgroup reduces a kArgmaxSlice-value slice to
// (max, first index) and the last one to finish (a device counter, reset by that workgroup for
// the next launch) reduces the partials and advances the state: one launch, no wait on other
// workgroups.
__global__ __launch_bounds__(256) void k_step_end(const float * __restrict__ logits, int n, StepState * st,
                                                  int32_t * __restrict__ out_tokens, int max_out,
                                                  float2 * __restrict__ part, unsigned int * __restrict__ counter) {
    __shared__ bool last;
    __shared__ float pv[4];
    __shared__ int pi[4];
    float v;
    int idx;
    const int lo = blockIdx.x * kArgmaxSlice;
    slice_argmax(logits, lo, min(n, lo + kArgmaxSlice), (reinterpret_cast<uintptr_t>(logits) & 15) == 0, v, idx);
    if (threadIdx.x == 0) {
        part[blockIdx.x] = make_float2(v, __int_as_float(idx));
        __threadfence();
        last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    v = -INFINITY;
    idx = 0x7fffffff;
    for (int b = threadIdx.x; b < (int) gridDim.x; b += 256) {
        const float2 p = part[b];
        argmax_take(v, idx, p.x, __float_as_int(p.y));
    }
    for (int o = 32; o > 0; o >>= 1) argmax_take(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) {
        pv[threadIdx.x >> 6] = v;
        pi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) argmax_take(v, idx, pv[w], pi[w]);
        const int tok = (v == -INFINITY || idx == 0x7fffffff) ? 0 : idx;
        if (out_tokens && st->step < max_out) out_tokens[st->step] = tok;
        st->step += 1;
        st->token = tok;
        st->pos += 1;
        st->n_kv = st->pos + 1;
        *counter = 0u;
    }
}

// ------------------------------------------------------------------------------ launchers

static inline unsigned nblk(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }

void launch_rmsnorm_q8(const float * x, int64_t ldx, const float * w, float eps, int64_t rows, int64_t n, void * act,
                       hipStream_t s) {
    const ActLayout L = act_layout(T_Q4_0, rows, n);
    k_rmsnorm_q8<<<(unsigned) rows, 256, 0, s>>>(x, ldx, w, eps, (int) n, (int8_t *) act,
                                                 (float2 *) ((uint8_t *) act + L.meta));
    check_launch("rmsnorm_q8");
}

void launch_swiglu_q8(const float * g, const float * u, int64_t ld, int64_t n, int64_t rows, void * act,
                      hipStream_t s) {
    const ActLayout L = act_layout(T_Q4_0, rows, n);
    k_swiglu_q8<<<nblk(rows * n / 4, 256), 256, 0, s>>>(g, u, ld, (int) n, (int) rows, (int8_t *) act,
                                                        (float2 *) ((uint8_t *) act + L.meta));
    check_launch("swiglu_q8");
}

void launch_rope_kv(float * qkv, int64_t ld, const int32_t * pos, int S, int H, int Hkv, int D, float base,
                    void * cache, int64_t ctx, hipStream_t s) {
    const float theta_scale = powf(base, -2.0f / (float) D);
    const int64_t n = (int64_t) S * (H + 2 * Hkv) * (D / 2);
    k_rope_kv<<<nblk(n, 256), 256, 0, s>>>(qkv, ld, pos, S, H, Hkv, D, theta_scale, (uint16_t *) cache, ctx);
    check_launch("rope_kv");
}

void launch_merge_q8(const float * part_o, const float2 * part_ml, int nsplit, int Sq, int H, int D, float * out,
                     void * act, hipStream_t s) {
    const ActLayout L = act_layout(T_Q4_0, Sq, (int64_t) H * D);
    int8_t * codes = (int8_t *) act;
    float2 * meta = (float2 *) ((uint8_t *) act + L.meta);
    if (D == 128) k_merge_q8<128><<<(unsigned) (Sq * H), 32, 0, s>>>(part_o, part_ml, nsplit, H, out, codes, meta);
    else if (D == 64) k_merge_q8<64><<<(unsigned) (Sq * H), 16, 0, s>>>(part_o, part_ml, nsplit, H, out, codes, meta);
    else fail("merge_q8: head size must be 64 or 128");
    check_launch("merge_q8");
}

void launch_embed_rope(int type, const void * tab, int64_t nrows, int64_t D, const int32_t * idx, float * x,
                       const int32_t * pos, int head_dim, float base, void * cs, hipStream_t s) {
    const int half = head_dim / 2;
    const float theta_scale = powf(base, -2.0f / (float) head_dim);
    const int64_t n = std::max<int64_t>(D, half);
    k_embed_rope<<<nblk(n, 256), 256, 0, s>>>(type, (const uint8_t *) tab, nrows, (int) D, idx, x, pos, half,
                                             theta_scale, (float2 *) cs);
    check_launch("embed_rope");
}

void launch_scatter_cols(const float * src, int64_t lds, float * dst, int64_t ldd, const int32_t * map, int S, int n,
                         hipStream_t s) {
    k_scatter_cols<<<nblk((int64_t) S * n, 256), 256, 0, s>>>(src, lds, dst, ldd, map, S, n);
    check_launch("scatter_cols");
}

void launch_causal_mask(void * mask, int S, int n_kv, int pos0, hipStream_t s) {
    k_causal_mask<<<nblk((int64_t) S * n_kv, 256), 256, 0, s>>>((uint16_t *) mask, S, n_kv, pos0);
    check_launch("causal_mask");
}

// part: kStepEndBlocks float2, counter: one zeroed unsigned int (left zeroed after each launch);
// n <= kStepEndBlocks * kArgmaxSlice.
void launch_step_end(const float * logits, int n, void * state, int32_t * out_tokens, int max_out, void * part,
                     void * counter, hipStream_t s) {
    require(n >= 1 && n <= kStepEndBlocks * kArgmaxSlice, "step end: vocabulary of 1 to 524288 logits");
    k_step_end<<<nblk(n, kArgmaxSlice), 256, 0, s>>>(logits, n, (StepState *) state, out_tokens, max_out, (float2 *) part,
                                              (unsigned int *) counter);
    check_launch("step_end");
}

}  // namespace gcq
