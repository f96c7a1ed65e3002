// elementwise.hip - the decode step's row-wise and glue ops, and synthetic-data fills.
//
//  rms_norm  ggml_rms_norm (runtime/src/ops.cpp:144-148), optionally fused with the ggml_mul by a
//            norm weight that the graph applies next (passes/fold.py:93-114 emits the pair)
//  rope      ggml_rope_ext, NEOX mode (runtime/src/ops.cpp:277-291, mode 2 from
//            emit/gguf_runtime.py:76-78)
//  set_rows  ggml_set_rows f32 -> f16 KV-cache write (runtime/src/ops.cpp:260-275)
//  get_rows  ggml_get_rows from a Q4_0 / Q8_0 / F16 / F32 table (runtime/src/ops.cpp:302-309)
//  swiglu    ggml_swiglu_split (runtime/src/ops.cpp:251-258)
//  add, mul  ggml_add / ggml_mul with a broadcast second operand
//  argmax    ggml_argmax (runtime/src/ops.cpp:293-300)
//  cpy       ggml_cpy / ggml_cont / ggml_cast between f32 and f16 at any strides (runtime/src/ops.cpp:101,
//            :344-348)
//  scale     ggml_scale / ggml_scale_bias (runtime/src/ops.cpp:121-131)
// All are HBM- or launch-bound and move whole rows with 16-byte accesses where the shapes allow.
#include "gcq_common.h"

#include <stdexcept>

namespace gcq {

// ------------------------------------------------------------------------------ rms_norm

// One 256-thread block per row: y = x * (1/sqrt(mean(x^2) + eps)) [* w]. As ggml-cpu, each x*x
// is rounded to f32 and summed in double, and the mean rounded to f32: a Q4_0 embedding row (exact
// multiples of its scale) normalized and quantized to Q8_0 hits exact rounding ties, so the scale
// must come out bit-identical for the codes to.
__global__ __launch_bounds__(256) void k_rms_norm(const float * __restrict__ x, int64_t ldx, float * __restrict__ y,
                                                  int64_t ldy, const float * __restrict__ w, int n, float eps) {
    const float * xr = x + blockIdx.x * ldx;
    float * yr = y + blockIdx.x * ldy;
    const float scale = rms_scale(xr, n, eps);
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * 256) {  // 8 strides of loads in flight at once
        float xv[8], wv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = i0 + 256 * k;
            xv[k] = i < n ? xr[i] : 0.0f;
            wv[k] = i < n && w ? w[i] : 1.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = i0 + 256 * k;
            if (i < n) yr[i] = w ? (xv[k] * scale) * wv[k] : xv[k] * scale;
        }
    }
}

// ---------------------------------------------------------------------------------- rope

// One workgroup per (token s, block of RH heads): its first n_dims/2 threads build the rotation of
// every pair i of the token (theta as ggml's rope cache: the position multiplied by theta_scale
// once per pair, theta_scale = powf(base, -2/n_dims) computed on the host in f32 as ggml does),
// then all threads rotate the block's heads with it; dims n_dims .. D-1 pass through.
constexpr int RH = 8;
// A second tensor (x2 / out2, H2 heads, the same positions and parameters: q and k of a layer)
// takes the grid rows past the first's.
__global__ __launch_bounds__(256) void k_rope_neox(const float * __restrict__ x, int64_t sx_s, int64_t sx_h,
                                                   float * __restrict__ out, int64_t so_s, int64_t so_h,
                                                   const int32_t * __restrict__ pos, int D, int H, int S, int n_dims,
                                                   float theta_scale, float freq_scale, float attn_factor,
                                                   const float * __restrict__ ff, const float * __restrict__ x2,
                                                   int64_t sx2_s, int64_t sx2_h, float * __restrict__ out2,
                                                   int64_t so2_s, int64_t so2_h, int H2) {
    __shared__ float2 cs[128];  // n_dims / 2 <= 128
    const int half = n_dims / 2;
    const int s = blockIdx.x, yb1 = (H + RH - 1) / RH;
    if ((int) blockIdx.y >= yb1) {  // the second tensor's heads
        x = x2;
        sx_s = sx2_s;
        sx_h = sx2_h;
        out = out2;
        so_s = so2_s;
        so_h = so2_h;
        H = H2;
    }
    const int h0 = ((int) blockIdx.y < yb1 ? (int) blockIdx.y : (int) blockIdx.y - yb1) * RH;
    const int nh = min(RH, H - h0);
    if ((int) threadIdx.x < half) {
        const int i = threadIdx.x;
        float theta = (float) pos[s];
        for (int k = 0; k < i; k++) theta *= theta_scale;
        const float f = ff ? ff[i] : 1.0f;
        const float th = freq_scale * (theta / f);
        cs[i] = make_float2(cosf(th) * attn_factor, sinf(th) * attn_factor);
    }
    __syncthreads();
    const int per_row = D - half;  // pairs, then the pass-through dims
    for (int p = threadIdx.x; p < nh * per_row; p += 256) {
        const int h = h0 + p / per_row, i = p % per_row;
        const float * xr = x + s * sx_s + h * sx_h;
        float * o = out + s * so_s + h * so_h;
        if (i >= half) {
            const int d = i - half + n_dims;
            if (d < D) o[d] = xr[d];
            continue;
        }
        const float2 r = rope_pair(xr[i], xr[i + half], cs[i]);
        o[i] = r.x;
        o[i + half] = r.y;
    }
}

// The (cos, sin) pairs k_rope_neox builds for position pos[0], written out: the table the
// decode-row GEMV's rope epilogue reads (same arithmetic, so the same rotations).
__device__ __forceinline__ void rope_table_at(int i, const int32_t * __restrict__ pos, float theta_scale,
                                              float freq_scale, float attn_factor, const float * __restrict__ ff,
                                              float2 * __restrict__ cs) {
    float theta = (float) pos[0];
    for (int k = 0; k < i; k++) theta *= theta_scale;
    const float f = ff ? ff[i] : 1.0f;
    const float th = freq_scale * (theta / f);
    cs[i] = make_float2(cosf(th) * attn_factor, sinf(th) * attn_factor);
}

__global__ void k_rope_table(const int32_t * __restrict__ pos, int n_dims, float theta_scale, float freq_scale,
                             float attn_factor, const float * __restrict__ ff, float2 * __restrict__ cs) {
    const int i = threadIdx.x;
    if (i >= n_dims / 2) return;
    rope_table_at(i, pos, theta_scale, freq_scale, attn_factor, ff, cs);
}

// ------------------------------------------------------------------------------ set_rows

// dst[h][idx[j]][d] = f16(src[h][j][d]) for j < n, h < Hrows; 8 values per thread. Rows whose
// index falls outside [0, dst_rows) are not written.
__global__ void k_set_rows_f16(uint16_t * __restrict__ dst, int64_t dst_h, int64_t dst_j,
                               const float * __restrict__ src, int64_t src_h, int64_t src_j,
                               const int32_t * __restrict__ idx, int n, int D, int Hrows, int64_t dst_rows,
                               SetRowsSecond r2) {
    int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    int per = D / 8;
    const int64_t n1 = (int64_t) n * Hrows * per;
    if (t >= n1) {  // a second write of the same rows (k and v of a layer)
        t -= n1;
        dst = r2.dst;
        dst_h = r2.dst_h;
        dst_j = r2.dst_j;
        src = r2.src;
        src_h = r2.src_h;
        src_j = r2.src_j;
        D = r2.D;
        Hrows = r2.Hrows;
        dst_rows = r2.dst_rows;
        per = D / 8;
    }
    if (t >= (int64_t) n * Hrows * per) return;
    const int c = (int) (t % per);
    const int h = (int) ((t / per) % Hrows);
    const int j = (int) (t / ((int64_t) per * Hrows));
    const int64_t r = idx[j];
    if (r < 0 || r >= dst_rows) return;
    const float * sp = src + h * src_h + j * src_j + 8 * c;
    uint16_t * dp = dst + h * dst_h + r * dst_j + 8 * c;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = f2h(sp[2 * k]) | ((uint32_t) f2h(sp[2 * k + 1]) << 16);
    *reinterpret_cast<uint4 *>(dp) = make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------------------------------ get_rows

__device__ __forceinline__ void get_rows_at(int64_t t, int type, const uint8_t * __restrict__ tab, int64_t nrows_tab,
                                            int D, const int32_t * __restrict__ idx, float * __restrict__ out) {
    const int j = (int) (t / D), c = (int) (t % D);
    out[t] = table_value(type, tab, nrows_tab, D, idx[j], c);
}

__global__ void k_get_rows(int type, const uint8_t * __restrict__ tab, int64_t nrows_tab, int D,
                           const int32_t * __restrict__ idx, float * __restrict__ out, int n) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) n * D) return;
    get_rows_at(t, type, tab, nrows_tab, D, idx, out);
}

// ---------------------------------------------------------------------- swiglu, add, mul

__global__ void k_swiglu(const float * __restrict__ g, const float * __restrict__ u, float * __restrict__ y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float a = g[i];
    y[i] = a / (1.0f + expf(-a)) * u[i];
}

__global__ void k_binary(int op, const float * __restrict__ a, const float * __restrict__ b, float * __restrict__ y,
                         int64_t n, int64_t nb) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float av = a[i], bv = b[i % nb];
    y[i] = op == 0 ? av + bv : op == 1 ? av * bv : op == 2 ? av - bv : av / bv;
}

// b repeated over a along every dim (ggml_can_repeat(b, a)): element (i0, i1, i2, i3) of a meets
// element (i0 % bne0, i1 % bne1, i2 % bne2, i3 % bne3) of b. Both contiguous.
struct Bcast4 {
    int64_t ane[4], bne[4];
};

__global__ void k_binary_bcast(int op, const float * __restrict__ a, const float * __restrict__ b,
                               float * __restrict__ y, int64_t n, Bcast4 g) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t r = i, bi = 0, bstride = 1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        bi += (r % g.ane[k]) % g.bne[k] * bstride;
        r /= g.ane[k];
        bstride *= g.bne[k];
    }
    const float av = a[i], bv = b[bi];
    y[i] = op == 0 ? av + bv : op == 1 ? av * bv : op == 2 ? av - bv : av / bv;
}

// ----------------------------------------------------------------------- unary, softmax

bool unary_known(int op) {
    switch (op) {
        case UN_ABS: case UN_NEG: case UN_TANH: case UN_RELU: case UN_SIGMOID: case UN_GELU: case UN_SILU:
        case UN_EXP: case UN_GELU_ERF: case UN_SOFTPLUS: case UN_SQR: case UN_SQRT: case UN_LOG: case UN_SIN:
        case UN_COS: case UN_CLAMP:
            return true;
        default:
            return false;
    }
}

// y = f(x); the op is uniform over the launch, so the switch is one scalar branch per wave.
__global__ void k_unary(int op, const float * __restrict__ x, float * __restrict__ y, int64_t n, float lo, float hi) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    switch (op) {
        case UN_ABS: r = fabsf(v); break;
        case UN_NEG: r = -v; break;
        case UN_TANH: r = tanhf(v); break;
        case UN_RELU: r = v > 0.0f ? v : 0.0f; break;
        case UN_SIGMOID: r = 1.0f / (1.0f + expf(-v)); break;
        case UN_GELU: r = 0.5f * v * (1.0f + tanhf(0.7978845608f * v * (1.0f + 0.044715f * v * v))); break;
        case UN_SILU: r = v / (1.0f + expf(-v)); break;
        case UN_EXP: r = expf(v); break;
        case UN_GELU_ERF: r = 0.5f * v * (1.0f + erff(v * 0.70710678118f)); break;
        case UN_SOFTPLUS: r = v > 20.0f ? v : log1pf(expf(v)); break;
        case UN_SQR: r = v * v; break;
        case UN_SQRT: r = sqrtf(v); break;
        case UN_LOG: r = logf(v); break;
        case UN_SIN: r = sinf(v); break;
        case UN_CLAMP: r = fmaxf(fminf(v, hi), lo); break;
        default: r = cosf(v); break;
    }
    y[i] = r;
}

// One 256-thread block per contiguous row: the mean and then the variance of the row about it, both
// summed in double and rounded to f32 as ggml-cpu's norm, then (x - mean) / sqrt(var + eps). The
// last pass reads each element before the same thread writes it, after barriers that end the
// earlier passes, so y may alias x.
__global__ __launch_bounds__(256) void k_norm(const float * x, float * y, int n, float eps) {
    __shared__ double red[2][4];
    const float * xr = x + (int64_t) blockIdx.x * n;
    float * yr = y + (int64_t) blockIdx.x * n;
    const int w = threadIdx.x >> 6;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) s += (double) xr[i];
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[0][w] = s;
    __syncthreads();
    const float mean = (float) ((red[0][0] + red[0][1] + red[0][2] + red[0][3]) / (double) n);
    double s2 = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float dv = xr[i] - mean;
        s2 += (double) (dv * dv);
    }
    s2 = wave_sum_d(s2);
    if ((threadIdx.x & 63) == 0) red[1][w] = s2;
    __syncthreads();
    const float var = (float) ((red[1][0] + red[1][1] + red[1][2] + red[1][3]) / (double) n);
    const float sc = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < n; i += 256) yr[i] = (xr[i] - mean) * sc;
}

// Sum of each contiguous row in double, rounded to f32 (ggml_sum_rows); mean: that f32 sum divided
// by (float) n (ggml_mean: the rounded sum, then one f32 division).
__global__ __launch_bounds__(256) void k_row_sum(const float * __restrict__ x, float * __restrict__ y, int n,
                                                 int mean) {
    __shared__ double red[4];
    const float * xr = x + (int64_t) blockIdx.x * n;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) s += (double) xr[i];
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float sum = (float) (red[0] + red[1] + red[2] + red[3]);
        y[blockIdx.x] = mean ? sum / (float) n : sum;
    }
}

// One 256-thread block per row: the row maximum of x * scale + mask, then e^(v - max) written
// with its sum, then scaled by 1 / sum. Each thread reads an element before it writes the same
// element, and all reads of the first pass end at a barrier, so y may alias x. A row masked to
// -inf everywhere comes out NaN, as ggml's.
__global__ __launch_bounds__(256) void k_soft_max(const float * x, float * y, int n, int r1, int r2,
                                                  const void * __restrict__ mask, int mask_f16, int64_t mld,
                                                  int64_t ms2, int64_t ms3, int m2, int m3, float scale) {
    __shared__ float red[2][4];
    const int64_t row = blockIdx.x;
    const int64_t i1 = row % r1, i23 = row / r1, i2 = i23 % r2, i3 = i23 / r2;
    const float * xr = x + row * n;
    float * yr = y + row * n;
    const int64_t mo = i1 * mld + (i2 % m2) * ms2 + (i3 % m3) * ms3;
    auto val = [&](int i) {
        float v = xr[i] * scale;
        if (mask) v += mask_f16 ? h2f(static_cast<const uint16_t *>(mask)[mo + i]) : static_cast<const float *>(mask)[mo + i];
        return v;
    };
    const int w = threadIdx.x >> 6;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, val(i));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[0][w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float sum = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float e = expf(val(i) - mx);
        yr[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) red[1][w] = sum;
    __syncthreads();
    const float inv = 1.0f / (red[1][0] + red[1][1] + red[1][2] + red[1][3]);
    for (int i = threadIdx.x; i < n; i += 256) yr[i] *= inv;
}

// -------------------------------------------------------------------------------- argmax

// One 1024-thread block per row, 16-byte loads with 8 in flight per thread (a vocabulary row of
// 128256 logits is 500 KB: a 256-thread block walking it with one 4-byte load at a time spent
// 130 us waiting); the first index of the maximum (NaN never wins; a row of -inf / NaN gives 0,
// as ggml's forward_argmax).

__global__ __launch_bounds__(1024) void k_argmax(const float * __restrict__ x, int64_t ldx, int n,
                                                 int32_t * __restrict__ out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float * xr = x + blockIdx.x * ldx;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    const bool vec = (reinterpret_cast<uintptr_t>(xr) & 15) == 0;
    const int n4 = vec ? n / 4 : 0;
    const float4 * x4 = reinterpret_cast<const float4 *>(xr);
    for (int base = threadIdx.x; base < n4; base += 8 * 1024) {
        float4 q[8];
#pragma unroll
        for (int u = 0; u < 8; u++) q[u] = x4[min(base + u * 1024, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = base + u * 1024;
            if (e < n4) {
                argmax_take(v, idx, q[u].x, 4 * e);
                argmax_take(v, idx, q[u].y, 4 * e + 1);
                argmax_take(v, idx, q[u].z, 4 * e + 2);
                argmax_take(v, idx, q[u].w, 4 * e + 3);
            }
        }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += 1024) argmax_take(v, idx, xr[i], i);
    for (int o = 32; o > 0; o >>= 1) argmax_take(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = v;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++) argmax_take(v, idx, bv[w], bi[w]);
        out[blockIdx.x] = (v == -INFINITY || idx == 0x7fffffff) ? 0 : idx;
    }
}

// Long rows, few of them: workgroup (slice, row) reduces kArgmaxSlice values of the row to (max,
// first index) and the last of the row's workgroups to finish (a per-row device counter, which
// that workgroup resets for the next launch) picks among the row's partials - one launch whose
// workgroups all load at once (a single block per 128256-value row measured 15 us, bound by one
// CU's loads). Same result as k_argmax: the selection does not depend on the order.
__global__ __launch_bounds__(256) void k_argmax_split(const float * __restrict__ x, int64_t ldx, int n,
                                                      int32_t * __restrict__ out, float2 * __restrict__ part,
                                                      unsigned int * __restrict__ counter) {
    __shared__ bool last;
    __shared__ float pv[4];
    __shared__ int pi[4];
    const int row = blockIdx.y, slices = gridDim.x;
    const float * xr = x + row * ldx;
    const int lo = blockIdx.x * kArgmaxSlice;
    float v;
    int idx;
    slice_argmax(xr, lo, min(n, lo + kArgmaxSlice), (reinterpret_cast<uintptr_t>(xr) & 15) == 0, v, idx);
    float2 * pr = part + (int64_t) row * slices;
    if (threadIdx.x == 0) {
        pr[blockIdx.x] = make_float2(v, __int_as_float(idx));
        __threadfence();
        last = atomicAdd(counter + row, 1u) == (unsigned) slices - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    v = -INFINITY;
    idx = 0x7fffffff;
    for (int b = threadIdx.x; b < slices; b += 256) {
        const float2 p = pr[b];
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
        out[row] = (v == -INFINITY || idx == 0x7fffffff) ? 0 : idx;
        counter[row] = 0u;
    }
}

// --------------------------------------------------------------------------- synthetic data

// Same stream as the oracle's: twelve 24-bit uniforms summed (Irwin-Hall), centred, scaled by
// 2^-24 and by stddev. Integer work, an exact scaling and one rounded multiply: bit-identical.
__global__ void k_fill_normal(float * __restrict__ dst, int64_t n, uint64_t seed, uint64_t offset, float stddev) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t e = offset + (uint64_t) i;
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        const uint64_t r = rnd64(seed, 6 * e + (uint64_t) j);
        s += (int64_t) (r & 0xffffffu) + (int64_t) ((r >> 32) & 0xffffffu);
    }
    const int32_t c = (int32_t) (s - 6 * (int64_t) 0xffffff);
    dst[i] = ((float) c * (1.0f / 16777216.0f)) * stddev;
}

__global__ void k_fill_ids(int32_t * __restrict__ dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    dst[i] = (int32_t) (rnd64(seed, offset + (uint64_t) i) % (uint64_t) vocab);
}

// ----------------------------------------------------------------------------- cpy, scale

// Element i in row-major order of the logical shape: source element (shape sne, byte strides snb)
// to destination element (dne, dnb); the two shapes have the same element count. f32 / f16 either
// side, f32 -> f16 rounding to nearest even as ggml's conversion.
__device__ __forceinline__ void cpy_at(int64_t i, const uint8_t * __restrict__ src, int st, uint8_t * __restrict__ dst,
                                       int dt, const Cpy4 & g) {
    int64_t r = i, so = 0, dof = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        so += (r % g.sne[k]) * g.snb[k];
        r /= g.sne[k];
    }
    r = i;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        dof += (r % g.dne[k]) * g.dnb[k];
        r /= g.dne[k];
    }
    if (st == T_I32) {  // i32 -> i32: the bits
        *reinterpret_cast<int32_t *>(dst + dof) = *reinterpret_cast<const int32_t *>(src + so);
        return;
    }
    const float v = st == T_F32 ? *reinterpret_cast<const float *>(src + so)
                                : h2f(*reinterpret_cast<const uint16_t *>(src + so));
    if (dt == T_F32) *reinterpret_cast<float *>(dst + dof) = v;
    else *reinterpret_cast<uint16_t *>(dst + dof) = f2h(v);
}

__global__ void k_cpy(const uint8_t * __restrict__ src, int st, uint8_t * __restrict__ dst, int dt, Cpy4 g, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    cpy_at(i, src, st, dst, dt, g);
}

// ------------------------------------------------------------------------------ small jobs

// Up to three independent get_rows / cpy / rope-table jobs in one launch (a graph's first steps:
// the embedding row, the mask's cast, the rotation table). Job k takes blocks first[k] ..
// first[k + 1] - 1 and runs the same per-element code as its own kernel, so its values are the
// same. Independent: no job reads or writes what another writes (the caller checks).
__device__ __forceinline__ void small_job_at(const SmallJob & j, int64_t t) {
    if (t >= j.n) return;
    if (j.kind == SJ_GETROWS)
        get_rows_at(t, j.type, (const uint8_t *) j.src, j.rows, j.D, (const int32_t *) j.aux, (float *) j.dst);
    else if (j.kind == SJ_CPY)
        cpy_at(t, (const uint8_t *) j.src, j.type, (uint8_t *) j.dst, j.type2, j.g);
    else
        rope_table_at((int) t, (const int32_t *) j.src, j.f[0], j.f[1], j.f[2], (const float *) j.aux,
                      (float2 *) j.dst);
}

__global__ __launch_bounds__(256) void k_small_jobs(SmallJobs js) {
    const unsigned b = blockIdx.x;
    if (js.nj > 2 && b >= js.first[2]) small_job_at(js.j[2], (int64_t) (b - js.first[2]) * 256 + threadIdx.x);
    else if (js.nj > 1 && b >= js.first[1]) small_job_at(js.j[1], (int64_t) (b - js.first[1]) * 256 + threadIdx.x);
    else small_job_at(js.j[0], (int64_t) b * 256 + threadIdx.x);
}

__global__ void k_repeat(const uint8_t * __restrict__ src, float * __restrict__ dst, Cpy4 g, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t r = i, so = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        so += ((r % g.dne[k]) % g.sne[k]) * g.snb[k];
        r /= g.dne[k];
    }
    dst[i] = *reinterpret_cast<const float *>(src + so);
}

__global__ void k_scale(const float * __restrict__ x, float * __restrict__ y, int64_t n, float sc, float b) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    y[i] = x[i] * sc + b;
}

// ------------------------------------------------------------------------- host launchers

static inline unsigned nblk(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }

void launch_rms_norm(const float * x, int64_t ldx, float * y, int64_t ldy, const float * w, int64_t rows, int64_t n,
                     float eps, hipStream_t s) {
    if (rows == 0) return;
    k_rms_norm<<<(unsigned) rows, 256, 0, s>>>(x, ldx, y, ldy, w, (int) n, eps);
    check_launch("rms_norm");
}

void launch_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, int64_t so_s, int64_t so_h,
                      const int32_t * pos, int64_t D, int64_t H, int64_t S, int n_dims, float freq_base,
                      float freq_scale, float attn_factor, const float * ff, hipStream_t s, const RopeSecond * r2) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int64_t H2 = r2 ? r2->H : 0;
    if (S * (H + H2) * D == 0) return;
    require(n_dims <= 256, "rope: n_dims above 256");
    require(H > 0 || H2 == 0, "rope: the second tensor needs a first");
    const dim3 grid((unsigned) S, (unsigned) ((H + RH - 1) / RH + (H2 + RH - 1) / RH));
    k_rope_neox<<<grid, 256, 0, s>>>(x, sx_s, sx_h, out, so_s, so_h, pos, (int) D, (int) H, (int) S, n_dims,
                                     theta_scale, freq_scale, attn_factor, ff, r2 ? r2->x : nullptr,
                                     r2 ? r2->sx_s : 0, r2 ? r2->sx_h : 0, r2 ? r2->out : nullptr,
                                     r2 ? r2->so_s : 0, r2 ? r2->so_h : 0, (int) H2);
    check_launch("rope");
}

void launch_rope_table(const int32_t * pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                       const float * ff, float2 * cs, hipStream_t s) {
    require(n_dims > 0 && n_dims % 2 == 0 && n_dims <= 256, "rope table: n_dims must be even, <= 256");
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    k_rope_table<<<1, 128, 0, s>>>(pos, n_dims, theta_scale, freq_scale, attn_factor, ff, cs);
    check_launch("rope table");
}

void launch_set_rows_f16(void * dst, int64_t dst_h, int64_t dst_j, const float * src, int64_t src_h, int64_t src_j,
                         const int32_t * idx, int64_t n, int64_t D, int64_t Hrows, int64_t dst_rows, hipStream_t s,
                         const SetRowsSecond * r2) {
    const int64_t t = n * Hrows * (D / 8) + (r2 ? n * r2->Hrows * (r2->D / 8) : 0);
    if (t == 0) return;
    SetRowsSecond z{};
    k_set_rows_f16<<<nblk(t, 256), 256, 0, s>>>((uint16_t *) dst, dst_h, dst_j, src, src_h, src_j, idx, (int) n,
                                                (int) D, (int) Hrows, dst_rows, r2 ? *r2 : z);
    check_launch("set_rows");
}

void launch_get_rows(int type, const void * tab, int64_t nrows_tab, int64_t D, const int32_t * idx, int64_t n,
                     float * out, hipStream_t s) {
    if (n * D == 0) return;
    k_get_rows<<<nblk(n * D, 256), 256, 0, s>>>(type, (const uint8_t *) tab, nrows_tab, (int) D, idx, out, (int) n);
    check_launch("get_rows");
}

void launch_swiglu(const float * g, const float * u, float * y, int64_t n, hipStream_t s) {
    if (n == 0) return;
    k_swiglu<<<nblk(n, 256), 256, 0, s>>>(g, u, y, n);
    check_launch("swiglu");
}

void launch_binary(int op, const float * a, const float * b, float * y, int64_t n, int64_t nb, hipStream_t s) {
    if (n == 0) return;
    k_binary<<<nblk(n, 256), 256, 0, s>>>(op, a, b, y, n, nb);
    check_launch(op == 0 ? "add" : op == 1 ? "mul" : op == 2 ? "sub" : "div");
}

void launch_binary_bcast(int op, const float * a, const float * b, float * y, const int64_t * ane, const int64_t * bne,
                         hipStream_t s) {
    Bcast4 g;
    int64_t n = 1;
    for (int k = 0; k < 4; k++) {
        if (bne[k] <= 0 || ane[k] % bne[k] != 0) throw std::runtime_error("binary: the second operand does not repeat over the first");
        g.ane[k] = ane[k];
        g.bne[k] = bne[k];
        n *= ane[k];
    }
    if (n == 0) return;
    k_binary_bcast<<<nblk(n, 256), 256, 0, s>>>(op, a, b, y, n, g);
    check_launch(op == 0 ? "add" : op == 1 ? "mul" : op == 2 ? "sub" : "div");
}

void launch_unary(int op, const float * x, float * y, int64_t n, float lo, float hi, hipStream_t s) {
    if (!unary_known(op)) throw std::runtime_error("unary: unknown op " + std::to_string(op));
    if (n == 0) return;
    k_unary<<<nblk(n, 256), 256, 0, s>>>(op, x, y, n, lo, hi);
    check_launch("unary");
}

void launch_repeat(const float * src, float * dst, const Cpy4 & g, int64_t n, hipStream_t s) {
    if (n == 0) return;
    k_repeat<<<nblk(n, 256), 256, 0, s>>>((const uint8_t *) src, dst, g, n);
    check_launch("repeat");
}

void launch_norm(const float * x, float * y, int64_t rows, int64_t n, float eps, hipStream_t s) {
    if (rows == 0 || n == 0) return;
    if (rows > INT32_MAX || n > INT32_MAX) throw std::runtime_error("norm: sizes out of range");
    k_norm<<<(unsigned) rows, 256, 0, s>>>(x, y, (int) n, eps);
    check_launch("norm");
}

void launch_row_sum(const float * x, float * y, int64_t rows, int64_t n, bool mean, hipStream_t s) {
    if (rows == 0) return;
    if (rows > INT32_MAX || n > INT32_MAX) throw std::runtime_error("sum_rows: sizes out of range");
    k_row_sum<<<(unsigned) rows, 256, 0, s>>>(x, y, (int) n, mean ? 1 : 0);
    check_launch("sum_rows");
}

void launch_soft_max(const float * x, float * y, int64_t n, int64_t r1, int64_t r2, int64_t r3, const void * mask,
                     bool mask_f16, int64_t mld, int64_t ms2, int64_t ms3, int64_t m2, int64_t m3, float scale,
                     hipStream_t s) {
    const int64_t rows = r1 * r2 * r3;
    if (rows == 0 || n == 0) return;
    if (n > INT32_MAX || r1 > INT32_MAX || r2 > INT32_MAX || rows > INT32_MAX || m2 < 1 || m3 < 1 || m2 > INT32_MAX ||
        m3 > INT32_MAX)
        throw std::runtime_error("soft_max: sizes out of range");
    k_soft_max<<<(unsigned) rows, 256, 0, s>>>(x, y, (int) n, (int) r1, (int) r2, mask, mask_f16 ? 1 : 0, mld, ms2,
                                                 ms3, (int) m2, (int) m3, scale);
    check_launch("soft_max");
}

void launch_argmax(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, hipStream_t s) {
    if (rows == 0) return;
    k_argmax<<<(unsigned) rows, 1024, 0, s>>>(x, ldx, (int) n, out);
    check_launch("argmax");
}

// The sliced argmax's scratch: 64 row counters, then up to 16384 partials.
size_t argmax_split_scratch() { return 256 + 16384 * sizeof(float2); }

bool argmax_split_fits(int64_t rows, int64_t n) {
    return rows >= 1 && rows <= 64 && n >= 4 * kArgmaxSlice && n <= INT32_MAX &&
           rows * ((n + kArgmaxSlice - 1) / kArgmaxSlice) <= 16384;
}

// scratch: argmax_split_scratch() bytes whose first 256 are zero before the first launch (each
// launch leaves them zero).
void launch_argmax_split(const float * x, int64_t ldx, int64_t rows, int64_t n, int32_t * out, void * scratch,
                         hipStream_t s) {
    require(argmax_split_fits(rows, n), "argmax: the sliced kernel takes 1 to 64 rows of 8192 or more values");
    const unsigned slices = (unsigned) ((n + kArgmaxSlice - 1) / kArgmaxSlice);
    unsigned int * counter = (unsigned int *) scratch;
    float2 * part = (float2 *) ((uint8_t *) scratch + 256);
    k_argmax_split<<<dim3(slices, (unsigned) rows), 256, 0, s>>>(x, ldx, (int) n, out, part, counter);
    check_launch("argmax split");
}

SmallJob small_job_get_rows(int type, const void * tab, int64_t nrows_tab, int64_t D, const int32_t * idx, int64_t n,
                            float * out) {
    SmallJob j{};
    j.kind = SJ_GETROWS;
    j.type = type;
    j.D = (int) D;
    j.n = n * D;
    j.src = tab;
    j.aux = idx;
    j.dst = out;
    j.rows = nrows_tab;
    return j;
}

SmallJob small_job_cpy(const void * src, int st, void * dst, int dt, const Cpy4 & g, int64_t n) {
    SmallJob j{};
    j.kind = SJ_CPY;
    j.type = st;
    j.type2 = dt;
    j.n = n;
    j.src = src;
    j.dst = dst;
    j.g = g;
    return j;
}

SmallJob small_job_rope_table(const int32_t * pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                              const float * ff, float2 * cs) {
    require(n_dims > 0 && n_dims % 2 == 0 && n_dims <= 256, "rope table: n_dims must be even, <= 256");
    SmallJob j{};
    j.kind = SJ_ROPE_TABLE;
    j.D = n_dims;
    j.n = n_dims / 2;
    j.src = pos;
    j.aux = ff;
    j.dst = cs;
    j.f[0] = powf(freq_base, -2.0f / (float) n_dims);  // theta_scale, as launch_rope_table
    j.f[1] = freq_scale;
    j.f[2] = attn_factor;
    return j;
}

void launch_small_jobs(const SmallJob * jobs, int n, hipStream_t s) {
    require(n >= 1 && n <= 3, "small jobs: 1 to 3 per launch");
    SmallJobs js{};
    js.nj = n;
    unsigned blocks = 0;
    for (int k = 0; k < n; k++) {
        js.j[k] = jobs[k];
        js.first[k] = blocks;
        const int64_t nb = (jobs[k].n + 255) / 256;
        require(jobs[k].n >= 0 && blocks + nb < (1u << 30), "small jobs: too many threads");
        blocks += (unsigned) nb;
    }
    if (blocks == 0) return;
    k_small_jobs<<<blocks, 256, 0, s>>>(js);
    check_launch("small jobs");
}

void launch_cpy(const void * src, int st, void * dst, int dt, const Cpy4 & g, int64_t n, hipStream_t s) {
    if (n == 0) return;
    k_cpy<<<nblk(n, 256), 256, 0, s>>>((const uint8_t *) src, st, (uint8_t *) dst, dt, g, n);
    check_launch("cpy");
}

void launch_scale(const float * x, float * y, int64_t n, float sc, float b, hipStream_t s) {
    if (n == 0) return;
    k_scale<<<nblk(n, 256), 256, 0, s>>>(x, y, n, sc, b);
    check_launch("scale");
}

void launch_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev, hipStream_t s) {
    if (n == 0) return;
    k_fill_normal<<<nblk(n, 256), 256, 0, s>>>(dst, n, seed, offset, stddev);
    check_launch("fill_normal");
}

void launch_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab, hipStream_t s) {
    if (n == 0) return;
    k_fill_ids<<<nblk(n, 256), 256, 0, s>>>(dst, n, seed, offset, vocab);
    check_launch("fill_ids");
}

}  // namespace gcq
