// quant.hip - weight encoders, weight repacking, dequantization and activation quantizers.
//
// Weight encoders produce ggml's block bytes exactly (the ggml_compiler_quantize contract,
// runtime/include/ggml_compiler_rt.h:83-87, whose CPU implementation is ggml_quantize_chunk with
// no importance matrix, runtime/src/ggml_compiler_rt.cpp:859-876). They run one thread per block
// (one per 256-super-block for the K-quants) in ggml's sequential order with contraction off, so every
// float operation rounds as the C reference does. Activation quantizers produce the vec_dot_type
// that ggml-cpu converts src1 into before a quantized mul_mat (Q8_0 for Q4_0/Q8_0 weights, Q8_K
// for Q4_K / Q5_K / Q6_K), in the device "act" layout described in gcq_common.h.
#include "gcq_common.h"

namespace gcq {

// ----------------------------------------------------------------------- weight encoders

// ggml quantize_row_q8_0_ref: d = amax/127, q = roundf(x * (1/d)).
__global__ void k_enc_q8_0(const float * __restrict__ x, uint8_t * __restrict__ out, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float * xb = x + i * QK;
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t * o = out + i * 34;
    const uint16_t dh = f2h_exact(d);
    o[0] = (uint8_t) dh;
    o[1] = (uint8_t) (dh >> 8);
    for (int j = 0; j < QK; j++) o[2 + j] = (uint8_t) (int8_t) roundf(xb[j] * id);
}

// ggml quantize_row_q4_0_ref: d = (first largest-|x| value)/-8, q = min(15, trunc(x/d + 8.5)).
__global__ void k_enc_q4_0(const float * __restrict__ x, uint8_t * __restrict__ out, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float * xb = x + i * QK;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < QK; j++) {
        const float a = fabsf(xb[j]);
        if (amax < a) {
            amax = a;
            max = xb[j];
        }
    }
    const float d = __fdiv_rn(max, -8.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t * o = out + i * 18;
    const uint16_t dh = f2h_exact(d);
    o[0] = (uint8_t) dh;
    o[1] = (uint8_t) (dh >> 8);
    for (int j = 0; j < QK / 2; j++) {
        int lo = (int) (xb[j] * id + 8.5f);
        int hi = (int) (xb[j + 16] * id + 8.5f);
        lo = lo < 15 ? lo : 15;
        hi = hi < 15 ? hi : 15;
        o[2 + j] = (uint8_t) (lo | (hi << 4));
    }
}

__device__ __forceinline__ int near_int(float v) { return __float2int_rn(v); }

// ggml make_qkx2_quants(32, NMAX, x, w, L, &min, Laux, rmin, 0.1, NSTEP, false): weighted
// least-squares (scale, min) over NSTEP + 1 candidate inverse scales. Sequential, as the C
// reference. Q4_K: NMAX 15, rmin -1, NSTEP 20; Q5_K: NMAX 31, rmin -0.5, NSTEP 15.
template <int NMAX, int NSTEP>
__device__ float qkx2_fit(const float * x, const float * w, uint8_t * L, float * the_min, float rmin) {
#pragma clang fp contract(off)
    uint8_t Laux[32];
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < 32; i++) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float wi = w[i];
        sum_w += wi;
        sum_x += wi * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < 32; i++) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = __fdiv_rn((float) NMAX, max - min);
    float scale = __fdiv_rn(1.0f, iscale);
    float best = 0;
    for (int i = 0; i < 32; i++) {
        int l = near_int(iscale * (x[i] - min));
        l = l < 0 ? 0 : (l > NMAX ? NMAX : l);
        L[i] = (uint8_t) l;
        const float diff = scale * (float) L[i] + min - x[i];
        best += w[i] * (diff * diff);
    }
    for (int is = 0; is <= NSTEP; is++) {
        iscale = __fdiv_rn(rmin + 0.1f * (float) is + (float) NMAX, max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < 32; i++) {
            int l = near_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > NMAX ? NMAX : l);
            Laux[i] = (uint8_t) l;
            const float wi = w[i];
            const float lf = (float) l;
            sum_l += wi * lf;
            sum_l2 += wi * lf * lf;
            sum_xl += wi * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = __fdiv_rn(sum_w * sum_xl - sum_x * sum_l, D);
            float this_min = __fdiv_rn(sum_l2 * sum_x - sum_l * sum_xl, D);
            if (this_min > 0) {
                this_min = 0;
                this_scale = __fdiv_rn(sum_xl, sum_l2);
            }
            float mad = 0;
            for (int i = 0; i < 32; i++) {
                const float diff = this_scale * (float) Laux[i] + this_min - x[i];
                mad += w[i] * (diff * diff);
            }
            if (mad < best) {
                for (int i = 0; i < 32; i++) L[i] = Laux[i];
                best = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t * q, int & sc, int & m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// The 6-bit (scale, min) pairs of a Q4_K / Q5_K super-block, relative to its largest scale and
// min (ggml quantize_row_q4_K_ref / q5_K_ref): writes scales[12], returns fp16 (d, dmin).
__device__ void pack_scale_min_k4(const float * scales, const float * mins, float max_scale, float max_min,
                                  uint8_t * sb, uint16_t & dh, uint16_t & mh) {
#pragma clang fp contract(off)
    const float inv_scale = max_scale > 0 ? __fdiv_rn(63.f, max_scale) : 0.f;
    const float inv_min = max_min > 0 ? __fdiv_rn(63.f, max_min) : 0.f;
    for (int j = 0; j < 12; j++) sb[j] = 0;
    for (int j = 0; j < 8; j++) {
        int ls = near_int(inv_scale * scales[j]);
        int lm = near_int(inv_min * mins[j]);
        ls = ls > 63 ? 63 : ls;
        lm = lm > 63 ? 63 : lm;
        if (j < 4) {
            sb[j] = (uint8_t) ls;
            sb[j + 4] = (uint8_t) lm;
        } else {
            sb[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
            sb[j - 4] |= (uint8_t) ((ls >> 4) << 6);
            sb[j] |= (uint8_t) ((lm >> 4) << 6);
        }
    }
    dh = f2h_exact(__fdiv_rn(max_scale, 63.f));
    mh = f2h_exact(__fdiv_rn(max_min, 63.f));
}

// ggml quantize_row_q4_K_ref, one thread per 256-value super-block.
__global__ void k_enc_q4_K(const float * __restrict__ xall, uint8_t * __restrict__ out, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float * x = xall + i * QKK;
    uint8_t L[QKK];
    float w[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; j++) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; l++) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(__fdiv_rn(sum_x2, 32.0f));  // IEEE sqrt: __fsqrt_rn is the native approximation here
        for (int l = 0; l < 32; l++) w[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = qkx2_fit<15, 20>(x + 32 * j, w, L + 32 * j, &mins[j], -1.0f);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    uint8_t sb[12];
    uint16_t dh, mh;
    pack_scale_min_k4(scales, mins, max_scale, max_min, sb, dh, mh);
    for (int j = 0; j < 8; j++) {
        int sc, m;
        scale_min_k4(j, sb, sc, m);
        const float d = h2f(dh) * (float) sc;
        if (d == 0.0f) continue;  // the fit's codes stay, as in ggml
        const float dm = h2f(mh) * (float) m;
        for (int l = 0; l < 32; l++) {
            int q = near_int(__fdiv_rn(x[32 * j + l] + dm, d));
            L[32 * j + l] = (uint8_t) (q < 0 ? 0 : (q > 15 ? 15 : q));
        }
    }
    uint8_t * o = out + i * 144;
    o[0] = (uint8_t) dh;
    o[1] = (uint8_t) (dh >> 8);
    o[2] = (uint8_t) mh;
    o[3] = (uint8_t) (mh >> 8);
    for (int j = 0; j < 12; j++) o[4 + j] = sb[j];
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) o[16 + 32 * c + l] = (uint8_t) (L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

// ggml quantize_row_q5_K_ref, one thread per 256-value super-block: the Q4_K fit with 5-bit codes
// (make_qkx2_quants(32, 31, ..., -0.5, 0.1, 15)), the fifth bit of value 64c + l (c < 4, l < 64)
// in bit 2c + (l >= 32) of qh[l % 32].
__global__ void k_enc_q5_K(const float * __restrict__ xall, uint8_t * __restrict__ out, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float * x = xall + i * QKK;
    uint8_t L[QKK];
    float w[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; j++) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; l++) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(__fdiv_rn(sum_x2, 32.0f));  // IEEE sqrt: __fsqrt_rn is the native approximation here
        for (int l = 0; l < 32; l++) w[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = qkx2_fit<31, 15>(x + 32 * j, w, L + 32 * j, &mins[j], -0.5f);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    uint8_t sb[12];
    uint16_t dh, mh;
    pack_scale_min_k4(scales, mins, max_scale, max_min, sb, dh, mh);
    for (int j = 0; j < 8; j++) {
        int sc, m;
        scale_min_k4(j, sb, sc, m);
        const float d = h2f(dh) * (float) sc;
        if (d == 0.0f) continue;  // the fit's codes stay, as in ggml
        const float dm = h2f(mh) * (float) m;
        for (int l = 0; l < 32; l++) {
            int q = near_int(__fdiv_rn(x[32 * j + l] + dm, d));
            L[32 * j + l] = (uint8_t) (q < 0 ? 0 : (q > 31 ? 31 : q));
        }
    }
    uint8_t * o = out + i * 176;
    o[0] = (uint8_t) dh;
    o[1] = (uint8_t) (dh >> 8);
    o[2] = (uint8_t) mh;
    o[3] = (uint8_t) (mh >> 8);
    for (int j = 0; j < 12; j++) o[4 + j] = sb[j];
    uint8_t * qh = o + 16;
    uint8_t * ql = o + 48;
    for (int l = 0; l < 32; l++) qh[l] = 0;
    for (int c = 0; c < 4; c++) {
        for (int l = 0; l < 32; l++) {
            int l1 = L[64 * c + l], l2 = L[64 * c + 32 + l];
            if (l1 > 15) {
                l1 -= 16;
                qh[l] |= (uint8_t) (1u << (2 * c));
            }
            if (l2 > 15) {
                l2 -= 16;
                qh[l] |= (uint8_t) (2u << (2 * c));
            }
            ql[32 * c + l] = (uint8_t) (l1 | (l2 << 4));
        }
    }
}

// ggml make_qx_quants(16, 32, x, L, rmse_type = 1, no weights): the symmetric scale of 16 values
// with codes l + 32, l in [-32, 31], refined over 18 candidate inverse scales by the x^2-weighted
// least-squares fit. L receives the codes (0..63).
__device__ float qx_fit16(const float * x, uint8_t * L) {
#pragma clang fp contract(off)
    constexpr int nmax = 32;
    float max = 0, amax = 0;
    for (int i = 0; i < 16; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) {  // GROUP_MAX_EPS
        for (int i = 0; i < 16; i++) L[i] = 0;
        return 0.0f;
    }
    float iscale = __fdiv_rn((float) -nmax, max);
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < 16; i++) {
        int l = near_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (uint8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float) l;
        suml2 += w * (float) l * (float) l;
    }
    float scale = suml2 != 0.0f ? __fdiv_rn(sumlx, suml2) : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0) continue;
        iscale = __fdiv_rn(-((float) nmax + 0.1f * (float) is), max);
        sumlx = suml2 = 0;
        for (int i = 0; i < 16; i++) {
            int l = near_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float) l;
            suml2 += w * (float) l * (float) l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < 16; i++) {
                int l = near_int(iscale * x[i]);
                L[i] = (uint8_t) (nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = __fdiv_rn(sumlx, suml2);
            best = scale * sumlx;
        }
    }
    return scale;
}

// ggml quantize_row_q6_K_ref, one thread per 256-value super-block, written in ggml's 210-byte
// block_q6_K {ql[128], qh[64], scales[16] int8, fp16 d}: 16 sub-block fits, int8 scales against
// the largest-magnitude one (iscale = -128 / max), codes recomputed against the rounded scales.
__global__ void k_enc_q6_K(const float * __restrict__ xall, uint8_t * __restrict__ out, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float * x = xall + i * QKK;
    uint8_t * o = out + i * 210;
    uint8_t L[QKK];
    float scales[16];
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < 16; ib++) {
        const float sc = qx_fit16(x + 16 * ib, L + 16 * ib);
        scales[ib] = sc;
        if (fabsf(sc) > max_abs_scale) {
            max_abs_scale = fabsf(sc);
            max_scale = sc;
        }
    }
    if (max_abs_scale < 1e-15f) {  // an all-zero block
        for (int j = 0; j < 210; j++) o[j] = 0;
        return;
    }
    const float iscale = __fdiv_rn(-128.0f, max_scale);
    const uint16_t dh = f2h_exact(__fdiv_rn(1.0f, iscale));
    int8_t sc8[16];
    for (int ib = 0; ib < 16; ib++) {
        const int v = near_int(iscale * scales[ib]);
        sc8[ib] = (int8_t) (v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; j++) {
        const float d = h2f(dh) * (float) sc8[j];
        if (d == 0.0f) continue;
        for (int ii = 0; ii < 16; ii++) {
            int l = near_int(__fdiv_rn(x[16 * j + ii], d));
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            L[16 * j + ii] = (uint8_t) (l + 32);
        }
    }
    uint8_t * ql = o;
    uint8_t * qh = o + 128;
    for (int h = 0; h < 2; h++) {
        const uint8_t * Lh = L + 128 * h;
        for (int l = 0; l < 32; l++) {
            ql[64 * h + l] = (uint8_t) ((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
            ql[64 * h + 32 + l] = (uint8_t) ((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
            qh[32 * h + l] = (uint8_t) ((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                                        ((Lh[l + 96] >> 4) << 6));
        }
    }
    for (int j = 0; j < 16; j++) o[192 + j] = (uint8_t) sc8[j];
    o[208] = (uint8_t) dh;
    o[209] = (uint8_t) (dh >> 8);
}

// f32 -> f16 rows (ggml_quantize_chunk for F16: round to nearest even).
__global__ void k_enc_f16(const float * __restrict__ x, uint16_t * __restrict__ out, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2h_exact(x[i]);
}

// ------------------------------------------------------------------------------ repacking

// ggml block rows -> packed: Q4_0 / Q8_0 split into 16/32-byte code blocks and an fp16 scale
// array; one thread per block.
template <int CB>  // code bytes per block: 16 (Q4_0) or 32 (Q8_0)
__global__ void k_pack(const uint8_t * __restrict__ src, uint8_t * __restrict__ qs, uint16_t * __restrict__ d,
                       int64_t nblocks) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t * b = src + i * (2 + CB);
    d[i] = (uint16_t) (b[0] | (b[1] << 8));
    uint32_t w[CB / 4];
#pragma unroll
    for (int j = 0; j < CB / 4; j++)
        w[j] = b[2 + 4 * j] | (b[3 + 4 * j] << 8) | (b[4 + 4 * j] << 16) | ((uint32_t) b[5 + 4 * j] << 24);
    uint4 * o = reinterpret_cast<uint4 *>(qs + i * CB);
#pragma unroll
    for (int j = 0; j < CB / 16; j++) o[j] = make_uint4(w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]);
}

// ggml block_q6_K rows -> packed: the first 208 bytes (ql, qh, scales) of each 210-byte block as
// 13 aligned 16-byte pieces into their fields, the fp16 d into its own array; one thread per piece.
__global__ void k_pack_q6_K(const uint8_t * __restrict__ src, uint8_t * __restrict__ qs, uint16_t * __restrict__ d,
                            int64_t nblocks) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 13) return;
    const int64_t i = t / 13;
    const int c = (int) (t % 13);
    const uint8_t * b = src + i * 210 + 16 * c;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        w[j] = b[4 * j] | (b[4 * j + 1] << 8) | (b[4 * j + 2] << 16) | ((uint32_t) b[4 * j + 3] << 24);
    *reinterpret_cast<uint4 *>(qs + q6_off(q6_regions(nblocks), i, 16 * c)) = make_uint4(w[0], w[1], w[2], w[3]);
    if (c == 0) d[i] = (uint16_t) (src[i * 210 + 208] | (src[i * 210 + 209] << 8));
}

// packed Q6_K -> ggml block rows; one thread per output byte.
__global__ void k_unpack_q6_K(const uint8_t * __restrict__ qs, const uint16_t * __restrict__ d, uint8_t * __restrict__ dst,
                              int64_t nblocks) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 210) return;
    const int64_t i = t / 210;
    const int j = (int) (t % 210);
    dst[t] = j < 208 ? qs[q6_off(q6_regions(nblocks), i, j)] : (uint8_t) (d[i] >> (8 * (j - 208)));
}

// Whole ggml rows moved by a row map, 16 bytes per thread (row_bytes % 16 == 0) or 2 (otherwise):
// gather dst[r] = src[map[r]], scatter dst[map[r]] = src[r].
template <class U>
__global__ void k_move_rows(const U * __restrict__ src, U * __restrict__ dst, const int32_t * __restrict__ map,
                            int64_t rows, int64_t per_row, bool scatter) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * per_row) return;
    const int64_t r = t / per_row, c = t % per_row;
    const int64_t m = map[r];
    if (scatter) dst[m * per_row + c] = src[r * per_row + c];
    else dst[r * per_row + c] = src[m * per_row + c];
}

// packed -> ggml block rows (the inverse of k_pack).
template <int CB>
__global__ void k_unpack(const uint8_t * __restrict__ qs, const uint16_t * __restrict__ d, uint8_t * __restrict__ dst,
                         int64_t nblocks) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    uint8_t * b = dst + i * (2 + CB);
    b[0] = (uint8_t) d[i];
    b[1] = (uint8_t) (d[i] >> 8);
    for (int j = 0; j < CB; j++) b[2 + j] = qs[i * CB + j];
}

// ------------------------------------------------------------------------------ dequant

// Packed weight rows -> f32 (ggml dequantize_row_*). Exact: every product is representable.
__global__ void k_dequant_q4_0(const uint8_t * __restrict__ qs, const uint16_t * __restrict__ d, float * __restrict__ y,
                               int64_t nblocks) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;  // one thread per byte
    if (t >= nblocks * 16) return;
    const int64_t i = t / 16;
    const int j = (int) (t % 16);
    const float dd = h2f(d[i]);
    const uint8_t b = qs[t];
    y[i * 32 + j] = (float) ((b & 0xF) - 8) * dd;
    y[i * 32 + j + 16] = (float) ((b >> 4) - 8) * dd;
}

__global__ void k_dequant_q8_0(const int8_t * __restrict__ qs, const uint16_t * __restrict__ d, float * __restrict__ y,
                               int64_t nblocks) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 32) return;
    y[t] = (float) qs[t] * h2f(d[t / 32]);
}

__global__ void k_dequant_q4_K(const uint8_t * __restrict__ w, float * __restrict__ y, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;  // one thread per qs byte
    if (t >= nblocks * 128) return;
    const int64_t i = t / 128;
    const int k = (int) (t % 128);
    const int c = k / 32, l = k % 32;
    const KqRegions R = kq_regions(T_Q4_K, nblocks);
    const uint8_t * b = w + R.hdr + i * 16;  // d, dmin, scales[12]
    const float d = h2f((uint16_t) (b[0] | (b[1] << 8)));
    const float dmin = h2f((uint16_t) (b[2] | (b[3] << 8)));
    int sc, m;
    scale_min_k4(2 * c, b + 4, sc, m);
    const float d1 = d * (float) sc, m1 = dmin * (float) m;
    scale_min_k4(2 * c + 1, b + 4, sc, m);
    const float d2 = d * (float) sc, m2 = dmin * (float) m;
    const uint8_t q = w[R.qs + i * 128 + k];
    y[i * 256 + 64 * c + l] = d1 * (float) (q & 0xF) - m1;
    y[i * 256 + 64 * c + 32 + l] = d2 * (float) (q >> 4) - m2;
}

// ggml dequantize_row_q5_K: y = d * sc * (nibble + 16 * high bit) - dmin * m; one thread per qs byte.
__global__ void k_dequant_q5_K(const uint8_t * __restrict__ w, float * __restrict__ y, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 128) return;
    const int64_t i = t / 128;
    const int k = (int) (t % 128);
    const int c = k / 32, l = k % 32;
    const KqRegions R = kq_regions(T_Q5_K, nblocks);
    const uint8_t * b = w + R.hdr + i * 16;  // d, dmin, scales[12]
    const float d = h2f((uint16_t) (b[0] | (b[1] << 8)));
    const float dmin = h2f((uint16_t) (b[2] | (b[3] << 8)));
    int sc, m;
    scale_min_k4(2 * c, b + 4, sc, m);
    const float d1 = d * (float) sc, m1 = dmin * (float) m;
    scale_min_k4(2 * c + 1, b + 4, sc, m);
    const float d2 = d * (float) sc, m2 = dmin * (float) m;
    const uint8_t q = w[R.qs + i * 128 + k], h = w[R.qh + i * 32 + l];
    y[i * 256 + 64 * c + l] = d1 * (float) ((q & 0xF) + ((h >> (2 * c)) & 1 ? 16 : 0)) - m1;
    y[i * 256 + 64 * c + 32 + l] = d2 * (float) ((q >> 4) + ((h >> (2 * c + 1)) & 1 ? 16 : 0)) - m2;
}

// ggml dequantize_row_q6_K on the packed layout: y = d * sc * (q - 32); one thread per (block,
// half h, l < 32), four values each.
__global__ void k_dequant_q6_K(const uint8_t * __restrict__ qs, const uint16_t * __restrict__ dv,
                               float * __restrict__ y, int64_t nblocks) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 64) return;
    const int64_t i = t / 64;
    const int h = (int) (t % 64) / 32, l = (int) (t % 32);
    const Q6Regions R = q6_regions(nblocks);
    const float d = h2f(dv[i]);
    const uint8_t a0 = qs[q6_off(R, i, 64 * h + l)], a1 = qs[q6_off(R, i, 64 * h + 32 + l)];
    const uint8_t qh = qs[q6_off(R, i, 128 + 32 * h + l)];
    const int8_t * sc = reinterpret_cast<const int8_t *>(qs + q6_off(R, i, 192 + 8 * h));
    const int is = l / 16;
    const int q1 = (int) ((a0 & 0xF) | (((qh >> 0) & 3) << 4)) - 32;
    const int q2 = (int) ((a1 & 0xF) | (((qh >> 2) & 3) << 4)) - 32;
    const int q3 = (int) ((a0 >> 4) | (((qh >> 4) & 3) << 4)) - 32;
    const int q4 = (int) ((a1 >> 4) | (((qh >> 6) & 3) << 4)) - 32;
    float * o = y + i * 256 + 128 * h + l;
    o[0] = d * (float) sc[is + 0] * (float) q1;
    o[32] = d * (float) sc[is + 2] * (float) q2;
    o[64] = d * (float) sc[is + 4] * (float) q3;
    o[96] = d * (float) sc[is + 6] * (float) q4;
}

// ------------------------------------------------------------------ activation quantizers

// Q8_0 vec_dot_type, canonical variant (ggml-cpu x86 AVX2 quantize_row_q8_0): d = amax/127 kept
// as fp16, id = 127/amax, q = rint(x*id) (ties to even). 8 lanes per 32-block, 4 values each.
__global__ void k_act_q8_0(const float * __restrict__ x, int64_t ldx, int8_t * __restrict__ codes,
                           float2 * __restrict__ meta, int64_t B, int64_t K) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = K / 4;
    if (t >= B * per_row) return;  // B*K/4 is a multiple of 8: whole 8-lane groups stay together
    const int64_t b = t / per_row;
    const int64_t e = (t % per_row) * 4;
    const float4 v = *reinterpret_cast<const float4 *>(x + b * ldx + e);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    const int q0 = (int) __builtin_rintf(v.x * id);
    const int q1 = (int) __builtin_rintf(v.y * id);
    const int q2 = (int) __builtin_rintf(v.z * id);
    const int q3 = (int) __builtin_rintf(v.w * id);
    *reinterpret_cast<int *>(codes + b * K + e) =
        (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if ((threadIdx.x & 7) == 0) {
        const float d = h2f(f2h_exact(__fdiv_rn(amax, 127.0f)));
        meta[b * (K / QK) + e / QK] = make_float2(d, __int_as_float(s));
    }
}

// Q8_K vec_dot_type (ggml quantize_row_q8_K_ref): max = signed value of the first largest |x|,
// iscale = -127/max, q = min(127, rint(iscale*x)), d = 1/iscale, bsums of 16. One wave per
// super-block, 4 values per lane; an all-zero block stores zeros.
__global__ void k_act_q8_K(const float * __restrict__ x, int64_t ldx, int8_t * __restrict__ codes,
                           int16_t * __restrict__ bsums, float * __restrict__ dout, int64_t B, int64_t K) {
#pragma clang fp contract(off)
    const int64_t wave = ((int64_t) blockIdx.x * blockDim.x + threadIdx.x) / 64;
    const int lane = threadIdx.x & 63;
    const int64_t nsb = K / QKK;
    if (wave >= B * nsb) return;
    const int64_t b = wave / nsb, sbi = wave % nsb;
    const int64_t e = sbi * QKK + lane * 4;
    const float4 v = *reinterpret_cast<const float4 *>(x + b * ldx + e);
    const float vv[4] = {v.x, v.y, v.z, v.w};
    float ax = 0.0f, mx = 0.0f;
    int idx = 1 << 30;
    for (int j = 0; j < 4; j++) {
        if (fabsf(vv[j]) > ax) {
            ax = fabsf(vv[j]);
            mx = vv[j];
            idx = lane * 4 + j;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {  // largest |x|, ties to the lowest index
        const float ax2 = __shfl_xor(ax, o, 64);
        const float mx2 = __shfl_xor(mx, o, 64);
        const int idx2 = __shfl_xor(idx, o, 64);
        if (ax2 > ax || (ax2 == ax && idx2 < idx)) {
            ax = ax2;
            mx = mx2;
            idx = idx2;
        }
    }
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (ax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
        for (int j = 0; j < 4; j++) {
            const int r = (int) __builtin_rintf((iscale * vv[j]));
            q[j] = r < 127 ? r : 127;
        }
        d = __fdiv_rn(1.0f, iscale);
    }
    *reinterpret_cast<int *>(codes + b * K + e) =
        (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((q[3] & 0xff) << 24);
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) bsums[b * (K / 16) + sbi * 16 + lane / 4] = (int16_t) s;
    if (lane == 0) dout[b * nsb + sbi] = d;
}

// Device act layout -> ggml block bytes (block_q8_0 / block_q8_K), for byte comparisons.
__global__ void k_act_to_ggml_q8_0(const int8_t * codes, const float2 * meta, uint8_t * out, int64_t nblocks) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t h = f2h_exact(meta[i].x);
    uint8_t * o = out + i * 34;
    o[0] = (uint8_t) h;
    o[1] = (uint8_t) (h >> 8);
    for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) codes[i * 32 + j];
}

__global__ void k_act_to_ggml_q8_K(const int8_t * codes, const int16_t * bsums, const float * d, uint8_t * out,
                                   int64_t nblocks) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    uint8_t * o = out + i * 292;
    const float dv = d[i];
    __builtin_memcpy(o, &dv, 4);
    for (int j = 0; j < 256; j++) o[4 + j] = (uint8_t) codes[i * 256 + j];
    for (int j = 0; j < 16; j++) {
        const int16_t s = bsums[i * 16 + j];
        o[260 + 2 * j] = (uint8_t) s;
        o[261 + 2 * j] = (uint8_t) ((uint16_t) s >> 8);
    }
}

// ------------------------------------------------------------------------- host launchers

static inline unsigned nblk(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }

void launch_encode(int type, const float * src, int64_t nrows, int64_t k, void * dst, hipStream_t s) {
    const int64_t nb = nrows * (k / (int64_t) block_elems(type));
    if (nb == 0) return;
    switch (type) {
        case T_Q8_0: k_enc_q8_0<<<nblk(nb, 128), 128, 0, s>>>(src, (uint8_t *) dst, nb); break;
        case T_Q4_0: k_enc_q4_0<<<nblk(nb, 128), 128, 0, s>>>(src, (uint8_t *) dst, nb); break;
        case T_Q4_K: k_enc_q4_K<<<nblk(nb, 64), 64, 0, s>>>(src, (uint8_t *) dst, nb); break;
        case T_Q5_K: k_enc_q5_K<<<nblk(nb, 64), 64, 0, s>>>(src, (uint8_t *) dst, nb); break;
        case T_Q6_K: k_enc_q6_K<<<nblk(nb, 64), 64, 0, s>>>(src, (uint8_t *) dst, nb); break;
        case T_F16: k_enc_f16<<<nblk(nb, 256), 256, 0, s>>>(src, (uint16_t *) dst, nb); break;
        default: fail("encode: unsupported type " + std::to_string(type));
    }
    check_launch("encode");
}

// ggml Q4_K / Q5_K super-blocks <-> the packed fields, one thread per 16-byte piece of a super-block
// (ggml's order: the header {d, dmin, scales[12]}, Q5_K's qh[32] in two, qs[128] in eight).
template <bool PACK>
__global__ void k_pack_kq(int type, const uint4 * __restrict__ src, uint4 * __restrict__ dst, int64_t nb) {
    const int pp = type == T_Q5_K ? 11 : 9;
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nb * pp) return;
    const int64_t i = t / pp;
    const int p = (int) (t % pp);
    const KqRegions R = kq_regions(type, nb);
    size_t o;  // the piece's byte offset in the packed weight
    if (p == 0) o = R.hdr + (size_t) i * 16;
    else if (type == T_Q5_K && p < 3) o = R.qh + (size_t) i * 32 + (size_t) (p - 1) * 16;
    else o = R.qs + (size_t) i * 128 + (size_t) (p - (type == T_Q5_K ? 3 : 1)) * 16;
    if (PACK) dst[o / 16] = src[t];
    else dst[t] = src[o / 16];
}

void launch_pack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s) {
    const WeightLayout L = weight_layout(type, nrows, k);
    uint8_t * o = (uint8_t *) dst;
    if (type == T_Q4_K || type == T_Q5_K) {
        require(aligned(src, 16) && aligned(dst, 16), "pack: K-quant rows need 16-byte aligned buffers");
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_pack_kq<true><<<nblk(nb * (type == T_Q5_K ? 11 : 9), 256), 256, 0, s>>>(type, (const uint4 *) src, (uint4 *) dst, nb);
        check_launch("pack");
        return;
    }
    if (type == T_Q6_K) {
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_pack_q6_K<<<nblk(nb * 13, 256), 256, 0, s>>>((const uint8_t *) src, o + L.qs, (uint16_t *) (o + L.d), nb);
        check_launch("pack");
        return;
    }
    const int64_t nb = nrows * (k / QK);
    if (nb == 0) return;
    if (type == T_Q4_0)
        k_pack<16><<<nblk(nb, 256), 256, 0, s>>>((const uint8_t *) src, o + L.qs, (uint16_t *) (o + L.d), nb);
    else if (type == T_Q8_0)
        k_pack<32><<<nblk(nb, 256), 256, 0, s>>>((const uint8_t *) src, o + L.qs, (uint16_t *) (o + L.d), nb);
    else
        fail("pack: unsupported type " + std::to_string(type));
    check_launch("pack");
}

void launch_move_rows(const void * src, void * dst, const int32_t * map, int64_t rows, int64_t row_bytes, bool scatter,
                      hipStream_t s) {
    if (rows == 0) return;
    if (row_bytes % 16 == 0) {
        const int64_t per = row_bytes / 16;
        k_move_rows<uint4><<<nblk(rows * per, 256), 256, 0, s>>>((const uint4 *) src, (uint4 *) dst, map, rows, per,
                                                                 scatter);
    } else {
        require(row_bytes % 2 == 0, "move_rows: odd row size");
        const int64_t per = row_bytes / 2;
        k_move_rows<uint16_t><<<nblk(rows * per, 256), 256, 0, s>>>((const uint16_t *) src, (uint16_t *) dst, map,
                                                                    rows, per, scatter);
    }
    check_launch("move_rows");
}

void launch_unpack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s) {
    const WeightLayout L = weight_layout(type, nrows, k);
    const uint8_t * p = (const uint8_t *) src;
    if (type == T_Q4_K || type == T_Q5_K) {
        require(aligned(src, 16) && aligned(dst, 16), "unpack: K-quant rows need 16-byte aligned buffers");
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_pack_kq<false><<<nblk(nb * (type == T_Q5_K ? 11 : 9), 256), 256, 0, s>>>(type, (const uint4 *) src, (uint4 *) dst, nb);
        check_launch("unpack");
        return;
    }
    if (type == T_Q6_K) {
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_unpack_q6_K<<<nblk(nb * 210, 256), 256, 0, s>>>(p + L.qs, (const uint16_t *) (p + L.d), (uint8_t *) dst, nb);
        check_launch("unpack");
        return;
    }
    const int64_t nb = nrows * (k / QK);
    if (nb == 0) return;
    if (type == T_Q4_0)
        k_unpack<16><<<nblk(nb, 256), 256, 0, s>>>(p + L.qs, (const uint16_t *) (p + L.d), (uint8_t *) dst, nb);
    else if (type == T_Q8_0)
        k_unpack<32><<<nblk(nb, 256), 256, 0, s>>>(p + L.qs, (const uint16_t *) (p + L.d), (uint8_t *) dst, nb);
    else
        fail("unpack: unsupported type " + std::to_string(type));
    check_launch("unpack");
}

void launch_dequant(int type, const void * w, int64_t nrows, int64_t k, float * y, hipStream_t s) {
    const WeightLayout L = weight_layout(type, nrows, k);
    const uint8_t * p = (const uint8_t *) w;
    if (type == T_Q4_0) {
        const int64_t nb = nrows * (k / QK);
        if (nb) k_dequant_q4_0<<<nblk(nb * 16, 256), 256, 0, s>>>(p + L.qs, (const uint16_t *) (p + L.d), y, nb);
    } else if (type == T_Q8_0) {
        const int64_t nb = nrows * (k / QK);
        if (nb) k_dequant_q8_0<<<nblk(nb * 32, 256), 256, 0, s>>>((const int8_t *) (p + L.qs), (const uint16_t *) (p + L.d), y, nb);
    } else if (type == T_Q4_K) {
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_dequant_q4_K<<<nblk(nb * 128, 256), 256, 0, s>>>(p, y, nb);
    } else if (type == T_Q5_K) {
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_dequant_q5_K<<<nblk(nb * 128, 256), 256, 0, s>>>(p, y, nb);
    } else if (type == T_Q6_K) {
        const int64_t nb = nrows * (k / QKK);
        if (nb) k_dequant_q6_K<<<nblk(nb * 64, 256), 256, 0, s>>>(p + L.qs, (const uint16_t *) (p + L.d), y, nb);
    } else {
        fail("dequantize: unsupported type " + std::to_string(type));
    }
    check_launch("dequantize");
}

void launch_act_quant(int wtype, const float * x, int64_t ldx, int64_t B, int64_t k, void * act, hipStream_t s) {
    const ActLayout L = act_layout(wtype, B, k);
    uint8_t * a = (uint8_t *) act;
    if (wtype == T_Q4_0 || wtype == T_Q8_0) {
        const int64_t n = B * k / 4;
        k_act_q8_0<<<nblk(n, 256), 256, 0, s>>>(x, ldx, (int8_t *) (a + L.codes), (float2 *) (a + L.meta), B, k);
    } else if (is_kquant(wtype)) {
        const int64_t waves = B * (k / QKK);
        k_act_q8_K<<<nblk(waves * 64, 256), 256, 0, s>>>(x, ldx, (int8_t *) (a + L.codes), (int16_t *) (a + L.meta),
                                                        (float *) (a + L.d), B, k);
    } else {
        fail("activation quantize: unsupported weight type " + std::to_string(wtype));
    }
    check_launch("activation quantize");
}

void launch_act_to_ggml(int wtype, const void * act, int64_t B, int64_t k, void * out, hipStream_t s) {
    const ActLayout L = act_layout(wtype, B, k);
    const uint8_t * a = (const uint8_t *) act;
    if (wtype == T_Q4_0 || wtype == T_Q8_0) {
        const int64_t nb = B * k / QK;
        k_act_to_ggml_q8_0<<<nblk(nb, 128), 128, 0, s>>>((const int8_t *) (a + L.codes), (const float2 *) (a + L.meta),
                                                         (uint8_t *) out, nb);
    } else {
        const int64_t nb = B * k / QKK;
        k_act_to_ggml_q8_K<<<nblk(nb, 64), 64, 0, s>>>((const int8_t *) (a + L.codes), (const int16_t *) (a + L.meta),
                                                       (const float *) (a + L.d), (uint8_t *) out, nb);
    }
    check_launch("act_to_ggml");
}

}  // namespace gcq
