/*
 * gcq_oracle.c - CPU oracle for the quantized mat-mul / KV-cache attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libgcq.so's HIP kernels and the CPU baseline that
 * bench.py reports beside them. Nothing in the product links or calls it.
 *
 * Every function restates the semantics of one ggml CPU routine that ggml-compiler's runtime
 * reaches for this path. ggml (llama.cpp b11223, fetched by runtime/CMakeLists.txt:33-40) is not
 * present, so the restatement follows ggml's published algorithms; each function names the ggml
 * routine and the reference call site it stands for. Floating-point contraction is off for this
 * file (-ffp-contract=off): ggml's reference encoders live in ggml-base, which is built without
 * FMA code generation, so a contracted a*b+c would change codes at rounding boundaries.
 *
 * Parity pins (tests/test_oracle.py): fp16 against numpy's IEEE conversion; encoders against
 * hand-worked blocks, on-grid round trips (the tests/unit/test_modelopt.py:60-72 pattern) and
 * error invariants; integer block sums against int64 brute force; mul_mat / rms_norm / rope /
 * flash_attn against float64 closed forms. The K-quant encoders' searches (make_qkx2_quants,
 * make_qx_quants) are pinned by tests/test_kquant_search.py in float64: each candidate step
 * against the published candidate formula, each fit against the closed-form weighted least-squares
 * solution for its codes, the result the least weighted error of the fits made (Q6_K: of the
 * published candidate set, enumerated), and a wrong search parameter rejected. ggml's float summation
 * order inside mul_mat / flash_attn is parity unpinned: no ggml build exists to compare against.
 */
#include "gcq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define QK32 32
#define QKK 256

typedef struct { uint16_t d; int8_t qs[QK32]; } blk_q8_0;                       /* 34 B */
typedef struct { uint16_t d; uint8_t qs[QK32 / 2]; } blk_q4_0;                  /* 18 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QKK / 2]; } blk_q4_K;  /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[QKK / 8]; uint8_t qs[QKK / 2]; } blk_q5_K; /* 176 B */
typedef struct { uint8_t ql[QKK / 2]; uint8_t qh[QKK / 4]; int8_t scales[QKK / 16]; uint16_t d; } blk_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[QKK]; int16_t bsums[QKK / 16]; } blk_q8_K; /* 292 B */

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 block");
_Static_assert(sizeof(blk_q4_0) == 18, "q4_0 block");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K block");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K block");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K block");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K block");

static int nthreads_of(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void) n;
    return 1;
#endif
}

/* ---------------------------------------------------------------- fp16 (IEEE binary16, RNE) */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);   /* NaN */
    if (ax >= 0x47800000u) return (uint16_t) (sign | 0x7c00u);  /* >= 65536 (and inf): inf */
    if (ax < 0x38800000u) {                                      /* below 2^-14: subnormal half */
        const uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t) sign;                     /* < 2^-25: rounds to zero */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;                          /* 14 .. 24 */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t) (sign | h);
    }
    uint32_t h = ((((ax >> 23) - 112) << 10) | ((ax >> 13) & 0x3ffu));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;     /* carry may reach inf: correct */
    return (uint16_t) (sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in f32 */
            float v = (float) m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_fp32_to_fp16_n(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp32_to_fp16(x[i]);
}

void orc_fp16_to_fp32_n(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------- synthetic data (PRNG) */

/* splitmix64: output i of a generator whose state starts at `seed` (counter-based, so any
 * element can be produced on its own, on the CPU or the GPU). */
uint64_t orc_rnd64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* An approximately N(0, 1) value from twelve 24-bit uniforms (Irwin-Hall, variance 1 up to
 * 2^-48): integer arithmetic, one int->float conversion and exact power-of-two scaling, so the
 * GPU produces the same bits. */
static float normal_at(uint64_t seed, uint64_t i) {
    int64_t s = 0;
    for (int j = 0; j < 6; j++) {
        const uint64_t r = orc_rnd64(seed, 6 * i + (uint64_t) j);
        s += (int64_t) (r & 0xffffffu) + (int64_t) ((r >> 32) & 0xffffffu);
    }
    const int32_t c = (int32_t) (s - 6 * (int64_t) 0xffffff);
    return (float) c * (1.0f / 16777216.0f);
}

void orc_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) dst[i] = normal_at(seed, offset + (uint64_t) i) * stddev;
}

void orc_fill_ids(int32_t * dst, int64_t n, uint64_t seed, uint64_t offset, int32_t vocab) {
    for (int64_t i = 0; i < n; i++) dst[i] = (int32_t) (orc_rnd64(seed, offset + (uint64_t) i) % (uint64_t) vocab);
}

/* ---------------------------------------------------------------------------- type table */

size_t orc_block_size(int type) {
    switch (type) {
        case ORC_F32: case ORC_F16: return 1;
        case ORC_Q4_0: case ORC_Q8_0: return QK32;
        case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return QKK;
        default: return 0;
    }
}

size_t orc_type_size(int type) {
    switch (type) {
        case ORC_F32: return 4;
        case ORC_F16: return 2;
        case ORC_Q4_0: return sizeof(blk_q4_0);
        case ORC_Q8_0: return sizeof(blk_q8_0);
        case ORC_Q4_K: return sizeof(blk_q4_K);
        case ORC_Q5_K: return sizeof(blk_q5_K);
        case ORC_Q6_K: return sizeof(blk_q6_K);
        case ORC_Q8_K: return sizeof(blk_q8_K);
        default: return 0;
    }
}

size_t orc_row_size(int type, int64_t n) {
    const size_t bs = orc_block_size(type);
    if (!bs || n % (int64_t) bs) return 0;
    return orc_type_size(type) * (size_t) (n / (int64_t) bs);
}

/* ------------------------------------------------------------------------- weight encoders */

/* ggml quantize_row_q8_0_ref: d = amax/127, q = roundf(x / d) (half away from zero). */
static void enc_q8_0(const float * x, blk_q8_0 * y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, x += QK32) {
        float amax = 0.0f;
        for (int j = 0; j < QK32; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK32; j++) y[i].qs[j] = (int8_t) roundf(x[j] * id);
    }
}

/* ggml quantize_row_q4_0_ref: d = (signed value of largest |x|, first one) / -8,
 * q = min(15, (int8)(x/d + 8.5)); byte j holds element j (low) and element j+16 (high). */
static void enc_q4_0(const float * x, blk_q4_0 * y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, x += QK32) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK32; j++) {
            if (amax < fabsf(x[j])) {
                amax = fabsf(x[j]);
                max = x[j];
            }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK32 / 2; j++) {
            const int lo = (int8_t) (x[j] * id + 8.5f);
            const int hi = (int8_t) (x[j + QK32 / 2] * id + 8.5f);
            y[i].qs[j] = (uint8_t) ((lo < 15 ? lo : 15) | ((hi < 15 ? hi : 15) << 4));
        }
    }
}

/* ggml nearest_int: round to nearest, ties to even, for |v| < 2^22. */
static inline int nearest_int(float v) { return (int) lrintf(v); }

/* ggml make_qkx2_quants(n=32, nmax, rmin, rdelta=0.1, nstep, use_mad=false): an asymmetric
 * (scale, min) fit by weighted least squares over nstep + 1 candidate scales. Q4_K calls it with
 * (nmax 15, rmin -1, nstep 20), Q5_K with (31, -0.5, 15). */
/* trace (optional, tests): row 0 the min/max fit, row 1 + s candidate s, QKX2_TRACE floats each:
 * [iscale, D > 0, scale, min, weighted error, taken, min the codes were made against, 0, codes[32]]. */
#define QKX2_TRACE 40
static float make_qkx2(const float * x, const float * w, uint8_t * L, float * the_min, int nmax, float rmin, int nstep,
                       float * trace) {
    const int n = 32;
    const float rdelta = 0.1f;
    uint8_t Laux[32];
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float wi = w[i];
        sum_w += wi;
        sum_x += wi * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; i++) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * (x[i] - min));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t) l;
        const float diff = scale * L[i] + min - x[i];
        best += w[i] * (diff * diff);
    }
    if (trace) {
        float * t = trace;
        t[0] = iscale, t[1] = 1, t[2] = scale, t[3] = min, t[4] = best, t[5] = 1, t[6] = min, t[7] = 0;
        for (int i = 0; i < n; i++) t[8 + i] = L[i];
    }
    for (int is = 0; is <= nstep; is++) {
        float * t = trace ? trace + QKX2_TRACE * (1 + is) : NULL;
        if (t) memset(t, 0, QKX2_TRACE * sizeof(float));
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        if (t) t[0] = iscale, t[6] = min;
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t) l;
            if (t) t[8 + i] = (float) l;
            const float wi = w[i];
            sum_l += wi * l;
            sum_l2 += wi * l * l;
            sum_xl += wi * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; i++) {
                const float diff = this_scale * Laux[i] + this_min - x[i];
                mad += w[i] * (diff * diff);
            }
            if (t) t[1] = 1, t[2] = this_scale, t[3] = this_min, t[4] = mad, t[5] = mad < best;
            if (mad < best) {
                for (int i = 0; i < n; i++) L[i] = Laux[i];
                best = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* The search of one 32-value sub-block alone (the fit enc_q4_K / enc_q5_K run per sub-block), for
 * the tests that check each of its steps against the published definition; trace: NULL or
 * (nstep + 2) x QKX2_TRACE floats (see make_qkx2). */
float orc_make_qkx2(const float * x, const float * w, uint8_t * L, float * the_min, int nmax, float rmin, int nstep,
                    float * trace) {
    return make_qkx2(x, w, L, the_min, nmax, rmin, nstep, trace);
}

/* ggml get_scale_min_k4: 6-bit (scale, min) of sub-block j from the 12 packed bytes. */
static inline void scale_min_k4(int j, const uint8_t * q, uint8_t * sc, uint8_t * m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* The 6-bit (scale, min) pairs of a Q4_K / Q5_K super-block against its largest scale and min,
 * and the fp16 (d, dmin) they are relative to (quantize_row_q4_K_ref / q5_K_ref). */
static void pack_scale_min_k4(const float * scales, const float * mins, float max_scale, float max_min,
                              uint8_t sb[12], uint16_t * d, uint16_t * dmin) {
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(sb, 0, 12);
    for (int j = 0; j < 8; j++) {
        int ls = nearest_int(inv_scale * scales[j]);
        int lm = nearest_int(inv_min * mins[j]);
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
    *d = orc_fp32_to_fp16(max_scale / 63.f);
    *dmin = orc_fp32_to_fp16(max_min / 63.f);
}

/* ggml quantize_row_q4_K_ref: per 32-sub-block make_qkx2 fit with weights sqrt(mean x^2) + |x|,
 * then 6-bit scales/mins relative to the super-block's max scale and max min, then codes
 * recomputed against the rounded scales. */
static void enc_q4_K(const float * x, blk_q4_K * y, int64_t nb) {
    uint8_t L[QKK];
    float weights[32], mins[8], scales[8];
    for (int64_t i = 0; i < nb; i++, x += QKK) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; j++) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; l++) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; l++) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2(x + 32 * j, weights, L + 32 * j, &mins[j], 15, -1.0f, 20, NULL);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        pack_scale_min_k4(scales, mins, max_scale, max_min, y[i].scales, &y[i].d, &y[i].dmin);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = orc_fp16_to_fp32(y[i].d) * sc;
            if (d == 0.0f) continue;
            const float dm = orc_fp16_to_fp32(y[i].dmin) * m;
            for (int l = 0; l < 32; l++) {
                int q = nearest_int((x[32 * j + l] + dm) / d);
                L[32 * j + l] = (uint8_t) (q < 0 ? 0 : (q > 15 ? 15 : q));
            }
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++)
                y[i].qs[32 * c + l] = (uint8_t) (L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

/* ggml quantize_row_q5_K_ref: the Q4_K scheme with 5-bit codes (make_qkx2 with nmax 31, rmin
 * -0.5, 15 steps); the fifth bit of value 64c + l (l < 32) goes to bit 2c of qh[l], that of value
 * 64c + 32 + l to bit 2c + 1. */
static void enc_q5_K(const float * x, blk_q5_K * y, int64_t nb) {
    uint8_t L[QKK];
    float weights[32], mins[8], scales[8];
    for (int64_t i = 0; i < nb; i++, x += QKK) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; j++) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; l++) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; l++) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2(x + 32 * j, weights, L + 32 * j, &mins[j], 31, -0.5f, 15, NULL);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        pack_scale_min_k4(scales, mins, max_scale, max_min, y[i].scales, &y[i].d, &y[i].dmin);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = orc_fp16_to_fp32(y[i].d) * sc;
            if (d == 0.0f) continue;
            const float dm = orc_fp16_to_fp32(y[i].dmin) * m;
            for (int l = 0; l < 32; l++) {
                int q = nearest_int((x[32 * j + l] + dm) / d);
                L[32 * j + l] = (uint8_t) (q < 0 ? 0 : (q > 31 ? 31 : q));
            }
        }
        memset(y[i].qh, 0, sizeof(y[i].qh));
        for (int c = 0; c < 4; c++) {
            for (int l = 0; l < 32; l++) {
                int l1 = L[64 * c + l], l2 = L[64 * c + 32 + l];
                if (l1 > 15) {
                    l1 -= 16;
                    y[i].qh[l] |= (uint8_t) (1u << (2 * c));
                }
                if (l2 > 15) {
                    l2 -= 16;
                    y[i].qh[l] |= (uint8_t) (2u << (2 * c));
                }
                y[i].qs[32 * c + l] = (uint8_t) (l1 | (l2 << 4));
            }
        }
    }
}

/* ggml make_qx_quants(n = 16, nmax = 32, rmse_type = 1, no importance weights): the symmetric scale
 * of a 16-value sub-block, codes L = l + 32 with l in [-32, 31], the first scale -32/max refined
 * over 18 candidates -(32 + 0.1 is)/max (is = -9..9, not 0) by the x^2-weighted fit. */
static float make_qx16(const float * x, uint8_t * L) {
    const int n = 16, nmax = 32;
    float max = 0, amax = 0;
    for (int i = 0; i < n; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) { /* GROUP_MAX_EPS */
        memset(L, 0, (size_t) n);
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (uint8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; i++) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (uint8_t) (nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* The search of one 16-value sub-block alone (enc_q6_K's per-sub-block fit), for the tests. */
float orc_make_qx16(const float * x, uint8_t * L) { return make_qx16(x, L); }

/* ggml quantize_row_q6_K_ref: 16 sub-block fits (make_qx16), int8 scales against the scale of
 * largest magnitude (iscale = -128/max, d = 1/iscale), codes recomputed against the rounded
 * scales, then 4 low bits to ql and 2 high bits to qh in ggml's interleaved order. */
static void enc_q6_K(const float * x, blk_q6_K * y, int64_t nb) {
    uint8_t L[QKK];
    float scales[16];
    for (int64_t i = 0; i < nb; i++, x += QKK) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ib++) {
            const float sc = make_qx16(x + 16 * ib, L + 16 * ib);
            scales[ib] = sc;
            if (fabsf(sc) > max_abs_scale) {
                max_abs_scale = fabsf(sc);
                max_scale = sc;
            }
        }
        if (max_abs_scale < 1e-15f) {
            memset(&y[i], 0, sizeof(blk_q6_K));
            continue;
        }
        const float iscale = -128.f / max_scale;
        y[i].d = orc_fp32_to_fp16(1 / iscale);
        for (int ib = 0; ib < 16; ib++) {
            const int v = nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            const float d = orc_fp16_to_fp32(y[i].d) * y[i].scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (uint8_t) (l + 32);
            }
        }
        for (int h = 0; h < 2; h++) {
            const uint8_t * Lh = L + 128 * h;
            uint8_t * ql = y[i].ql + 64 * h;
            uint8_t * qh = y[i].qh + 32 * h;
            for (int l = 0; l < 32; l++) {
                ql[l] = (uint8_t) ((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
                ql[l + 32] = (uint8_t) ((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
                qh[l] = (uint8_t) ((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                                   ((Lh[l + 96] >> 4) << 6));
            }
        }
    }
}

size_t orc_quantize(int type, const float * src, int64_t nrows, int64_t n_per_row, void * dst) {
    const size_t rs = orc_row_size(type, n_per_row);
    if (!rs || nrows < 0) return 0;
    const int64_t nb = n_per_row / (int64_t) orc_block_size(type);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; r++) {
        const float * x = src + r * n_per_row;
        uint8_t * y = (uint8_t *) dst + (size_t) r * rs;
        switch (type) {
            case ORC_Q8_0: enc_q8_0(x, (blk_q8_0 *) y, nb); break;
            case ORC_Q4_0: enc_q4_0(x, (blk_q4_0 *) y, nb); break;
            case ORC_Q4_K: enc_q4_K(x, (blk_q4_K *) y, nb); break;
            case ORC_Q5_K: enc_q5_K(x, (blk_q5_K *) y, nb); break;
            case ORC_Q6_K: enc_q6_K(x, (blk_q6_K *) y, nb); break;
            case ORC_F16: orc_fp32_to_fp16_n(x, (uint16_t *) y, n_per_row); break;
            case ORC_F32: memcpy(y, x, rs); break;
            default: break;
        }
    }
    return rs * (size_t) nrows;
}

/* ------------------------------------------------------------------ activation quantizers */

/* The Q8_0 vec_dot_type conversion of ggml-cpu (quantize_row_q8_0). ORC_ACT_Q8_0_AVX2, the
 * canonical one (x86-64-v3 AVX2 build): d = amax/127, id = 127/amax, q = rint(x*id) (ties to
 * even). ORC_ACT_Q8_0_SCALAR: the generic path = the weight encoder (id = 1/d, roundf). */
void orc_quantize_act_q8_0(const float * x, void * yv, int64_t k, int variant) {
    blk_q8_0 * y = (blk_q8_0 *) yv;
    const int64_t nb = k / QK32;
    if (variant == ORC_ACT_Q8_0_SCALAR) {
        enc_q8_0(x, y, nb);
        return;
    }
    for (int64_t i = 0; i < nb; i++, x += QK32) {
        float amax = 0.0f;
        for (int j = 0; j < QK32; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK32; j++) y[i].qs[j] = (int8_t) lrintf(x[j] * id);
    }
}

/* ggml quantize_row_q8_K_ref: max = signed value of the (first) largest |x|, iscale = -127/max,
 * q = min(127, nearest_int(iscale*x)), d = 1/iscale (f32), bsums = sums of 16 codes. An all-zero
 * block stores d = 0 and zero codes and sums. */
void orc_quantize_act_q8_K(const float * x, void * yv, int64_t k) {
    blk_q8_K * y = (blk_q8_K *) yv;
    const int64_t nb = k / QKK;
    for (int64_t i = 0; i < nb; i++, x += QKK) {
        float max = 0, amax = 0;
        for (int j = 0; j < QKK; j++) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(blk_q8_K));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QKK; j++) {
            const int v = nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < QKK / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t) s;
        }
        y[i].d = 1 / iscale;
    }
}

/* ------------------------------------------------------------------------------ dequant */

/* ggml dequantize_row_q8_0 / q4_0 / q4_K / q5_K / q6_K. */
int orc_dequantize(int type, const void * src, float * dst, int64_t nrows, int64_t n_per_row) {
    const size_t rs = orc_row_size(type, n_per_row);
    if (!rs) return -1;
    for (int64_t r = 0; r < nrows; r++) {
        const uint8_t * row = (const uint8_t *) src + (size_t) r * rs;
        float * y = dst + r * n_per_row;
        if (type == ORC_Q8_0) {
            const blk_q8_0 * b = (const blk_q8_0 *) row;
            for (int64_t i = 0; i < n_per_row / QK32; i++) {
                const float d = orc_fp16_to_fp32(b[i].d);
                for (int j = 0; j < QK32; j++) y[i * QK32 + j] = b[i].qs[j] * d;
            }
        } else if (type == ORC_Q4_0) {
            const blk_q4_0 * b = (const blk_q4_0 *) row;
            for (int64_t i = 0; i < n_per_row / QK32; i++) {
                const float d = orc_fp16_to_fp32(b[i].d);
                for (int j = 0; j < QK32 / 2; j++) {
                    y[i * QK32 + j] = ((b[i].qs[j] & 0xF) - 8) * d;
                    y[i * QK32 + j + 16] = ((b[i].qs[j] >> 4) - 8) * d;
                }
            }
        } else if (type == ORC_Q4_K) {
            const blk_q4_K * b = (const blk_q4_K *) row;
            for (int64_t i = 0; i < n_per_row / QKK; i++) {
                const float d = orc_fp16_to_fp32(b[i].d), dmin = orc_fp16_to_fp32(b[i].dmin);
                const uint8_t * q = b[i].qs;
                float * o = y + i * QKK;
                for (int c = 0; c < 4; c++) {
                    uint8_t sc, m;
                    scale_min_k4(2 * c, b[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = dmin * m;
                    scale_min_k4(2 * c + 1, b[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = dmin * m;
                    for (int l = 0; l < 32; l++) o[64 * c + l] = d1 * (q[32 * c + l] & 0xF) - m1;
                    for (int l = 0; l < 32; l++) o[64 * c + 32 + l] = d2 * (q[32 * c + l] >> 4) - m2;
                }
            }
        } else if (type == ORC_Q5_K) {
            const blk_q5_K * b = (const blk_q5_K *) row;
            for (int64_t i = 0; i < n_per_row / QKK; i++) {
                const float d = orc_fp16_to_fp32(b[i].d), dmin = orc_fp16_to_fp32(b[i].dmin);
                float * o = y + i * QKK;
                for (int c = 0; c < 4; c++) {
                    uint8_t sc, m;
                    scale_min_k4(2 * c, b[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = dmin * m;
                    scale_min_k4(2 * c + 1, b[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = dmin * m;
                    const uint8_t * q = b[i].qs + 32 * c;
                    for (int l = 0; l < 32; l++)
                        o[64 * c + l] = d1 * ((q[l] & 0xF) + (b[i].qh[l] & (1u << (2 * c)) ? 16 : 0)) - m1;
                    for (int l = 0; l < 32; l++)
                        o[64 * c + 32 + l] = d2 * ((q[l] >> 4) + (b[i].qh[l] & (2u << (2 * c)) ? 16 : 0)) - m2;
                }
            }
        } else if (type == ORC_Q6_K) {
            const blk_q6_K * b = (const blk_q6_K *) row;
            for (int64_t i = 0; i < n_per_row / QKK; i++) {
                const float d = orc_fp16_to_fp32(b[i].d);
                for (int h = 0; h < 2; h++) {
                    const uint8_t * ql = b[i].ql + 64 * h;
                    const uint8_t * qh = b[i].qh + 32 * h;
                    const int8_t * sc = b[i].scales + 8 * h;
                    float * o = y + i * QKK + 128 * h;
                    for (int l = 0; l < 32; l++) {
                        const int is = l / 16;
                        const int q1 = (int) ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = (int) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        o[l] = d * sc[is + 0] * q1;
                        o[l + 32] = d * sc[is + 2] * q2;
                        o[l + 64] = d * sc[is + 4] * q3;
                        o[l + 96] = d * sc[is + 6] * q4;
                    }
                }
            }
        } else if (type == ORC_F16) {
            orc_fp16_to_fp32_n((const uint16_t *) row, y, n_per_row);
        } else if (type == ORC_F32) {
            memcpy(y, row, rs);
        } else {
            return -1;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- integer block dot sums */

/* ggml vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0 integer part: one sum per 32-block. */
static inline int32_t isum_q4_0(const blk_q4_0 * w, const blk_q8_0 * x) {
    int32_t s0 = 0, s1 = 0;
    for (int j = 0; j < 16; j++) {
        s0 += ((w->qs[j] & 0xF) - 8) * x->qs[j];
        s1 += ((w->qs[j] >> 4) - 8) * x->qs[j + 16];
    }
    return s0 + s1;
}

static inline int32_t isum_q8_0(const blk_q8_0 * w, const blk_q8_0 * x) {
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += w->qs[j] * x->qs[j];
    return s;
}

/* ggml vec_dot_q4_K_q8_K integer parts of one super-block: dot[j] = sum over sub-block j of
 * q4*q8, isc = sum_j sc_j*dot[j], imin = sum_j m_j*(bsums[2j] + bsums[2j+1]). */
static inline void isum_q4_K(const blk_q4_K * w, const blk_q8_K * x, int32_t dot[8], int32_t * isc, int32_t * imin) {
    *isc = 0;
    *imin = 0;
    for (int j = 0; j < 8; j++) {
        const int c = j / 2, hi = j & 1;
        int32_t s = 0;
        for (int l = 0; l < 32; l++) {
            const int q = hi ? (w->qs[32 * c + l] >> 4) : (w->qs[32 * c + l] & 0xF);
            s += q * x->qs[32 * j + l];
        }
        uint8_t sc, m;
        scale_min_k4(j, w->scales, &sc, &m);
        dot[j] = s;
        *isc += sc * s;
        *imin += m * (x->bsums[2 * j] + x->bsums[2 * j + 1]);
    }
}

/* ggml vec_dot_q5_K_q8_K integer parts: as Q4_K with q = nibble + 16 * (its qh bit). */
static inline void isum_q5_K(const blk_q5_K * w, const blk_q8_K * x, int32_t dot[8], int32_t * isc, int32_t * imin) {
    *isc = 0;
    *imin = 0;
    for (int j = 0; j < 8; j++) {
        const int c = j / 2, hi = j & 1;
        int32_t s = 0;
        for (int l = 0; l < 32; l++) {
            const int nib = hi ? (w->qs[32 * c + l] >> 4) : (w->qs[32 * c + l] & 0xF);
            const int q = nib + ((w->qh[l] >> j) & 1) * 16;
            s += q * x->qs[32 * j + l];
        }
        uint8_t sc, m;
        scale_min_k4(j, w->scales, &sc, &m);
        dot[j] = s;
        *isc += sc * s;
        *imin += m * (x->bsums[2 * j] + x->bsums[2 * j + 1]);
    }
}

/* ggml vec_dot_q6_K_q8_K integer parts: sub[j] = sum over 16-value sub-block j of (q - 32) * q8,
 * total = sum_j scales[j] * sub[j]. The 6-bit code of value v (half h = v / 128, r = v % 128,
 * l = r % 32, part p = r / 32) is ql[64h + 32(p & 1) + l] (low nibble for p < 2, high for
 * p >= 2) | ((qh[32h + l] >> 2p) & 3) << 4. */
static inline void isum_q6_K(const blk_q6_K * w, const blk_q8_K * x, int32_t sub[16], int32_t * total) {
    *total = 0;
    for (int j = 0; j < 16; j++) {
        int32_t s = 0;
        for (int t = 0; t < 16; t++) {
            const int v = 16 * j + t, h = v / 128, r = v % 128, p = r / 32, l = r % 32;
            const uint8_t b = w->ql[64 * h + 32 * (p & 1) + l];
            const int lo4 = p < 2 ? (b & 0xF) : (b >> 4);
            const int q = lo4 | (((w->qh[32 * h + l] >> (2 * p)) & 3) << 4);
            s += (q - 32) * x->qs[v];
        }
        sub[j] = s;
        *total += w->scales[j] * s;
    }
}

int64_t orc_block_isums(int type, const void * w_row, const void * xq_row, int64_t k, int32_t * out) {
    if (type == ORC_Q4_0 || type == ORC_Q8_0) {
        const int64_t nb = k / QK32;
        for (int64_t i = 0; i < nb; i++) {
            const blk_q8_0 * x = (const blk_q8_0 *) xq_row + i;
            out[i] = type == ORC_Q4_0 ? isum_q4_0((const blk_q4_0 *) w_row + i, x)
                                      : isum_q8_0((const blk_q8_0 *) w_row + i, x);
        }
        return nb;
    }
    if (type == ORC_Q4_K || type == ORC_Q5_K) {
        const int64_t nb = k / QKK;
        for (int64_t i = 0; i < nb; i++) {
            if (type == ORC_Q4_K)
                isum_q4_K((const blk_q4_K *) w_row + i, (const blk_q8_K *) xq_row + i, out + 10 * i, out + 10 * i + 8,
                          out + 10 * i + 9);
            else
                isum_q5_K((const blk_q5_K *) w_row + i, (const blk_q8_K *) xq_row + i, out + 10 * i, out + 10 * i + 8,
                          out + 10 * i + 9);
        }
        return 10 * nb;
    }
    if (type == ORC_Q6_K) {
        const int64_t nb = k / QKK;
        for (int64_t i = 0; i < nb; i++)
            isum_q6_K((const blk_q6_K *) w_row + i, (const blk_q8_K *) xq_row + i, out + 17 * i, out + 17 * i + 16);
        return 17 * nb;
    }
    return 0;
}

/* ------------------------------------------------------------------------------ mul_mat */

/* ggml_compute_forward_mul_mat for a quantized src0 and f32 src1 (runtime/src/ops.cpp:107-119):
 * src1 rows converted to the vec_dot_type, then per output the block dot with the fp32
 * epilogue sumf += isum * d_w * d_x (Q4_K, Q5_K: d*isc - dmin*imin with d = fp16(d_w)*d_x; Q6_K:
 * (fp16(d_w)*d_x) * sum_j sc_j*sub_j). */
int orc_mul_mat(int type, const void * w, int64_t N, int64_t K, const float * x, int64_t M, float * y,
                int n_threads) {
    const size_t wrs = orc_row_size(type, K);
    const int kq = type == ORC_Q4_K || type == ORC_Q5_K || type == ORC_Q6_K;
    if (!wrs || (type != ORC_Q4_0 && type != ORC_Q8_0 && !kq && type != ORC_F16 && type != ORC_F32)) return -1;
    const int xtype = kq ? ORC_Q8_K : (type == ORC_F16 || type == ORC_F32 ? ORC_F32 : ORC_Q8_0);
    const size_t xrs = orc_row_size(xtype, K);
    uint8_t * xq = (uint8_t *) malloc(xrs * (size_t) M);
    if (!xq) return -1;
    for (int64_t m = 0; m < M; m++) {
        if (xtype == ORC_Q8_0) orc_quantize_act_q8_0(x + m * K, xq + m * xrs, K, ORC_ACT_Q8_0_AVX2);
        else if (xtype == ORC_Q8_K) orc_quantize_act_q8_K(x + m * K, xq + m * xrs, K);
        else memcpy(xq + m * xrs, x + m * K, xrs);
    }
    const int nt = nthreads_of(n_threads);
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t n = 0; n < N; n++) {
        const uint8_t * wr = (const uint8_t *) w + (size_t) n * wrs;
        for (int64_t m = 0; m < M; m++) {
            const uint8_t * xr = xq + (size_t) m * xrs;
            float sumf = 0.0f;
            if (type == ORC_Q4_0) {
                const blk_q4_0 * wb = (const blk_q4_0 *) wr;
                const blk_q8_0 * xb = (const blk_q8_0 *) xr;
                for (int64_t i = 0; i < K / QK32; i++)
                    sumf += (float) isum_q4_0(wb + i, xb + i) * orc_fp16_to_fp32(wb[i].d) * orc_fp16_to_fp32(xb[i].d);
            } else if (type == ORC_Q8_0) {
                const blk_q8_0 * wb = (const blk_q8_0 *) wr;
                const blk_q8_0 * xb = (const blk_q8_0 *) xr;
                for (int64_t i = 0; i < K / QK32; i++)
                    sumf += (float) isum_q8_0(wb + i, xb + i) * orc_fp16_to_fp32(wb[i].d) * orc_fp16_to_fp32(xb[i].d);
            } else if (type == ORC_Q4_K) {
                const blk_q4_K * wb = (const blk_q4_K *) wr;
                const blk_q8_K * xb = (const blk_q8_K *) xr;
                for (int64_t i = 0; i < K / QKK; i++) {
                    int32_t dot[8], isc, imin;
                    isum_q4_K(wb + i, xb + i, dot, &isc, &imin);
                    const float d = orc_fp16_to_fp32(wb[i].d) * xb[i].d;
                    const float dmin = orc_fp16_to_fp32(wb[i].dmin) * xb[i].d;
                    sumf += d * (float) isc - dmin * (float) imin;
                }
            } else if (type == ORC_Q5_K) {
                const blk_q5_K * wb = (const blk_q5_K *) wr;
                const blk_q8_K * xb = (const blk_q8_K *) xr;
                for (int64_t i = 0; i < K / QKK; i++) {
                    int32_t dot[8], isc, imin;
                    isum_q5_K(wb + i, xb + i, dot, &isc, &imin);
                    const float d = orc_fp16_to_fp32(wb[i].d) * xb[i].d;
                    const float dmin = orc_fp16_to_fp32(wb[i].dmin) * xb[i].d;
                    sumf += d * (float) isc - dmin * (float) imin;
                }
            } else if (type == ORC_Q6_K) {
                const blk_q6_K * wb = (const blk_q6_K *) wr;
                const blk_q8_K * xb = (const blk_q8_K *) xr;
                for (int64_t i = 0; i < K / QKK; i++) {
                    int32_t sub[16], tot;
                    isum_q6_K(wb + i, xb + i, sub, &tot);
                    sumf += (orc_fp16_to_fp32(wb[i].d) * xb[i].d) * (float) tot;
                }
            } else {
                const float * xf = (const float *) xr;
                for (int64_t i = 0; i < K; i++) {
                    const float wv = type == ORC_F16 ? orc_fp16_to_fp32(((const uint16_t *) wr)[i]) : ((const float *) wr)[i];
                    sumf += wv * xf[i];
                }
            }
            y[m * N + n] = sumf;
        }
    }
    free(xq);
    return 0;
}

/* ------------------------------------------------------------------------------ rms_norm */

/* ggml_compute_forward_rms_norm_f32: sum of x*x in double, mean rounded to f32,
 * scale = 1/sqrtf(mean + eps), y = x * scale. */
void orc_rms_norm(const float * x, float * y, int64_t rows, int64_t n, float eps, int n_threads) {
    const int nt = nthreads_of(n_threads);
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t r = 0; r < rows; r++) {
        const float * xr = x + r * n;
        double sum = 0.0;
        for (int64_t i = 0; i < n; i++) sum += (double) (xr[i] * xr[i]);
        const float mean = (float) (sum / (double) n);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < n; i++) y[r * n + i] = xr[i] * scale;
    }
}

/* ------------------------------------------------------------------------------ rope */

/* ggml rope_f32 with mode NEOX and ext_factor 0 (runtime/src/ops.cpp:289-290 passes ext_factor
 * 0, beta_fast 32, beta_slow 1, which then do not matter): theta_scale = powf(base, -2/n_dims);
 * theta starts at the position and is multiplied by theta_scale once per pair (ggml's rope
 * cache); cos/sin of freq_scale*theta/ff times attn_factor rotate (x[i], x[i + n_dims/2]). */
void orc_rope_neox(const float * x, int64_t sx_s, int64_t sx_h, float * out, const int32_t * pos, int64_t D,
                   int64_t H, int64_t S, int n_dims, float freq_base, float freq_scale, float attn_factor,
                   const float * freq_factors) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    float * cache = (float *) malloc(sizeof(float) * (size_t) n_dims);
    for (int64_t s = 0; s < S; s++) {
        float theta = (float) pos[s];
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const float ff = freq_factors ? freq_factors[i0 / 2] : 1.0f;
            const float th = freq_scale * (theta / ff);
            cache[i0] = cosf(th) * attn_factor;
            cache[i0 + 1] = sinf(th) * attn_factor;
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < H; h++) {
            const float * xr = x + s * sx_s + h * sx_h;
            float * o = out + (s * H + h) * D;
            const int half = n_dims / 2;
            for (int i0 = 0; i0 < n_dims; i0 += 2) {
                const int ic = i0 / 2;
                const float c = cache[i0], sn = cache[i0 + 1];
                const float x0 = xr[ic], x1 = xr[ic + half];
                o[ic] = x0 * c - x1 * sn;
                o[ic + half] = x0 * sn + x1 * c;
            }
            for (int64_t i = n_dims; i < D; i++) o[i] = xr[i];
        }
    }
    free(cache);
}

/* ------------------------------------------------------------------------ flash attention */

/* ggml_compute_forward_flash_attn_ext_f16 for f16 K/V (runtime/include/ggml_compiler_ops.h:
 * 133-136, GGML_PREC_F32): Q rounded to f16 (K's vec_dot type), s = (K.Q)*scale + mask, keys
 * whose mask is -inf skipped, online softmax with running max M and sum S, output V-sum / S
 * (0 when no key was visible). The V accumulator is f32 here (ggml-cpu keeps it in f16 for f16
 * V; the 1e-3 tolerance of the parity tests covers that). */
void orc_flash_attn_ext(const float * q, int64_t q_h, int64_t q_s, const uint16_t * k, int64_t k_h, int64_t k_j,
                        const uint16_t * v, int64_t v_h, int64_t v_j, const uint16_t * mask, int64_t m_s, float * out,
                        int D, int Dv, int Sq, int H, int Hkv, int n_kv, float scale, int n_threads) {
    const int nt = nthreads_of(n_threads);
    const int rep = H / Hkv;
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt)
    for (int s = 0; s < Sq; s++) {
        for (int h = 0; h < H; h++) {
            float qh[1024], acc[1024], kr[1024];
            const float * qp = q + (int64_t) h * q_h + (int64_t) s * q_s;
            for (int d = 0; d < D; d++) qh[d] = orc_fp16_to_fp32(orc_fp32_to_fp16(qp[d]));
            for (int d = 0; d < Dv; d++) acc[d] = 0.0f;
            const int hk = h / rep;
            float M = -INFINITY, Ssum = 0.0f;
            for (int j = 0; j < n_kv; j++) {
                const float mv = mask ? orc_fp16_to_fp32(mask[(int64_t) s * m_s + j]) : 0.0f;
                if (mv == -INFINITY) continue;
                const uint16_t * kp = k + (int64_t) hk * k_h + (int64_t) j * k_j;
                for (int d = 0; d < D; d++) kr[d] = orc_fp16_to_fp32(kp[d]);
                float dot = 0.0f;
                for (int d = 0; d < D; d++) dot += kr[d] * qh[d];
                const float sc = dot * scale + mv;
                float ms = 1.0f, vs = 1.0f;
                if (sc > M) {
                    ms = expf(M - sc);
                    M = sc;
                    for (int d = 0; d < Dv; d++) acc[d] *= ms;
                } else {
                    vs = expf(sc - M);
                }
                const uint16_t * vp = v + (int64_t) hk * v_h + (int64_t) j * v_j;
                for (int d = 0; d < Dv; d++) acc[d] += orc_fp16_to_fp32(vp[d]) * vs;
                Ssum = Ssum * ms + vs;
            }
            const float inv = Ssum == 0.0f ? 0.0f : 1.0f / Ssum;
            float * o = out + ((int64_t) s * H + h) * Dv;
            for (int d = 0; d < Dv; d++) o[d] = acc[d] * inv;
        }
    }
}

/* ------------------------------------------------------------------------------ glue */

/* ggml_swiglu_split (runtime/src/ops.cpp:251-258): silu(g) * u, silu(v) = v / (1 + exp(-v)). */
void orc_swiglu(const float * g, const float * u, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* ggml_argmax over one row: the first index of the maximum. */
int orc_argmax(const float * x, int64_t n) {
    int best = 0;
    float bv = x[0];
    for (int64_t i = 1; i < n; i++) {
        if (x[i] > bv) {
            bv = x[i];
            best = (int) i;
        }
    }
    return best;
}
