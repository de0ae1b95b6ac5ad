/*
 * CPU oracle, part 1: scalar conversions, GGML block codecs, candle's CPU
 * activation quantizers and integer vec-dots, and the quantized matmul.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * The block formats are the GGML public spec as candle-core 0.11.0 stores
 * them (crate pinned at Cargo.lock:383-386, source not present in the
 * reference tree). Call sites in the reference:
 *   QTensor::dequantize   src/gguf_loader.rs:35-38, src/quantized_transformer.rs:68,108,110
 *   QMatMul::forward      src/quantized_transformer.rs:19-33 (via Linear)
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* scalar conversions                                                  */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oq_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oq_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? (0x200u | (m >> 13)) : 0u));
    int32_t he = (int32_t)e - 112; /* rebias 127 -> 15 */
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        uint32_t m24 = m | 0x800000u;
        uint32_t shift = (uint32_t)(14 - he);
        uint32_t q = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = sign | ((uint32_t)he << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float oq_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t oq_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

void oq_f32_to_bf16_n(const float *x, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; i++) out[i] = oq_f32_to_bf16(x[i]);
}

void oq_bf16_to_f32_n(const uint16_t *x, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = oq_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------ */
/* block layouts (GGML spec)                                           */
/* ------------------------------------------------------------------ */

#define QK8_0 32
#define QK_K 256

typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;               /* 34 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_k; /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6_k; /* 210 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[16]; } blk_q8_k; /* 292 B */

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 size");
_Static_assert(sizeof(blk_q4_k) == 144, "q4_k size");
_Static_assert(sizeof(blk_q6_k) == 210, "q6_k size");
_Static_assert(sizeof(blk_q8_k) == 292, "q8_k size");

int oq_block_size(int type) {
    switch (type) {
    case OQ_F32: case OQ_F16: case OQ_BF16: return 1;
    case OQ_Q8_0: return QK8_0;
    case OQ_Q4_K: case OQ_Q6_K: case OQ_Q8_K: return QK_K;
    default: return 0;
    }
}

int oq_block_bytes(int type) {
    switch (type) {
    case OQ_F32: return 4;
    case OQ_F16: case OQ_BF16: return 2;
    case OQ_Q8_0: return (int)sizeof(blk_q8_0);
    case OQ_Q4_K: return (int)sizeof(blk_q4_k);
    case OQ_Q6_K: return (int)sizeof(blk_q6_k);
    case OQ_Q8_K: return (int)sizeof(blk_q8_k);
    default: return 0;
    }
}

int64_t oq_row_bytes(int type, int64_t n) {
    int bs = oq_block_size(type);
    if (!bs || n % bs) return -1;
    return n / bs * oq_block_bytes(type);
}

/* Scale/min of Q4_K sub-block j from the 12 packed bytes (GGML spec:
 * 6-bit values; j < 4 in the low bits of bytes j / j+4, j >= 4 split between
 * a nibble of byte j+4 and the top two bits of byte j-4 / j). */
static inline void q4k_scale_min(int j, const uint8_t *s, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static inline int nearest(float x) { return (int)lrintf(x); }

/* ---- Q8_0 (candle BlockQ8_0::from_float / to_float) ---- */
static void quant_q8_0(const float *x, int64_t n, blk_q8_0 *y) {
    for (int64_t b = 0; b < n / QK8_0; b++) {
        const float *xs = x + b * QK8_0;
        float amax = 0.f;
        for (int i = 0; i < QK8_0; i++) amax = fmaxf(amax, fabsf(xs[i]));
        float d = amax / 127.f;
        float id = d != 0.f ? 1.f / d : 0.f;
        y[b].d = oq_f32_to_f16(d);
        for (int i = 0; i < QK8_0; i++) y[b].qs[i] = (int8_t)roundf(xs[i] * id);
    }
}

static void dequant_q8_0(const blk_q8_0 *x, int64_t n, float *y) {
    for (int64_t b = 0; b < n / QK8_0; b++) {
        float d = oq_f16_to_f32(x[b].d);
        for (int i = 0; i < QK8_0; i++) y[b * QK8_0 + i] = (float)x[b].qs[i] * d;
    }
}

/* ---- Q4_K ----
 * Dequant: y = d*sc_j*q - dmin*m_j; within each 64-value chunk c the first 32
 * values are the low nibbles of qs[32c..32c+32) (sub-block 2c), the next 32
 * the high nibbles (sub-block 2c+1). Both products are exact in f32, so the
 * one rounding is the subtraction.
 * The quantizer is a plain min/max fit used to generate test weights; it is
 * not on the measured path and any valid block is a legal input. */
static void quant_q4_k(const float *x, int64_t n, blk_q4_k *y) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *xs = x + b * QK_K;
        float scales[8], mins[8];
        for (int j = 0; j < 8; j++) {
            float mn = 0.f, mx = 0.f;
            for (int i = 0; i < 32; i++) {
                float v = xs[32 * j + i];
                if (i == 0 || v < mn) mn = v;
                if (i == 0 || v > mx) mx = v;
            }
            if (mn > 0.f) mn = 0.f;
            scales[j] = (mx - mn) / 15.f;
            mins[j] = -mn;
        }
        float max_scale = 0.f, max_min = 0.f;
        for (int j = 0; j < 8; j++) {
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        float inv_scale = max_scale > 0.f ? 63.f / max_scale : 0.f;
        float inv_min = max_min > 0.f ? 63.f / max_min : 0.f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            int a = nearest(inv_scale * scales[j]);
            int c = nearest(inv_min * mins[j]);
            ls[j] = (uint8_t)(a > 63 ? 63 : (a < 0 ? 0 : a));
            lm[j] = (uint8_t)(c > 63 ? 63 : (c < 0 ? 0 : c));
        }
        memset(y[b].scales, 0, 12);
        for (int j = 0; j < 8; j++) {
            if (j < 4) {
                y[b].scales[j] |= ls[j];
                y[b].scales[j + 4] |= lm[j];
            } else {
                y[b].scales[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
                y[b].scales[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
                y[b].scales[j] |= (uint8_t)((lm[j] >> 4) << 6);
            }
        }
        y[b].d = oq_f32_to_f16(max_scale / 63.f);
        y[b].dmin = oq_f32_to_f16(max_min / 63.f);
        uint8_t L[QK_K];
        float d = oq_f16_to_f32(y[b].d), dmin = oq_f16_to_f32(y[b].dmin);
        for (int j = 0; j < 8; j++) {
            int sc, m;
            q4k_scale_min(j, y[b].scales, &sc, &m);
            float ds = d * (float)sc, dm = dmin * (float)m;
            for (int i = 0; i < 32; i++) {
                int q = 0;
                if (ds != 0.f) q = nearest((xs[32 * j + i] + dm) / ds);
                L[32 * j + i] = (uint8_t)(q < 0 ? 0 : (q > 15 ? 15 : q));
            }
        }
        for (int c = 0; c < 4; c++)
            for (int i = 0; i < 32; i++)
                y[b].qs[32 * c + i] = (uint8_t)(L[64 * c + i] | (L[64 * c + 32 + i] << 4));
    }
}

static void dequant_q4_k(const blk_q4_k *x, int64_t n, float *y) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        float d = oq_f16_to_f32(x[b].d), dmin = oq_f16_to_f32(x[b].dmin);
        float *out = y + b * QK_K;
        for (int c = 0; c < 4; c++) {
            int sc0, m0, sc1, m1;
            q4k_scale_min(2 * c, x[b].scales, &sc0, &m0);
            q4k_scale_min(2 * c + 1, x[b].scales, &sc1, &m1);
            float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
            float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
            const uint8_t *q = x[b].qs + 32 * c;
            for (int i = 0; i < 32; i++) out[64 * c + i] = d0 * (float)(q[i] & 0xF) - mm0;
            for (int i = 0; i < 32; i++) out[64 * c + 32 + i] = d1 * (float)(q[i] >> 4) - mm1;
        }
    }
}

/* ---- Q6_K ----
 * Dequant: y = d*sc_j*(q-32), sub-blocks of 16. For each half h (128 values)
 * and l in [0,32): value 128h+l+32r (r=0..3) takes the low (r<2) or high (r>=2)
 * nibble of ql[64h + l + 32*(r&1)] and bits 2r..2r+1 of qh[32h + l]; its scale
 * index is 8h + l/16 + 2r. All products exact in f32.
 * The quantizer is a plain absmax fit used to generate test weights. */
static void quant_q6_k(const float *x, int64_t n, blk_q6_k *y) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *xs = x + b * QK_K;
        float sub[16];
        float max_scale = 0.f, max_abs_scale = 0.f;
        for (int j = 0; j < 16; j++) {
            float amax = 0.f, mx = 0.f;
            for (int i = 0; i < 16; i++) {
                float v = xs[16 * j + i];
                if (fabsf(v) > amax) { amax = fabsf(v); mx = v; }
            }
            sub[j] = amax > 0.f ? mx / -32.f : 0.f;
            if (fabsf(sub[j]) > max_abs_scale) { max_abs_scale = fabsf(sub[j]); max_scale = sub[j]; }
        }
        uint8_t L[QK_K];
        if (max_abs_scale == 0.f) {
            memset(y[b].ql, 0, 128);
            memset(y[b].qh, 0, 64);
            memset(y[b].scales, 0, 16);
            y[b].d = 0;
            continue;
        }
        float iscale = -128.f / max_scale;
        for (int j = 0; j < 16; j++) {
            int s = nearest(iscale * sub[j]);
            y[b].scales[j] = (int8_t)(s > 127 ? 127 : (s < -128 ? -128 : s));
        }
        y[b].d = oq_f32_to_f16(1.f / iscale);
        float d = oq_f16_to_f32(y[b].d);
        for (int j = 0; j < 16; j++) {
            float ds = d * (float)y[b].scales[j];
            for (int i = 0; i < 16; i++) {
                int q = 0;
                if (ds != 0.f) q = nearest(xs[16 * j + i] / ds);
                q = q < -32 ? -32 : (q > 31 ? 31 : q);
                L[16 * j + i] = (uint8_t)(q + 32);
            }
        }
        for (int h = 0; h < 2; h++) {
            for (int l = 0; l < 32; l++) {
                const uint8_t *Lh = L + 128 * h;
                y[b].ql[64 * h + l] = (uint8_t)((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
                y[b].ql[64 * h + l + 32] = (uint8_t)((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
                y[b].qh[32 * h + l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) |
                                                ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
            }
        }
    }
}

static inline int q6k_code(const blk_q6_k *x, int idx) {
    int h = idx / 128, w = idx % 128;
    int r = w / 32, l = w % 32;
    uint8_t qlb = x->ql[64 * h + l + 32 * (r & 1)];
    int lo = (r < 2) ? (qlb & 0xF) : (qlb >> 4);
    int hi = (x->qh[32 * h + l] >> (2 * r)) & 3;
    return (lo | (hi << 4)) - 32;
}

static inline int q6k_scale_index(int idx) {
    int h = idx / 128, w = idx % 128;
    int r = w / 32, l = w % 32;
    return 8 * h + l / 16 + 2 * r;
}

static void dequant_q6_k(const blk_q6_k *x, int64_t n, float *y) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        float d = oq_f16_to_f32(x[b].d);
        for (int i = 0; i < QK_K; i++) {
            float ds = d * (float)x[b].scales[q6k_scale_index(i)];
            y[b * QK_K + i] = ds * (float)q6k_code(&x[b], i);
        }
    }
}

/* ---- Q8_K activations (candle BlockQ8K::from_float) ----
 * iscale = -128 / (the value of largest magnitude), q = min(127, round(iscale*x)),
 * d = 1/iscale, bsums = sums of 16 codes. */
static void quant_q8_k(const float *x, int64_t n, blk_q8_k *y) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *xs = x + b * QK_K;
        float amax = 0.f, mx = 0.f;
        for (int i = 0; i < QK_K; i++)
            if (amax < fabsf(xs[i])) { amax = fabsf(xs[i]); mx = xs[i]; }
        if (amax == 0.f) {
            y[b].d = 0.f;
            memset(y[b].qs, 0, QK_K);
            memset(y[b].bsums, 0, sizeof(y[b].bsums));
            continue;
        }
        float iscale = -128.f / mx;
        for (int i = 0; i < QK_K; i++) {
            float v = roundf(iscale * xs[i]);
            y[b].qs[i] = (int8_t)(v > 127.f ? 127.f : v);
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += y[b].qs[16 * j + i];
            y[b].bsums[j] = (int16_t)s;
        }
        y[b].d = 1.f / iscale;
    }
}

static void dequant_q8_k(const blk_q8_k *x, int64_t n, float *y) {
    for (int64_t b = 0; b < n / QK_K; b++)
        for (int i = 0; i < QK_K; i++) y[b * QK_K + i] = x[b].d * (float)x[b].qs[i];
}

/* bf16 (round to nearest even) of a double, rounded once: frexp gives
 * v = f * 2^e with |f| in [0.5, 1); rint of f * 2^8 (the current rounding mode,
 * nearest even) keeps bf16's 8 significant bits. Values below the bf16
 * normal range round on its subnormal grid (spacing 2^-133). */
static uint16_t f64_to_bf16(double v) {
    if (v == 0.0) return 0u; /* a zero code: +0 whatever the scale's sign (the codes are integers) */
    double r;
    if (fabs(v) < 0x1p-126) {
        r = ldexp(rint(ldexp(v, 133)), -133);
    } else {
        int e;
        const double f = frexp(v, &e);
        r = ldexp(rint(f * 256.0), e - 8);
    }
    return oq_f32_to_bf16((float)r); /* r has <= 8 significant bits: exact in f32 and bf16 */
}

/* The bf16 MFMA operands of candle's activation rounding (QMatMul::forward,
 * src/quantized_transformer.rs:19-29 -> candle-core 0.11 BlockQ8_0 /
 * BlockQ8K::from_float): each row of k values quantized to the vec-dot type of
 * a wtype weight (Q8_0: 32-value blocks with an f16 scale; Q4_K / Q6_K: Q8_K
 * 256-value blocks with an f32 scale), then out = bf16(d * q) with d * q exact
 * in double and rounded once. */
int oq_quant_act_bf16(int wtype, const float *x, int64_t m, int64_t k, uint16_t *out) {
    const int kb = wtype == OQ_Q8_0 ? QK8_0 : (wtype == OQ_Q4_K || wtype == OQ_Q6_K) ? QK_K : 0;
    if (!kb || k % kb || m < 0) return -1;
    for (int64_t r = 0; r < m; r++) {
        const float *xr = x + r * k;
        uint16_t *o = out + r * k;
        for (int64_t b = 0; b < k / kb; b++) {
            if (kb == QK8_0) {
                blk_q8_0 y;
                quant_q8_0(xr + b * kb, kb, &y);
                const double d = oq_f16_to_f32(y.d);
                for (int i = 0; i < kb; i++) o[b * kb + i] = f64_to_bf16(d * y.qs[i]);
            } else {
                blk_q8_k y;
                quant_q8_k(xr + b * kb, kb, &y);
                for (int i = 0; i < kb; i++) o[b * kb + i] = f64_to_bf16((double)y.d * y.qs[i]);
            }
        }
    }
    return 0;
}

int oq_quantize(int type, const float *x, int64_t n, void *out) {
    int bs = oq_block_size(type);
    if (!bs || n % bs) return -1;
    switch (type) {
    case OQ_F32: memcpy(out, x, (size_t)n * 4); return 0;
    case OQ_F16: for (int64_t i = 0; i < n; i++) ((uint16_t *)out)[i] = oq_f32_to_f16(x[i]); return 0;
    case OQ_BF16: oq_f32_to_bf16_n(x, n, (uint16_t *)out); return 0;
    case OQ_Q8_0: quant_q8_0(x, n, (blk_q8_0 *)out); return 0;
    case OQ_Q4_K: quant_q4_k(x, n, (blk_q4_k *)out); return 0;
    case OQ_Q6_K: quant_q6_k(x, n, (blk_q6_k *)out); return 0;
    case OQ_Q8_K: quant_q8_k(x, n, (blk_q8_k *)out); return 0;
    default: return -1;
    }
}

int oq_dequantize(int type, const void *in, int64_t n, float *out) {
    int bs = oq_block_size(type);
    if (!bs || n % bs) return -1;
    switch (type) {
    case OQ_F32: memcpy(out, in, (size_t)n * 4); return 0;
    case OQ_F16: for (int64_t i = 0; i < n; i++) out[i] = oq_f16_to_f32(((const uint16_t *)in)[i]); return 0;
    case OQ_BF16: oq_bf16_to_f32_n((const uint16_t *)in, n, out); return 0;
    case OQ_Q8_0: dequant_q8_0((const blk_q8_0 *)in, n, out); return 0;
    case OQ_Q4_K: dequant_q4_k((const blk_q4_k *)in, n, out); return 0;
    case OQ_Q6_K: dequant_q6_k((const blk_q6_k *)in, n, out); return 0;
    case OQ_Q8_K: dequant_q8_k((const blk_q8_k *)in, n, out); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* quantized matmul                                                    */
/* ------------------------------------------------------------------ */

/* Weight row unpacked to int8 codes plus per-sub-block integer scales, so the
 * candle-mode vec-dots run as plain int8 loops. Lossless re-expression. */
typedef struct {
    int type;
    int64_t n, k;
    int8_t *codes;  /* [n][k]: Q8_0 q, Q4_K q (0..15), Q6_K q-32 */
    int16_t *isc;   /* Q4_K sc [n][k/32], Q6_K sc [n][k/16] */
    int16_t *imin;  /* Q4_K m  [n][k/32] */
    float *d;       /* Q8_0 d [n][k/32]; K-quants d [n][k/256] */
    float *dmin;    /* Q4_K dmin [n][k/256] */
} unpacked_w;

static void unpack_free(unpacked_w *u) {
    free(u->codes); free(u->isc); free(u->imin); free(u->d); free(u->dmin);
}

static int unpack_weights(int type, const void *w, int64_t n, int64_t k, unpacked_w *u) {
    memset(u, 0, sizeof(*u));
    u->type = type; u->n = n; u->k = k;
    u->codes = (int8_t *)malloc((size_t)(n * k));
    if (!u->codes) return -1;
    if (type == OQ_Q8_0) {
        u->d = (float *)malloc(sizeof(float) * (size_t)(n * k / 32));
        const blk_q8_0 *b = (const blk_q8_0 *)w;
#pragma omp parallel for
        for (int64_t r = 0; r < n; r++)
            for (int64_t j = 0; j < k / 32; j++) {
                const blk_q8_0 *x = &b[r * (k / 32) + j];
                u->d[r * (k / 32) + j] = oq_f16_to_f32(x->d);
                memcpy(u->codes + r * k + 32 * j, x->qs, 32);
            }
        return 0;
    }
    if (type == OQ_Q4_K) {
        u->isc = (int16_t *)malloc(sizeof(int16_t) * (size_t)(n * k / 32));
        u->imin = (int16_t *)malloc(sizeof(int16_t) * (size_t)(n * k / 32));
        u->d = (float *)malloc(sizeof(float) * (size_t)(n * k / 256));
        u->dmin = (float *)malloc(sizeof(float) * (size_t)(n * k / 256));
        const blk_q4_k *b = (const blk_q4_k *)w;
#pragma omp parallel for
        for (int64_t r = 0; r < n; r++)
            for (int64_t s = 0; s < k / 256; s++) {
                const blk_q4_k *x = &b[r * (k / 256) + s];
                u->d[r * (k / 256) + s] = oq_f16_to_f32(x->d);
                u->dmin[r * (k / 256) + s] = oq_f16_to_f32(x->dmin);
                for (int j = 0; j < 8; j++) {
                    int sc, m;
                    q4k_scale_min(j, x->scales, &sc, &m);
                    u->isc[r * (k / 32) + s * 8 + j] = (int16_t)sc;
                    u->imin[r * (k / 32) + s * 8 + j] = (int16_t)m;
                }
                int8_t *c = u->codes + r * k + s * 256;
                for (int ch = 0; ch < 4; ch++)
                    for (int i = 0; i < 32; i++) {
                        c[64 * ch + i] = (int8_t)(x->qs[32 * ch + i] & 0xF);
                        c[64 * ch + 32 + i] = (int8_t)(x->qs[32 * ch + i] >> 4);
                    }
            }
        return 0;
    }
    if (type == OQ_Q6_K) {
        u->isc = (int16_t *)malloc(sizeof(int16_t) * (size_t)(n * k / 16));
        u->d = (float *)malloc(sizeof(float) * (size_t)(n * k / 256));
        const blk_q6_k *b = (const blk_q6_k *)w;
#pragma omp parallel for
        for (int64_t r = 0; r < n; r++)
            for (int64_t s = 0; s < k / 256; s++) {
                const blk_q6_k *x = &b[r * (k / 256) + s];
                u->d[r * (k / 256) + s] = oq_f16_to_f32(x->d);
                for (int j = 0; j < 16; j++) u->isc[r * (k / 16) + s * 16 + j] = x->scales[j];
                int8_t *c = u->codes + r * k + s * 256;
                for (int i = 0; i < 256; i++) c[i] = (int8_t)q6k_code(x, i);
            }
        return 0;
    }
    free(u->codes);
    u->codes = NULL;
    return -1;
}

static inline int32_t dot_i8(const int8_t *a, const int8_t *b, int n) {
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

/* candle-mode vec-dot of one unpacked weight row with one quantized activation row. */
static float vdot_q8_0(const unpacked_w *u, int64_t r, const int8_t *xq, const float *xd) {
    const int8_t *wc = u->codes + r * u->k;
    const float *wd = u->d + r * (u->k / 32);
    float sumf = 0.f;
    for (int64_t j = 0; j < u->k / 32; j++) {
        int32_t si = dot_i8(wc + 32 * j, xq + 32 * j, 32);
        sumf += (float)si * wd[j] * xd[j];
    }
    return sumf;
}

static float vdot_q4_k(const unpacked_w *u, int64_t r, const int8_t *xq, const float *xd,
                       const int16_t *bsums) {
    const int8_t *wc = u->codes + r * u->k;
    const int16_t *sc = u->isc + r * (u->k / 32);
    const int16_t *mn = u->imin + r * (u->k / 32);
    float sumf = 0.f;
    for (int64_t s = 0; s < u->k / 256; s++) {
        int32_t isum = 0, msum = 0;
        for (int j = 0; j < 8; j++) {
            int32_t dj = dot_i8(wc + 256 * s + 32 * j, xq + 256 * s + 32 * j, 32);
            isum += (int32_t)sc[8 * s + j] * dj;
            msum += (int32_t)mn[8 * s + j] * ((int32_t)bsums[16 * s + 2 * j] + bsums[16 * s + 2 * j + 1]);
        }
        float d = u->d[r * (u->k / 256) + s] * xd[s];
        float dmin = u->dmin[r * (u->k / 256) + s] * xd[s];
        sumf += d * (float)isum - dmin * (float)msum;
    }
    return sumf;
}

static float vdot_q6_k(const unpacked_w *u, int64_t r, const int8_t *xq, const float *xd) {
    const int8_t *wc = u->codes + r * u->k;
    const int16_t *sc = u->isc + r * (u->k / 16);
    float sumf = 0.f;
    for (int64_t s = 0; s < u->k / 256; s++) {
        int32_t isum = 0;
        for (int j = 0; j < 16; j++)
            isum += (int32_t)sc[16 * s + j] * dot_i8(wc + 256 * s + 16 * j, xq + 256 * s + 16 * j, 16);
        sumf += u->d[r * (u->k / 256) + s] * xd[s] * (float)isum;
    }
    return sumf;
}

/* Exact-mode product y[m][n] = sum_k x[m][k] w[n][k] in f64. The product of
 * two f32 values is exact in f64, so only the additions round: each output
 * keeps four partial sums, lane l adding the terms k = l (mod 4) in increasing
 * k, and returns (s0 + s1) + (s2 + s3). That order depends on the output's own
 * row and column only, never on M, N or the tiling below, so a subset of rows
 * gives bit-identical outputs. Tiles of 32 x 32 outputs keep both operand
 * panels in the core's L2; 2 x 4 outputs share each operand load. */
typedef double v4d __attribute__((vector_size(32)));
typedef float v4f __attribute__((vector_size(16)));

static inline v4d ld4d(const float *p) {
    v4f f;
    memcpy(&f, p, sizeof(f));
    return __builtin_convertvector(f, v4d);
}

static inline float fin4(v4d a) { return (float)((a[0] + a[1]) + (a[2] + a[3])); }

static inline void tail4(v4d *acc, const float *xr, const float *wr, int64_t k4, int64_t K) {
    for (int64_t k = k4; k < K; k++) (*acc)[k - k4] += (double)xr[k] * (double)wr[k];
}

static void gemm_exact_f64(const float *x, int64_t M, const float *w, int64_t N, int64_t K, float *y) {
    const int64_t T = 32, k4 = K & ~(int64_t)3;
    const int64_t tm = (M + T - 1) / T, tn = (N + T - 1) / T;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t bi = 0; bi < tm; bi++)
        for (int64_t bj = 0; bj < tn; bj++) {
            const int64_t m0 = bi * T, m1 = m0 + T < M ? m0 + T : M;
            const int64_t n0 = bj * T, n1 = n0 + T < N ? n0 + T : N;
            for (int64_t m = m0; m < m1; m += 2) {
                const int two = m + 1 < m1;
                const float *x0 = x + m * K, *x1 = x + (two ? m + 1 : m) * K;
                int64_t n = n0;
                for (; n + 4 <= n1; n += 4) {
                    const float *w0 = w + n * K, *w1 = w0 + K, *w2 = w1 + K, *w3 = w2 + K;
                    v4d a00 = {0}, a01 = {0}, a02 = {0}, a03 = {0};
                    v4d a10 = {0}, a11 = {0}, a12 = {0}, a13 = {0};
                    for (int64_t k = 0; k < k4; k += 4) {
                        const v4d p0 = ld4d(x0 + k), p1 = ld4d(x1 + k);
                        const v4d q0 = ld4d(w0 + k), q1 = ld4d(w1 + k), q2 = ld4d(w2 + k), q3 = ld4d(w3 + k);
                        a00 += p0 * q0; a01 += p0 * q1; a02 += p0 * q2; a03 += p0 * q3;
                        a10 += p1 * q0; a11 += p1 * q1; a12 += p1 * q2; a13 += p1 * q3;
                    }
                    tail4(&a00, x0, w0, k4, K); tail4(&a01, x0, w1, k4, K);
                    tail4(&a02, x0, w2, k4, K); tail4(&a03, x0, w3, k4, K);
                    tail4(&a10, x1, w0, k4, K); tail4(&a11, x1, w1, k4, K);
                    tail4(&a12, x1, w2, k4, K); tail4(&a13, x1, w3, k4, K);
                    float *y0 = y + m * N + n;
                    y0[0] = fin4(a00); y0[1] = fin4(a01); y0[2] = fin4(a02); y0[3] = fin4(a03);
                    if (two) {
                        float *y1 = y0 + N;
                        y1[0] = fin4(a10); y1[1] = fin4(a11); y1[2] = fin4(a12); y1[3] = fin4(a13);
                    }
                }
                for (; n < n1; n++) {
                    const float *w0 = w + n * K;
                    v4d a0 = {0}, a1 = {0};
                    for (int64_t k = 0; k < k4; k += 4) {
                        const v4d q0 = ld4d(w0 + k);
                        a0 += ld4d(x0 + k) * q0;
                        a1 += ld4d(x1 + k) * q0;
                    }
                    tail4(&a0, x0, w0, k4, K);
                    tail4(&a1, x1, w0, k4, K);
                    y[m * N + n] = fin4(a0);
                    if (two) y[(m + 1) * N + n] = fin4(a1);
                }
            }
        }
}

int oq_qmatmul(int wtype, const void *w, int64_t N, int64_t K,
               const float *x, int64_t M, float *y, int mode) {
    int bs = oq_block_size(wtype);
    if (!bs || K % bs || M < 0 || N < 0) return -1;
    if (mode == OQ_MODE_EXACT || wtype == OQ_F32 || wtype == OQ_F16 || wtype == OQ_BF16) {
        /* Float-stored weights are a plain f32 matmul in candle
         * (src/quantized_transformer.rs:14-28); exact mode dequantizes any
         * type and accumulates in f64. */
        float *wf = (float *)malloc(sizeof(float) * (size_t)(N * K));
        if (!wf) return -2;
        oq_dequantize(wtype, w, N * K, wf);
        if (mode == OQ_MODE_EXACT) {
            gemm_exact_f64(x, M, wf, N, K, y);
            free(wf);
            return 0;
        }
#pragma omp parallel for collapse(2) schedule(static)
        for (int64_t m = 0; m < M; m++)
            for (int64_t n = 0; n < N; n++) {
                const float *xr = x + m * K, *wr = wf + n * K;
                float acc = 0.f;
                for (int64_t k = 0; k < K; k++) acc += xr[k] * wr[k];
                y[m * N + n] = acc;
            }
        free(wf);
        return 0;
    }
    unpacked_w u;
    if (unpack_weights(wtype, w, N, K, &u)) return -1;
    /* Activations quantized per row to the vec-dot type. */
    int8_t *xq = (int8_t *)malloc((size_t)(M * K));
    int kblk = wtype == OQ_Q8_0 ? 32 : 256;
    float *xd = (float *)malloc(sizeof(float) * (size_t)(M * (K / kblk)));
    int16_t *bsums = (int16_t *)malloc(sizeof(int16_t) * (size_t)(M * (K / 16)));
#pragma omp parallel for
    for (int64_t m = 0; m < M; m++) {
        if (wtype == OQ_Q8_0) {
            blk_q8_0 *tmp = (blk_q8_0 *)malloc(sizeof(blk_q8_0) * (size_t)(K / 32));
            quant_q8_0(x + m * K, K, tmp);
            for (int64_t j = 0; j < K / 32; j++) {
                memcpy(xq + m * K + 32 * j, tmp[j].qs, 32);
                xd[m * (K / 32) + j] = oq_f16_to_f32(tmp[j].d);
            }
            free(tmp);
        } else {
            blk_q8_k *tmp = (blk_q8_k *)malloc(sizeof(blk_q8_k) * (size_t)(K / 256));
            quant_q8_k(x + m * K, K, tmp);
            for (int64_t s = 0; s < K / 256; s++) {
                memcpy(xq + m * K + 256 * s, tmp[s].qs, 256);
                xd[m * (K / 256) + s] = tmp[s].d;
                memcpy(bsums + m * (K / 16) + 16 * s, tmp[s].bsums, 32);
            }
            free(tmp);
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const int8_t *q = xq + m * K;
            const float *d = xd + m * (K / kblk);
            float v;
            if (wtype == OQ_Q8_0) v = vdot_q8_0(&u, n, q, d);
            else if (wtype == OQ_Q4_K) v = vdot_q4_k(&u, n, q, d, bsums + m * (K / 16));
            else v = vdot_q6_k(&u, n, q, d);
            y[m * N + n] = v;
        }
    free(xq); free(xd); free(bsums);
    unpack_free(&u);
    return 0;
}

double oq_now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int oq_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
