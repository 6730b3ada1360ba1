/*
 * oracle/g4_oracle.c -- TEST INFRASTRUCTURE ONLY (see g4_oracle.h).
 *
 * CPU restatement of the decode-step hot path of thamada/Gemma4.c,
 * gemma4-4b/cpu-blas/main.c ("main.c" below).  Built with gcc -O3
 * -std=c11 -fopenmp (no -ffast-math, no FP contraction), the flags of the
 * reference's gemma4-4b/cpu-blas/Makefile:7-8.
 */
#define _POSIX_C_SOURCE 200809L
#include "g4_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================
 * scalar helpers
 * ====================================================================== */

/* main.c:128-149: exact binary16 -> binary32, subnormals included.  A
 * binary16 subnormal is man * 2^-24, which binary32 holds exactly. */
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u, man = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        float v = ldexpf((float)man, -24);
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (man << 13);
    }
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* main.c:151-156 */
float or_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* IEEE binary32 -> binary16, round to nearest even (synthetic generators). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* overflow -> inf */
    if (ax < 0x38800000u) {                                            /* subnormal / zero */
        if (ax < 0x33000000u) return (uint16_t)sign;                   /* < 2^-25 -> 0 */
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - (int)e;                                /* 14..24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 1023u);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

/* main.c:162-170: sub-block j's 6-bit scale and min from the 12 packed bytes. */
void or_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* main.c:373-380 / 490-495: the same unpack done on 32-bit words. */
void or_unpack_scales_words(const uint8_t s[12], uint8_t sc[8], uint8_t mn[8]) {
    uint32_t u[4];
    memcpy(u, s, 12);
    const uint32_t lo6 = 0x3f3f3f3fu, lo4 = 0x0f0f0f0fu, lo2 = 0x03030303u;
    u[3] = ((u[2] >> 4) & lo4) | (((u[1] >> 6) & lo2) << 4);
    const uint32_t mins_lo = u[1] & lo6;
    u[1] = (u[2] & lo4) | (((u[0] >> 6) & lo2) << 4);
    u[2] = mins_lo;
    u[0] &= lo6;
    memcpy(sc, &u[0], 8);
    memcpy(mn, &u[2], 8);
}

size_t or_block_bytes(int type) {
    switch (type) {
    case OR_Q4_K: return sizeof(or_q4K);
    case OR_Q5_K: return sizeof(or_q5K);
    case OR_Q6_K: return sizeof(or_q6K);
    default: return 0;
    }
}

/* ======================================================================
 * dequantizers, main.c:172-237
 * ====================================================================== */

void or_dequant_q4K(const or_q4K *x, float *y, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float d = or_f16_to_f32(x[b].d), dmin = or_f16_to_f32(x[b].dmin);
        const uint8_t *q = x[b].qs;
        for (int c = 0; c < 4; c++) {             /* 64 weights per chunk */
            uint8_t sc, m;
            or_scale_min_k4(2 * c, x[b].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            or_scale_min_k4(2 * c + 1, x[b].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (q[l] & 15) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
        }
    }
}

void or_dequant_q5K(const or_q5K *x, float *y, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float d = or_f16_to_f32(x[b].d), dmin = or_f16_to_f32(x[b].dmin);
        const uint8_t *q = x[b].qs, *qh = x[b].qh;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            or_scale_min_k4(2 * c, x[b].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            or_scale_min_k4(2 * c + 1, x[b].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            const uint8_t b1 = (uint8_t)(1u << (2 * c)), b2 = (uint8_t)(2u << (2 * c));
            for (int l = 0; l < 32; l++) *y++ = d1 * ((q[l] & 15) + ((qh[l] & b1) ? 16 : 0)) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * ((q[l] >> 4) + ((qh[l] & b2) ? 16 : 0)) - m2;
            q += 32;
        }
    }
}

/* q6 value of weight e (0..255) of a Q6_K block, already minus 32 */
static inline int q6_value(const or_q6K *x, int e) {
    const int h = e >> 7, r = e & 127, k = r >> 5, l = r & 31;
    const uint8_t qlb = x->ql[64 * h + 32 * (k & 1) + l];
    const uint8_t lo = (k < 2) ? (qlb & 15) : (qlb >> 4);
    const int hi = (x->qh[32 * h + l] >> (2 * k)) & 3;
    return (int)(lo | (hi << 4)) - 32;
}
/* scale index of weight e: main.c:221,226-229 (is = l/16, +2k, +8h) */
static inline int q6_scale_index(int e) {
    const int h = e >> 7, r = e & 127, k = r >> 5, l = r & 31;
    return 8 * h + (l >> 4) + 2 * k;
}

void or_dequant_q6K(const or_q6K *x, float *y, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float d = or_f16_to_f32(x[b].d);
        for (int e = 0; e < OR_QK_K; e++) {
            const int q = q6_value(&x[b], e);
            const int8_t sc = x[b].scales[q6_scale_index(e)];
            y[e] = d * sc * q;   /* (d * sc) * q, main.c:226 */
        }
        y += OR_QK_K;
    }
}

void or_dequant_block(const void *blk, int type, float *dst) {
    switch (type) {
    case OR_Q4_K: or_dequant_q4K((const or_q4K *)blk, dst, 1); break;
    case OR_Q5_K: or_dequant_q5K((const or_q5K *)blk, dst, 1); break;
    case OR_Q6_K: or_dequant_q6K((const or_q6K *)blk, dst, 1); break;
    default: break;
    }
}

/* ======================================================================
 * Q8_K quantization, main.c:247-279 (and its AVX2 twin 282-340, which
 * scans in the same order and rounds the same way)
 * ====================================================================== */

void or_quantize_q8K(const float *x, or_q8K *y, int k) {
    const int nb = k / OR_QK_K;
    for (int b = 0; b < nb; b++, x += OR_QK_K) {
        float amax = 0.0f, maxv = 0.0f;
        for (int j = 0; j < OR_QK_K; j++) {       /* first index of max |x| */
            const float a = fabsf(x[j]);
            if (a > amax) { amax = a; maxv = x[j]; }
        }
        if (amax == 0.0f) {
            memset(&y[b], 0, sizeof(or_q8K));
            continue;
        }
        const float iscale = -127.0f / maxv;
        for (int j = 0; j < OR_QK_K; j++) {
            const int v = (int)lrintf(iscale * x[j]);
            y[b].qs[j] = (int8_t)(v > 127 ? 127 : v);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += y[b].qs[16 * g + i];
            y[b].bsums[g] = (int16_t)s;
        }
        y[b].d = 1.0f / iscale;
    }
}

/* ======================================================================
 * per-block integer sums
 * ====================================================================== */

/* AVX2 lane partition, main.c:500-523: the madd of 32-byte chunks puts
 * bytes 4l..4l+3 of each chunk into int32 lane l. */
void or_q4K_lane_sums(const or_q4K *x, const or_q8K *y, int32_t sumi[8], int32_t prod[4]) {
    uint8_t sc[8], mn[8];
    or_unpack_scales_words(x->scales, sc, mn);
    for (int l = 0; l < 8; l++) {
        int32_t s = 0;
        for (int c = 0; c < 4; c++) {
            int32_t lo = 0, hi = 0;
            for (int t = 0; t < 4; t++) {
                const uint8_t q = x->qs[32 * c + 4 * l + t];
                lo += (q & 15) * y->qs[64 * c + 4 * l + t];
                hi += (q >> 4) * y->qs[64 * c + 32 + 4 * l + t];
            }
            s += sc[2 * c] * lo + sc[2 * c + 1] * hi;
        }
        sumi[l] = s;
    }
    for (int k = 0; k < 4; k++)
        prod[k] = mn[2 * k] * (y->bsums[4 * k] + y->bsums[4 * k + 1]) +
                  mn[2 * k + 1] * (y->bsums[4 * k + 2] + y->bsums[4 * k + 3]);
}

void or_q5K_lane_sums(const or_q5K *x, const or_q8K *y, int32_t sumi[8], int32_t prod[4]) {
    uint8_t sc[8], mn[8];
    or_unpack_scales_words(x->scales, sc, mn);
    for (int l = 0; l < 8; l++) {
        int32_t s = 0;
        for (int c = 0; c < 4; c++) {
            int32_t lo = 0, hi = 0;
            for (int t = 0; t < 4; t++) {
                const int i = 4 * l + t;
                const uint8_t q = x->qs[32 * c + i];
                const int h0 = (x->qh[i] >> (2 * c)) & 1, h1 = (x->qh[i] >> (2 * c + 1)) & 1;
                lo += ((q & 15) + 16 * h0) * y->qs[64 * c + i];
                hi += ((q >> 4) + 16 * h1) * y->qs[64 * c + 32 + i];
            }
            s += sc[2 * c] * lo + sc[2 * c + 1] * hi;
        }
        sumi[l] = s;
    }
    for (int k = 0; k < 4; k++)
        prod[k] = mn[2 * k] * (y->bsums[4 * k] + y->bsums[4 * k + 1]) +
                  mn[2 * k + 1] * (y->bsums[4 * k + 2] + y->bsums[4 * k + 3]);
}

void or_q4K_block_SM(const or_q4K *x, const or_q8K *y, int32_t *S, int32_t *M) {
    int32_t sumi[8], prod[4];
    or_q4K_lane_sums(x, y, sumi, prod);
    *S = sumi[0] + sumi[1] + sumi[2] + sumi[3] + sumi[4] + sumi[5] + sumi[6] + sumi[7];
    *M = prod[0] + prod[1] + prod[2] + prod[3];
}

void or_q5K_block_SM(const or_q5K *x, const or_q8K *y, int32_t *S, int32_t *M) {
    int32_t sumi[8], prod[4];
    or_q5K_lane_sums(x, y, sumi, prod);
    *S = sumi[0] + sumi[1] + sumi[2] + sumi[3] + sumi[4] + sumi[5] + sumi[6] + sumi[7];
    *M = prod[0] + prod[1] + prod[2] + prod[3];
}

int32_t or_q6K_block_S(const or_q6K *x, const or_q8K *y) {
    /* group-by-scale sum over all 256 weights (order-free integer math) */
    int32_t S = 0, acc[16] = {0};
    for (int e = 0; e < OR_QK_K; e++) acc[q6_scale_index(e)] += q6_value(x, e) * y->qs[e];
    for (int s = 0; s < 16; s++) S += x->scales[s] * acc[s];
    return S;
}

/* ======================================================================
 * dot products
 * ====================================================================== */

/* main.c:476-529: eight fp32 lanes accumulate d*sumi with FMA, four lanes
 * accumulate dmin*prod with FMA, then the fixed horizontal-add tree. */
float or_vec_dot_q4K_q8K(int n, const or_q4K *x, const or_q8K *y) {
    const int nb = n / OR_QK_K;
    float acc[8] = {0}, accm[4] = {0};
    for (int b = 0; b < nb; b++) {
        const float d = y[b].d * or_f16_to_f32(x[b].d);
        const float dmin = -y[b].d * or_f16_to_f32(x[b].dmin);
        int32_t sumi[8], prod[4];
        or_q4K_lane_sums(&x[b], &y[b], sumi, prod);
        for (int k = 0; k < 4; k++) accm[k] = fmaf(dmin, (float)prod[k], accm[k]);
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    const float h = ((acc[4] + acc[0]) + (acc[6] + acc[2])) + ((acc[5] + acc[1]) + (acc[7] + acc[3]));
    const float hm = (accm[0] + accm[2]) + (accm[1] + accm[3]);
    return h + hm;
}

/* main.c:531-593: as Q4_K, but the min term is one scalar, added with a
 * separate multiply (no contraction under -std=c11). */
float or_vec_dot_q5K_q8K(int n, const or_q5K *x, const or_q8K *y) {
    const int nb = n / OR_QK_K;
    float acc[8] = {0}, summs = 0.0f;
    for (int b = 0; b < nb; b++) {
        const float d = y[b].d * or_f16_to_f32(x[b].d);
        const float dmin = -y[b].d * or_f16_to_f32(x[b].dmin);
        int32_t sumi[8], prod[4];
        or_q5K_lane_sums(&x[b], &y[b], sumi, prod);
        const int32_t pm = (prod[0] + prod[1]) + (prod[2] + prod[3]);
        const float t = dmin * (float)pm;
        summs = summs + t;
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    const float h = ((acc[4] + acc[0]) + (acc[6] + acc[2])) + ((acc[5] + acc[1]) + (acc[7] + acc[3]));
    return h + summs;
}

/* main.c:347-407: lane l of aux32 collects elements e == l (mod 8);
 * sums[l] += d*aux32[l], sumf -= dmin*sumi, then sumf += sums[l]. */
static float generic_dot_tail(const int32_t aux32[8], int32_t sumi, float d, float dmin,
                              float sums[8], float sumf) {
    for (int l = 0; l < 8; l++) {
        const float t = d * (float)aux32[l];
        sums[l] = sums[l] + t;
    }
    const float t = dmin * (float)sumi;
    return sumf - t;
}

float or_vec_dot_q4K_q8K_generic(int n, const or_q4K *x, const or_q8K *y) {
    const int nb = n / OR_QK_K;
    float sums[8] = {0}, sumf = 0.0f;
    for (int b = 0; b < nb; b++) {
        uint8_t sc[8], mn[8];
        or_unpack_scales_words(x[b].scales, sc, mn);
        int32_t aux32[8] = {0}, sumi = 0;
        for (int g = 0; g < 16; g++) sumi += y[b].bsums[g] * mn[g / 2];
        for (int e = 0; e < OR_QK_K; e++) {
            const int c = e >> 6, r = e & 63;
            const uint8_t q = x[b].qs[32 * c + (r & 31)];
            const int v = (r < 32) ? (q & 15) : (q >> 4);
            aux32[e & 7] += sc[e >> 5] * (v * y[b].qs[e]);
        }
        const float d = or_f16_to_f32(x[b].d) * y[b].d;
        const float dmin = or_f16_to_f32(x[b].dmin) * y[b].d;
        sumf = generic_dot_tail(aux32, sumi, d, dmin, sums, sumf);
    }
    for (int l = 0; l < 8; l++) sumf = sumf + sums[l];
    return sumf;
}

float or_vec_dot_q5K_q8K_generic(int n, const or_q5K *x, const or_q8K *y) {
    const int nb = n / OR_QK_K;
    float sums[8] = {0}, sumf = 0.0f;
    for (int b = 0; b < nb; b++) {
        uint8_t sc[8], mn[8];
        or_unpack_scales_words(x[b].scales, sc, mn);
        int32_t aux32[8] = {0}, sumi = 0;
        for (int g = 0; g < 16; g++) sumi += y[b].bsums[g] * mn[g / 2];
        for (int e = 0; e < OR_QK_K; e++) {
            const int c = e >> 6, r = e & 63, l = r & 31;
            const uint8_t q = x[b].qs[32 * c + l];
            const int hb = (x[b].qh[l] >> (2 * c + (r >= 32))) & 1;
            const int v = ((r < 32) ? (q & 15) : (q >> 4)) + 16 * hb;
            aux32[e & 7] += sc[e >> 5] * (v * y[b].qs[e]);
        }
        const float d = or_f16_to_f32(x[b].d) * y[b].d;
        const float dmin = or_f16_to_f32(x[b].dmin) * y[b].d;
        sumf = generic_dot_tail(aux32, sumi, d, dmin, sums, sumf);
    }
    for (int l = 0; l < 8; l++) sumf = sumf + sums[l];
    return sumf;
}

/* No reference counterpart (the reference sends Q6_K through the fp32
 * path).  Defined here as: acc = fmaf(fp16(d) * y.d, (float)S_b, acc)
 * over the blocks in order. */
float or_vec_dot_q6K_q8K(int n, const or_q6K *x, const or_q8K *y) {
    const int nb = n / OR_QK_K;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const float d = or_f16_to_f32(x[b].d) * y[b].d;
        acc = fmaf(d, (float)or_q6K_block_S(&x[b], &y[b]), acc);
    }
    return acc;
}

float or_vec_dot_row_q8K(int n, const void *row, int type, const or_q8K *q8) {
    switch (type) {
    case OR_Q4_K: return or_vec_dot_q4K_q8K(n, (const or_q4K *)row, q8);
    case OR_Q5_K: return or_vec_dot_q5K_q8K(n, (const or_q5K *)row, q8);
    case OR_Q6_K: return or_vec_dot_q6K_q8K(n, (const or_q6K *)row, q8);
    default: return NAN;
    }
}

/* ======================================================================
 * GEMV
 * ====================================================================== */

/* main.c:1539-1556: per row, dequantize each block and accumulate x*w into
 * one sequential fp32 sum. */
void or_mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type) {
    const int nb = n / OR_QK_K;
    const size_t bs = or_block_bytes(type), row_sz = (size_t)nb * bs;
    const uint8_t *wb = (const uint8_t *)w;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) {
        float blk[OR_QK_K];
        float val = 0.0f;
        const uint8_t *row = wb + (size_t)i * row_sz;
        for (int b = 0; b < nb; b++) {
            or_dequant_block(row + (size_t)b * bs, type, blk);
            const float *xp = x + (size_t)b * OR_QK_K;
            for (int j = 0; j < OR_QK_K; j++) {
                const float t = xp[j] * blk[j];
                val = val + t;
            }
        }
        o[i] = val;
    }
}

/* main.c:1558-1566 */
void or_mm_quant_dot_rows(float *o, const void *w, int n, int d, int type, const or_q8K *q8) {
    const size_t row_sz = (size_t)(n / OR_QK_K) * or_block_bytes(type);
    const uint8_t *wb = (const uint8_t *)w;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) o[i] = or_vec_dot_row_q8K(n, wb + (size_t)i * row_sz, type, q8);
}

void or_mm_q6K_q8K_rows(float *o, const void *w, int n, int d, const or_q8K *q8) {
    or_mm_quant_dot_rows(o, w, n, d, OR_Q6_K, q8);
}

/* main.c:1529-1537 */
void or_mm_bf16(float *o, const float *x, const uint16_t *w, int n, int d) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) {
        const uint16_t *row = w + (size_t)i * n;
        float val = 0.0f;
        for (int j = 0; j < n; j++) {
            const float t = x[j] * or_bf16_to_f32(row[j]);
            val = val + t;
        }
        o[i] = val;
    }
}

/* main.c:1519-1527 */
void or_mm_f16(float *o, const float *x, const uint16_t *w, int n, int d) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) {
        const uint16_t *row = w + (size_t)i * n;
        float val = 0.0f;
        for (int j = 0; j < n; j++) {
            const float t = x[j] * or_f16_to_f32(row[j]);
            val = val + t;
        }
        o[i] = val;
    }
}

/* main.c:1494-1517 calls cblas_sgemv; its summation order is OpenBLAS's
 * (absent here).  This is the textbook row-major GEMV. */
void or_mm_f32(float *o, const float *x, const float *w, int n, int d) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) {
        const float *row = w + (size_t)i * n;
        float val = 0.0f;
        for (int j = 0; j < n; j++) {
            const float t = row[j] * x[j];
            val = val + t;
        }
        o[i] = val;
    }
}

/* the --f32-matmul switch, main.c:1568 (set by main.c:2736) */
static int or_f32_matmul = 0;
void or_set_f32_matmul(int on) { or_f32_matmul = on != 0; }

/* main.c:1669-1694 */
int or_mm(float *o, const float *x, const void *w, int n, int d, int type, or_q8K *q8, int q8_ready) {
    switch (type) {
    case OR_F32: or_mm_f32(o, x, (const float *)w, n, d); return 0;
    case OR_F16: or_mm_f16(o, x, (const uint16_t *)w, n, d); return 0;
    case OR_BF16: or_mm_bf16(o, x, (const uint16_t *)w, n, d); return 0;
    case OR_Q4_K:
    case OR_Q5_K:
        if (n % OR_QK_K) return -1;
        if (or_f32_matmul) {
            or_mm_quant_rows(o, x, w, n, d, type);
            return 0;
        }
        if (!q8_ready) or_quantize_q8K(x, q8, n);
        or_mm_quant_dot_rows(o, w, n, d, type, q8);
        return 0;
    case OR_Q6_K:
        if (n % OR_QK_K) return -1;
        or_mm_quant_rows(o, x, w, n, d, type);
        return 0;
    default:
        return -1;
    }
}

/* ======================================================================
 * step glue
 * ====================================================================== */

/* main.c:1451-1456: o = (x * s) * w */
void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) {
        const float t = x[i] * x[i];
        ss = ss + t;
    }
    ss = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * ss * w[i];
}

/* main.c:1458-1466: v = v * (s * w) */
void or_rmsnorm_head_inplace(float *v, const float *w, int n_heads, int hd, float eps) {
    for (int h = 0; h < n_heads; h++) {
        float *seg = v + (size_t)h * hd;
        float ss = 0.0f;
        for (int i = 0; i < hd; i++) {
            const float t = seg[i] * seg[i];
            ss = ss + t;
        }
        ss = 1.0f / sqrtf(ss / (float)hd + eps);
        for (int i = 0; i < hd; i++) seg[i] = seg[i] * (ss * w[i]);
    }
}

/* main.c:1468-1476 */
void or_rmsnorm_head_noweight_inplace(float *v, int n_heads, int hd, float eps) {
    for (int h = 0; h < n_heads; h++) {
        float *seg = v + (size_t)h * hd;
        float ss = 0.0f;
        for (int i = 0; i < hd; i++) {
            const float t = seg[i] * seg[i];
            ss = ss + t;
        }
        ss = 1.0f / sqrtf(ss / (float)hd + eps);
        for (int i = 0; i < hd; i++) seg[i] = seg[i] * ss;
    }
}

/* main.c:1478-1488 */
void or_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum = sum + x[i];
    }
    for (int i = 0; i < n; i++) x[i] = x[i] / sum;
}

/* main.c:1490-1492, tanh form; the operation order is the reference's */
float or_gelu(float x) {
    const float inner = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* main.c:1725-1745: Neox pairs (j, j+hd/2); the angle of pair j is pos
 * multiplied j times by ts = base^(-2/n_rot), one rounding per step. */
void or_apply_rope_neox(float *vec, int n_heads, int head_dim, int n_rot, int pos,
                        float freq_base, float freq_scale, const float *freq_factors) {
    const float ts = powf(freq_base, -2.0f / (float)n_rot);
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float *seg = vec + (size_t)h * head_dim;
        float theta = (float)pos;
        for (int j = 0; j < n_rot / 2; j++) {
            const float ff = freq_factors ? freq_factors[j] : 1.0f;
            const float angle = freq_scale * theta / ff;
            const float c = cosf(angle), s = sinf(angle);
            const float a = seg[j], b = seg[j + half];
            seg[j] = a * c - b * s;
            seg[j + half] = a * s + b * c;
            theta = theta * ts;
        }
    }
}

/* main.c:1696-1723 */
int or_emb_lookup(float *o, const void *w, int type, int id, int dim) {
    switch (type) {
    case OR_F32:
        memcpy(o, (const float *)w + (size_t)id * dim, (size_t)dim * sizeof(float));
        return 0;
    case OR_F16: {
        const uint16_t *row = (const uint16_t *)w + (size_t)id * dim;
        for (int i = 0; i < dim; i++) o[i] = or_f16_to_f32(row[i]);
        return 0;
    }
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: {
        const int nb = dim / OR_QK_K;
        const size_t bs = or_block_bytes(type);
        const uint8_t *row = (const uint8_t *)w + (size_t)id * nb * bs;
        for (int b = 0; b < nb; b++) or_dequant_block(row + (size_t)b * bs, type, o + (size_t)b * OR_QK_K);
        return 0;
    }
    default:
        return -1;
    }
}

/* ======================================================================
 * attention block, main.c:1909-1950 (sgemv NoTrans -> softmax -> sgemv Trans)
 * ====================================================================== */

void or_attn_decode(const float *q, const float *kc, const float *vc, int kv_stride,
                    int t_start, int nwin, int n_heads, int n_kv, int hd,
                    float attn_scale, float *att, float *out) {
    const int kv_mul = n_heads / n_kv;
    const int tlen = t_start + nwin;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const float *qh = q + (size_t)h * hd;
        const int kvh = h / kv_mul;
        float *a = att + (size_t)h * tlen;
        float *oh = out + (size_t)h * hd;
        for (int t = 0; t < t_start; t++) a[t] = 0.0f;
        if (nwin <= 0) {
            memset(oh, 0, (size_t)hd * sizeof(float));
            continue;
        }
        for (int t = t_start; t < tlen; t++) {
            const float *kr = kc + (size_t)t * kv_stride + (size_t)kvh * hd;
            float s = 0.0f;
            for (int i = 0; i < hd; i++) {
                const float p = kr[i] * qh[i];
                s = s + p;
            }
            a[t] = attn_scale * s;
        }
        or_softmax(a + t_start, nwin);
        for (int i = 0; i < hd; i++) oh[i] = 0.0f;
        for (int t = t_start; t < tlen; t++) {
            const float *vr = vc + (size_t)t * kv_stride + (size_t)kvh * hd;
            const float p = a[t];
            for (int i = 0; i < hd; i++) {
                const float m = p * vr[i];
                oh[i] = oh[i] + m;
            }
        }
    }
}

/* ======================================================================
 * sampler, main.c:2035-2126
 * ====================================================================== */

float or_rng_f32(uint64_t *state) {
    *state ^= *state >> 12;
    *state ^= *state << 25;
    *state ^= *state >> 27;
    return (float)((*state * 0x2545F4914F6CDD1DULL) >> 40) / (float)(1 << 24);
}

/* main.c:2045-2049: first index wins ties */
int or_argmax_first(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

typedef struct { float p; int idx; } or_prob_idx;

/* main.c:2044-2112: insertion top-k (stable for equal values), temperature
 * softmax, then plain or top-p draw from the xorshift64* stream. */
int or_sample_token(const float *logits, int n, float temp, float topp, int topk, uint64_t *rng) {
    if (temp <= 0.0f) return or_argmax_first(logits, n);
    if (topk <= 0 || topk > n) topk = n;
    or_prob_idx *pi = (or_prob_idx *)malloc((size_t)topk * sizeof(or_prob_idx));
    int np = 0;
    for (int i = 0; i < n; i++) {
        const float v = logits[i];
        int j;
        if (np < topk) j = np++;
        else if (v > pi[np - 1].p) j = np - 1;
        else continue;
        while (j > 0 && pi[j - 1].p < v) { pi[j] = pi[j - 1]; j--; }
        pi[j].p = v;
        pi[j].idx = i;
    }
    const float mx = pi[0].p;
    float sum = 0.0f;
    for (int i = 0; i < np; i++) {
        pi[i].p = expf((pi[i].p - mx) / temp);
        sum = sum + pi[i].p;
    }
    for (int i = 0; i < np; i++) pi[i].p = pi[i].p / sum;
    const float coin = or_rng_f32(rng);
    int result;
    if (topp <= 0.0f || topp >= 1.0f) {
        float cdf = 0.0f;
        result = pi[np - 1].idx;
        for (int i = 0; i < np; i++) {
            cdf = cdf + pi[i].p;
            if (coin < cdf) { result = pi[i].idx; break; }
        }
    } else {
        float cum = 0.0f;
        int last = np - 1;
        for (int i = 0; i < np; i++) {
            cum = cum + pi[i].p;
            if (cum > topp) { last = i; break; }
        }
        const float r = or_rng_f32(rng) * cum;
        float cdf = 0.0f;
        result = pi[last].idx;
        for (int i = 0; i <= last; i++) {
            cdf = cdf + pi[i].p;
            if (r < cdf) { result = pi[i].idx; break; }
        }
    }
    free(pi);
    return result;
}

/* main.c:2114-2126: each of the last penalty_last_n generated tokens (all of
 * them when penalty_last_n <= 0) divides a non-negative logit by the penalty
 * or multiplies a negative one, once per occurrence, in history order. */
void or_apply_repetition_penalty(float *logits, const int *tokens, int n_tokens, float penalty, int penalty_last_n) {
    if (penalty <= 1.0f || !tokens || n_tokens <= 0) return;
    const int start = penalty_last_n > 0 && n_tokens > penalty_last_n ? n_tokens - penalty_last_n : 0;
    for (int i = start; i < n_tokens; i++) {
        const int id = tokens[i];
        if (id < 0) continue;
        logits[id] = logits[id] >= 0.0f ? logits[id] / penalty : logits[id] * penalty;
    }
}

/* main.c:1814-1827 */
void or_hidden_stats(const float *v, int n, float *sum, float *l2, float *amax) {
    double s = 0.0, q = 0.0;
    float a = 0.0f;
    for (int i = 0; i < n; i++) {
        const float x = v[i];
        s += x;
        q += (double)x * x;
        const float ax = x >= 0.0f ? x : -x;
        if (ax > a) a = ax;
    }
    *sum = (float)s;
    *l2 = (float)sqrt(q);
    *amax = a;
}

/* ======================================================================
 * model: GGUF image -> weights -> forward()
 * ====================================================================== */

typedef struct { const void *p; int type; uint64_t ne[4]; int n_dims; } or_tensor;

struct or_model {
    /* config, main.c:623-629 and defaults main.c:854-871 */
    int dim, hidden, n_layers, n_heads, n_kv, vocab, max_seq, ple_dim, window, shared_kv;
    int swa_pattern, hd_swa, hd_full, rot_swa, rot_full;
    float theta, theta_swa, eps, softcap;
    int *swa_layers;
    int eos;
    /* weights, main.c:668-692 */
    or_tensor embd, ple_tok, ple_proj;
    const float *ple_proj_norm, *rope_freqs, *norm_out;
    const float **attn_norm, **post_attn_norm, **ffn_norm, **post_ffw_norm, **q_norm, **k_norm,
                **post_norm, **out_scale;
    or_tensor *wq, *wk, *wv, *wo, *gate, *up, *down, *inp_gate, *proj;
    /* state, main.c:694-701 */
    float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *att, *logits, *q_out, *ple, *ple_ctx, *ple_gate;
    float *kc, *vc;
    or_q8K *q8;
    float *stats; /* n_layers*3 + 8 */
    float *astats; /* n_layers*3: hidden_stats of x after each layer's attention residual (main.c:1964-1969) */
    float *layer_x; /* n_layers*dim: x after each layer of the last forward */
    /* Q8_K activations of the five quantization points of every layer
     * (OR_Q8_SLOT_*): q8_rec records the oracle's own quantize_row_q8_K
     * results of the last forward; q8_inj (borrowed, NULL unless
     * or_forward_inject_q8 runs) replaces them before use */
    or_q8K *q8_rec;
    const or_q8K *q8_inj;
    /* layer-0 dump_kv_fingerprint records of the last forward (OR_FP_*):
     * sum, l2, max, v0..v3 */
    float fp[OR_FP_TAGS * 7];
    int fp_have[OR_FP_TAGS];
};

/* dump_kv_fingerprint (main.c:1829-1836) into tag t */
static void fp_tag(or_model *m, int t, const float *v, int n) {
    or_hidden_stats(v, n, &m->fp[7 * t], &m->fp[7 * t + 1], &m->fp[7 * t + 2]);
    for (int i = 0; i < 4; i++) m->fp[7 * t + 3 + i] = i < n ? v[i] : 0.0f;
    m->fp_have[t] = 1;
}

typedef struct { const uint8_t *d; uint64_t p, size; int bad; } or_rd;

static uint32_t rd_u32(or_rd *r) {
    uint32_t v = 0;
    if (r->p + 4 > r->size) { r->bad = 1; return 0; }
    memcpy(&v, r->d + r->p, 4); r->p += 4; return v;
}
static uint64_t rd_u64(or_rd *r) {
    uint64_t v = 0;
    if (r->p + 8 > r->size) { r->bad = 1; return 0; }
    memcpy(&v, r->d + r->p, 8); r->p += 8; return v;
}
static const char *rd_str(or_rd *r, uint64_t *len) {
    *len = rd_u64(r);
    if (r->bad || r->p + *len > r->size) { r->bad = 1; *len = 0; return ""; }
    const char *s = (const char *)(r->d + r->p);
    r->p += *len;
    return s;
}
static int key_is(const char *k, uint64_t kl, const char *lit) {
    return strlen(lit) == kl && memcmp(k, lit, kl) == 0;
}
/* value readers, main.c:798-839 */
static void rd_skip(or_rd *r, uint32_t t) {
    static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (r->bad) return;
    if (t == 8) { uint64_t l; rd_str(r, &l); return; }
    if (t == 9) {
        uint32_t et = rd_u32(r); uint64_t n = rd_u64(r);
        if (et != 8 && et != 9 && et <= 12) {
            if (r->p + n * (uint64_t)sz[et] > r->size) { r->bad = 1; return; }
            r->p += n * (uint64_t)sz[et];
        } else {
            for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip(r, et);
        }
        return;
    }
    if (t > 12) { r->bad = 1; return; }
    if (r->p + (uint64_t)sz[t] > r->size) { r->bad = 1; return; }
    r->p += (uint64_t)sz[t];
}
static double rd_num(or_rd *r, uint32_t t) {
    double v = 0;
    if (r->bad) return 0;
    const uint8_t *s = r->d + r->p;
    switch (t) {
    case 0: case 7: v = s[0]; r->p += 1; break;
    case 1: v = (int8_t)s[0]; r->p += 1; break;
    case 2: { uint16_t x; memcpy(&x, s, 2); v = x; r->p += 2; break; }
    case 3: { int16_t x; memcpy(&x, s, 2); v = x; r->p += 2; break; }
    case 4: { uint32_t x; memcpy(&x, s, 4); v = x; r->p += 4; break; }
    case 5: { int32_t x; memcpy(&x, s, 4); v = x; r->p += 4; break; }
    case 6: { float x; memcpy(&x, s, 4); v = x; r->p += 4; break; }
    case 10: { uint64_t x; memcpy(&x, s, 8); v = (double)x; r->p += 8; break; }
    case 11: { int64_t x; memcpy(&x, s, 8); v = (double)x; r->p += 8; break; }
    case 12: { double x; memcpy(&x, s, 8); v = x; r->p += 8; break; }
    default: rd_skip(r, t); break;
    }
    return v;
}

static int is_swa(const or_model *m, int l) {      /* main.c:716-721 */
    if (m->swa_layers && l >= 0 && l < m->n_layers) return m->swa_layers[l];
    if (m->swa_pattern <= 0) return 0;
    return (l % m->swa_pattern) < (m->swa_pattern - 1);
}
static int layer_hd(const or_model *m, int l) { return is_swa(m, l) ? m->hd_swa : m->hd_full; }
static int kv_source(const or_model *m, int l) {    /* main.c:739-746 */
    if (l < OR_N_LAYER_KV) return l;
    return is_swa(m, l) ? 22 : 23;
}

typedef struct { const char *name; uint64_t nl; int n_dims; uint64_t ne[4]; int type; uint64_t off; } or_tinfo;

static int find_t(const or_tinfo *ti, int nt, const uint8_t *base, const char *name, or_tensor *out) {
    for (int i = 0; i < nt; i++) {
        if (key_is(ti[i].name, ti[i].nl, name)) {
            out->p = base + ti[i].off;
            out->type = ti[i].type;
            out->n_dims = ti[i].n_dims;
            memcpy(out->ne, ti[i].ne, sizeof(out->ne));
            return 1;
        }
    }
    memset(out, 0, sizeof(*out));
    return 0;
}

static void set_err(char *err, size_t n, const char *msg) {
    if (err && n) snprintf(err, n, "%s", msg);
}

or_model *or_model_open(const uint8_t *data, size_t size, int max_seq, char *err, size_t errlen) {
    or_rd r = {data, 0, size, 0};
    if (rd_u32(&r) != 0x46554747u) { set_err(err, errlen, "invalid GGUF magic"); return NULL; }
    rd_u32(&r);
    const uint64_t n_t = rd_u64(&r), n_kv = rd_u64(&r);
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    /* defaults, main.c:854-871 */
    m->theta = 1e6f; m->theta_swa = 10000.0f; m->eps = 1e-6f; m->max_seq = 8192;
    m->swa_pattern = 6; m->hd_swa = 256; m->hd_full = 512; m->rot_swa = 256; m->rot_full = 512;
    m->ple_dim = 256; m->window = 512; m->shared_kv = 18; m->softcap = 30.0f; m->eos = 106;
    uint32_t align = 32;
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        uint64_t kl;
        const char *k = rd_str(&r, &kl);
        const uint32_t vt = rd_u32(&r);
        /* metadata keys, main.c:881-948 */
        if (key_is(k, kl, "general.alignment")) align = (uint32_t)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.embedding_length")) m->dim = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.feed_forward_length")) m->hidden = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.block_count")) m->n_layers = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.head_count")) m->n_heads = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.head_count_kv")) m->n_kv = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.key_length_swa")) m->hd_swa = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.key_length")) m->hd_full = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.rope.dimension_count_swa")) m->rot_swa = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.rope.dimension_count")) m->rot_full = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.layer_norm_rms_epsilon")) m->eps = (float)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.rope.freq_base")) m->theta = (float)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.rope.freq_base_swa")) m->theta_swa = (float)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.sliding_window")) m->window = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.shared_kv_layers")) m->shared_kv = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.embedding_length_per_layer_input")) m->ple_dim = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.final_logit_softcapping")) m->softcap = (float)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.context_length")) m->max_seq = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "tokenizer.ggml.eos_token_id")) m->eos = (int)rd_num(&r, vt);
        else if (key_is(k, kl, "gemma4.attention.sliding_window_pattern") && vt == 9) {
            const uint32_t et = rd_u32(&r);
            const uint64_t n = rd_u64(&r);
            if (n > 0 && n <= 256) {
                m->swa_layers = (int *)calloc(n, sizeof(int));
                for (uint64_t j = 0; j < n; j++) m->swa_layers[j] = rd_num(&r, et) != 0;
            } else {
                for (uint64_t j = 0; j < n; j++) rd_skip(&r, et);
            }
        } else if (key_is(k, kl, "tokenizer.ggml.tokens") && vt == 9) {
            rd_u32(&r);
            const uint64_t n = rd_u64(&r);
            m->vocab = (int)n;
            for (uint64_t j = 0; j < n && !r.bad; j++) { uint64_t l; rd_str(&r, &l); }
        } else rd_skip(&r, vt);
    }
    or_tinfo *ti = (or_tinfo *)calloc(n_t ? n_t : 1, sizeof(or_tinfo));
    for (uint64_t i = 0; i < n_t && !r.bad; i++) {
        ti[i].name = rd_str(&r, &ti[i].nl);
        ti[i].n_dims = (int)rd_u32(&r);
        if (ti[i].n_dims > 4) { r.bad = 1; break; }
        for (int d = 0; d < ti[i].n_dims; d++) ti[i].ne[d] = rd_u64(&r);
        ti[i].type = (int)rd_u32(&r);
        ti[i].off = rd_u64(&r);
    }
    if (r.bad) { free(ti); or_model_close(m); set_err(err, errlen, "truncated GGUF"); return NULL; }
    const uint64_t doff = (r.p + (align - 1)) & ~(uint64_t)(align - 1);
    const uint8_t *base = data + doff;
    for (uint64_t i = 0; i < n_t; i++) {
        if (doff + ti[i].off > size) { free(ti); or_model_close(m); set_err(err, errlen, "tensor offset out of range"); return NULL; }
    }
    if (max_seq > 0) m->max_seq = max_seq;

    /* load_weights, main.c:1328-1400 */
    const int nt = (int)n_t, L = m->n_layers;
    or_tensor t;
    find_t(ti, nt, base, "token_embd.weight", &m->embd);
    find_t(ti, nt, base, "per_layer_token_embd.weight", &m->ple_tok);
    find_t(ti, nt, base, "per_layer_model_proj.weight", &m->ple_proj);
    m->ple_proj_norm = find_t(ti, nt, base, "per_layer_proj_norm.weight", &t) ? (const float *)t.p : NULL;
    m->rope_freqs = find_t(ti, nt, base, "rope_freqs.weight", &t) ? (const float *)t.p : NULL;
    m->norm_out = find_t(ti, nt, base, "output_norm.weight", &t) ? (const float *)t.p : NULL;
#define OR_ALLOC_PTRS(f) m->f = (const float **)calloc((size_t)L, sizeof(float *))
    OR_ALLOC_PTRS(attn_norm); OR_ALLOC_PTRS(post_attn_norm); OR_ALLOC_PTRS(ffn_norm);
    OR_ALLOC_PTRS(post_ffw_norm); OR_ALLOC_PTRS(q_norm); OR_ALLOC_PTRS(k_norm);
    OR_ALLOC_PTRS(post_norm); OR_ALLOC_PTRS(out_scale);
#undef OR_ALLOC_PTRS
#define OR_ALLOC_T(f) m->f = (or_tensor *)calloc((size_t)L, sizeof(or_tensor))
    OR_ALLOC_T(wq); OR_ALLOC_T(wk); OR_ALLOC_T(wv); OR_ALLOC_T(wo); OR_ALLOC_T(gate);
    OR_ALLOC_T(up); OR_ALLOC_T(down); OR_ALLOC_T(inp_gate); OR_ALLOC_T(proj);
#undef OR_ALLOC_T
    char name[128];
    for (int l = 0; l < L; l++) {
#define OR_NORM(f, s) snprintf(name, sizeof name, "blk.%d." s, l); \
        m->f[l] = find_t(ti, nt, base, name, &t) ? (const float *)t.p : NULL
#define OR_MAT(f, s) snprintf(name, sizeof name, "blk.%d." s, l); find_t(ti, nt, base, name, &m->f[l])
        OR_NORM(attn_norm, "attn_norm.weight");
        OR_NORM(post_attn_norm, "post_attention_norm.weight");
        OR_NORM(q_norm, "attn_q_norm.weight");
        OR_NORM(k_norm, "attn_k_norm.weight");
        OR_MAT(wq, "attn_q.weight");
        OR_MAT(wk, "attn_k.weight");
        OR_MAT(wv, "attn_v.weight");
        OR_MAT(wo, "attn_output.weight");
        OR_NORM(ffn_norm, "ffn_norm.weight");
        OR_NORM(post_ffw_norm, "post_ffw_norm.weight");
        OR_MAT(gate, "ffn_gate.weight");
        OR_MAT(up, "ffn_up.weight");
        OR_MAT(down, "ffn_down.weight");
        OR_MAT(inp_gate, "inp_gate.weight");
        OR_MAT(proj, "proj.weight");
        OR_NORM(post_norm, "post_norm.weight");
        OR_NORM(out_scale, "layer_output_scale.weight");
#undef OR_NORM
#undef OR_MAT
    }
    free(ti);
    if (!m->embd.p || !m->norm_out || !m->ple_tok.p || !m->ple_proj.p || !m->ple_proj_norm) {
        or_model_close(m);
        set_err(err, errlen, "missing critical global tensors");
        return NULL;
    }
    /* alloc_state, main.c:1402-1423 */
    const size_t kv_len = (size_t)OR_N_LAYER_KV * m->max_seq * OR_MAX_KV_DIM;
    m->x = (float *)calloc((size_t)m->dim, 4);
    m->xb = (float *)calloc(OR_MAX_Q_DIM, 4);
    m->xb2 = (float *)calloc((size_t)m->dim, 4);
    m->hb = (float *)calloc((size_t)m->hidden, 4);
    m->hb2 = (float *)calloc((size_t)m->hidden, 4);
    m->q = (float *)calloc(OR_MAX_Q_DIM, 4);
    m->k = (float *)calloc(OR_MAX_KV_DIM, 4);
    m->v = (float *)calloc(OR_MAX_KV_DIM, 4);
    m->q_out = (float *)calloc(OR_MAX_Q_DIM, 4);
    m->ple = (float *)calloc((size_t)m->ple_dim * L, 4);
    m->ple_ctx = (float *)calloc((size_t)m->ple_dim * L, 4);
    m->ple_gate = (float *)calloc((size_t)m->ple_dim, 4);
    m->att = (float *)calloc((size_t)m->n_heads * m->max_seq, 4);
    m->logits = (float *)calloc((size_t)(m->vocab > 0 ? m->vocab : 1), 4);
    m->kc = (float *)calloc(kv_len, 4);
    m->vc = (float *)calloc(kv_len, 4);
    const int q8n = (m->hidden > OR_MAX_Q_DIM ? m->hidden : OR_MAX_Q_DIM) / OR_QK_K + 1;
    m->q8 = (or_q8K *)calloc((size_t)q8n, sizeof(or_q8K));
    m->stats = (float *)calloc((size_t)L * 3 + 8, 4);
    m->astats = (float *)calloc((size_t)L * 3, 4);
    m->layer_x = (float *)calloc((size_t)L * m->dim, 4);
    m->q8_rec = (or_q8K *)calloc((size_t)L * OR_Q8_SLOTS * OR_Q8_SLOT_BLOCKS, sizeof(or_q8K));
    if (!m->kc || !m->vc) { or_model_close(m); set_err(err, errlen, "out of memory"); return NULL; }
    return m;
}

void or_model_close(or_model *m) {
    if (!m) return;
    free(m->swa_layers);
    free(m->attn_norm); free(m->post_attn_norm); free(m->ffn_norm); free(m->post_ffw_norm);
    free(m->q_norm); free(m->k_norm); free(m->post_norm); free(m->out_scale);
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->gate); free(m->up);
    free(m->down); free(m->inp_gate); free(m->proj);
    free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q); free(m->k);
    free(m->v); free(m->q_out); free(m->ple); free(m->ple_ctx); free(m->ple_gate); free(m->att);
    free(m->logits); free(m->kc); free(m->vc); free(m->q8); free(m->stats); free(m->astats); free(m->layer_x);
    free(m->q8_rec);
    free(m);
}

void or_model_config(const or_model *m, int out[9]) {
    out[0] = m->dim; out[1] = m->hidden; out[2] = m->n_layers; out[3] = m->n_heads;
    out[4] = m->n_kv; out[5] = m->vocab; out[6] = m->max_seq; out[7] = m->ple_dim; out[8] = m->window;
}

const float *or_model_logits(const or_model *m) { return m->logits; }
const float *or_model_x(const or_model *m) { return m->x; }
const float *or_model_layer_stats(const or_model *m) { return m->stats; }
const float *or_model_attn_stats(const or_model *m) { return m->astats; }
const float *or_model_layer_x(const or_model *m) { return m->layer_x; }
const or_q8K *or_model_q8_rec(const or_model *m) { return m->q8_rec; }
int or_model_kv_source(const or_model *m, int layer) { return kv_source(m, layer); }
const float *or_model_fingerprint(const or_model *m, int *have) {
    if (have) memcpy(have, m->fp_have, sizeof m->fp_have);
    return m->fp;
}

float *or_model_kv(or_model *m, int layer, int which) {
    if (layer < 0 || layer >= OR_N_LAYER_KV || layer >= m->n_layers) return NULL;
    return (which ? m->vc : m->kc) + (size_t)layer * m->max_seq * OR_MAX_KV_DIM;
}

/* The Q8_K activation of quantization point `slot` of layer l, for a matrix
 * of `type` with inputs x[n]: quantize_row_q8_K (main.c:282, called by
 * forward at 1884 and 1975, inside mm at 1685 otherwise) into m->q8,
 * recorded in q8_rec, then replaced by the injected blocks if any.  Returns
 * mm's q8_ready flag: 1 when m->q8 holds the activation, 0 when mm does not
 * take this matrix through Q8_K (other types, --f32-matmul). */
static int q8_point(or_model *m, int l, int slot, const float *x, int n, int type) {
    if (!((type == OR_Q4_K || type == OR_Q5_K) && !or_f32_matmul)) return 0;
    const int nb = n / OR_QK_K;
    if (n % OR_QK_K || nb > OR_Q8_SLOT_BLOCKS) return 0;
    or_quantize_q8K(x, m->q8, n);
    const size_t off = ((size_t)l * OR_Q8_SLOTS + slot) * OR_Q8_SLOT_BLOCKS;
    memcpy(m->q8_rec + off, m->q8, (size_t)nb * sizeof(or_q8K));
    if (m->q8_inj) memcpy(m->q8, m->q8_inj + off, (size_t)nb * sizeof(or_q8K));
    return 1;
}

/* main.c:1747-1778 */
static void build_ple(or_model *m, int token) {
    const int L = m->n_layers, pd = m->ple_dim, rd = pd * L;
    float *row = (float *)malloc((size_t)rd * sizeof(float));
    or_emb_lookup(row, m->ple_tok.p, m->ple_tok.type, token, rd);
    const float st = sqrtf((float)pd);
    for (int i = 0; i < rd; i++) row[i] = row[i] * st;
    or_mm(m->ple_ctx, m->x, m->ple_proj.p, m->dim, rd, m->ple_proj.type, m->q8, 0);
    const float sc = 1.0f / sqrtf((float)m->dim);
    for (int i = 0; i < rd; i++) m->ple_ctx[i] = m->ple_ctx[i] * sc;
    for (int l = 0; l < L; l++)
        or_rmsnorm(m->ple_ctx + (size_t)l * pd, m->ple_ctx + (size_t)l * pd, m->ple_proj_norm, pd, m->eps);
    const float mix = 1.0f / sqrtf(2.0f);
    for (int i = 0; i < rd; i++) m->ple[i] = (row[i] + m->ple_ctx[i]) * mix;
    free(row);
}

/* K and V of a storing layer from m->xb2 (and m->q8 when q8_ready):
 * projections, k_norm, the unweighted V norm, RoPE of K and the store at
 * pos (main.c:1888-1904). */
static int layer_kv(or_model *m, int l, int pos, int q8_ready) {
    const int dim = m->dim, nkv = m->n_kv, hd = layer_hd(m, l), kv_dim = nkv * hd;
    const int swa = is_swa(m, l);
    const int n_rot = swa ? m->rot_swa : m->rot_full;
    const float base = swa ? m->theta_swa : m->theta;
    const float *ff = swa ? NULL : m->rope_freqs;
    if (or_mm(m->k, m->xb2, m->wk[l].p, dim, kv_dim, m->wk[l].type, m->q8, q8_ready)) return -1;
    if (or_mm(m->v, m->xb2, m->wv[l].p, dim, kv_dim, m->wv[l].type, m->q8, q8_ready)) return -1;
    if (l == 0) fp_tag(m, OR_FP_K_PRE_NORM, m->k, kv_dim);           /* main.c:1893-1894 */
    or_rmsnorm_head_inplace(m->k, m->k_norm[l], nkv, hd, m->eps);
    or_rmsnorm_head_noweight_inplace(m->v, nkv, hd, m->eps);
    if (l == 0) fp_tag(m, OR_FP_K_PRE_ROPE, m->k, kv_dim);           /* main.c:1897-1898 */
    or_apply_rope_neox(m->k, nkv, hd, n_rot, pos, base, 1.0f, ff);
    const size_t off = ((size_t)l * m->max_seq + pos) * OR_MAX_KV_DIM;
    memcpy(m->kc + off, m->k, (size_t)kv_dim * sizeof(float));
    memcpy(m->vc + off, m->v, (size_t)kv_dim * sizeof(float));
    if (l == 0) fp_tag(m, OR_FP_K_STORE, m->k, kv_dim);              /* main.c:1905-1906 */
    if (l == 0) {
        float s, q2, a;
        or_hidden_stats(m->k, kv_dim, &s, &q2, &a);
        m->stats[(size_t)m->n_layers * 3 + 0] = s;
        m->stats[(size_t)m->n_layers * 3 + 1] = q2;
        m->stats[(size_t)m->n_layers * 3 + 2] = a;
    }
    return 0;
}

/* One decoder layer of forward() (main.c:1865-2011) on m->x; x_before is
 * dim floats of scratch. */
static int layer_step(or_model *m, int l, int pos, float *x_before) {
    const int dim = m->dim, hidden = m->hidden, nh = m->n_heads, nkv = m->n_kv;
    const int hd = layer_hd(m, l), q_dim = nh * hd;
    const int swa = is_swa(m, l);
    const int n_rot = swa ? m->rot_swa : m->rot_full;
    const float base = swa ? m->theta_swa : m->theta;
    const float *ff = swa ? NULL : m->rope_freqs;
    memcpy(x_before, m->x, (size_t)dim * sizeof(float));
    or_rmsnorm(m->xb2, m->x, m->attn_norm[l], dim, m->eps);
    if (l == 0) {
        memset(m->fp_have, 0, sizeof m->fp_have);
        fp_tag(m, OR_FP_ATTN_NORM, m->xb2, dim);                     /* main.c:1880-1881 */
    }
    const int q8_att = q8_point(m, l, OR_Q8_SLOT_ATTN, m->xb2, dim, m->wq[l].type);
    if (or_mm(m->q, m->xb2, m->wq[l].p, dim, q_dim, m->wq[l].type, m->q8, q8_att)) return -1;
    or_rmsnorm_head_inplace(m->q, m->q_norm[l], nh, hd, m->eps);
    or_apply_rope_neox(m->q, nh, hd, n_rot, pos, base, 1.0f, ff);
    const int src = kv_source(m, l);
    if (l < OR_N_LAYER_KV && layer_kv(m, l, pos, q8_att)) return -1;
    const int src_hd = layer_hd(m, src);
    int t_start = 0;
    if (swa) { t_start = pos + 1 - m->window; if (t_start < 0) t_start = 0; }
    const int nwin = pos + 1 - t_start;
    (void)src_hd;
    if (l == 0) {                                                    /* main.c:1916-1921 */
        const int kvd0 = nkv * layer_hd(m, 0);
        fp_tag(m, OR_FP_K_READ0, m->kc, kvd0);
        if (pos > 0) fp_tag(m, OR_FP_K_READN, m->kc + (size_t)pos * OR_MAX_KV_DIM, kvd0);
    }
    const float *kc0 = m->kc + (size_t)src * m->max_seq * OR_MAX_KV_DIM;
    const float *vc0 = m->vc + (size_t)src * m->max_seq * OR_MAX_KV_DIM;
    or_attn_decode(m->q, kc0, vc0, OR_MAX_KV_DIM, t_start, nwin, nh, nkv, hd, 1.0f, m->att, m->q_out);
    if (l == 0) {
        float s, q2, a;
        fp_tag(m, OR_FP_Q_OUT, m->q_out, q_dim);
        or_hidden_stats(m->q_out, q_dim, &s, &q2, &a);
        m->stats[(size_t)m->n_layers * 3 + 3] = s;
        m->stats[(size_t)m->n_layers * 3 + 4] = q2;
        m->stats[(size_t)m->n_layers * 3 + 5] = a;
    }
    const int q8_o = q8_point(m, l, OR_Q8_SLOT_O, m->q_out, q_dim, m->wo[l].type);
    if (or_mm(m->xb2, m->q_out, m->wo[l].p, q_dim, dim, m->wo[l].type, m->q8, q8_o)) return -1;
    or_rmsnorm(m->xb2, m->xb2, m->post_attn_norm[l], dim, m->eps);
    for (int i = 0; i < dim; i++) m->x[i] = x_before[i] + m->xb2[i];
    or_hidden_stats(m->x, dim, &m->astats[3 * l], &m->astats[3 * l + 1], &m->astats[3 * l + 2]);
    memcpy(x_before, m->x, (size_t)dim * sizeof(float));
    or_rmsnorm(m->xb2, m->x, m->ffn_norm[l], dim, m->eps);
    const int q8_ffn = q8_point(m, l, OR_Q8_SLOT_FFN, m->xb2, dim, m->gate[l].type);
    if (or_mm(m->hb, m->xb2, m->gate[l].p, dim, hidden, m->gate[l].type, m->q8, q8_ffn)) return -1;
    if (or_mm(m->hb2, m->xb2, m->up[l].p, dim, hidden, m->up[l].type, m->q8, q8_ffn)) return -1;
    for (int i = 0; i < hidden; i++) m->hb[i] = or_gelu(m->hb[i]) * m->hb2[i];
    if (or_mm(m->xb2, m->hb, m->down[l].p, hidden, dim, m->down[l].type, m->q8, 0)) return -1;
    or_rmsnorm(m->xb2, m->xb2, m->post_ffw_norm[l], dim, m->eps);
    for (int i = 0; i < dim; i++) m->x[i] = x_before[i] + m->xb2[i];
    memcpy(x_before, m->x, (size_t)dim * sizeof(float));
    const int q8_ig = q8_point(m, l, OR_Q8_SLOT_INP_GATE, m->x, dim, m->inp_gate[l].type);
    if (or_mm(m->ple_gate, m->x, m->inp_gate[l].p, dim, m->ple_dim, m->inp_gate[l].type, m->q8, q8_ig)) return -1;
    for (int i = 0; i < m->ple_dim; i++) m->ple_gate[i] = or_gelu(m->ple_gate[i]);
    const float *ple_l = m->ple + (size_t)l * m->ple_dim;
    for (int i = 0; i < m->ple_dim; i++) m->ple_gate[i] = m->ple_gate[i] * ple_l[i];
    const int q8_pr = q8_point(m, l, OR_Q8_SLOT_PROJ, m->ple_gate, m->ple_dim, m->proj[l].type);
    if (or_mm(m->xb2, m->ple_gate, m->proj[l].p, m->ple_dim, dim, m->proj[l].type, m->q8, q8_pr)) return -1;
    or_rmsnorm(m->xb2, m->xb2, m->post_norm[l], dim, m->eps);
    for (int i = 0; i < dim; i++) m->x[i] = x_before[i] + m->xb2[i];
    if (m->out_scale[l]) {
        const float sc = m->out_scale[l][0];
        for (int i = 0; i < dim; i++) m->x[i] = m->x[i] * sc;
    }
    or_hidden_stats(m->x, dim, &m->stats[3 * l], &m->stats[3 * l + 1], &m->stats[3 * l + 2]);
    if (m->layer_x) memcpy(m->layer_x + (size_t)l * dim, m->x, (size_t)dim * sizeof(float));
    return 0;
}

/* main.c:2021-2028: final norm and logits_tied (lm_mode 2 is unreachable with
 * softcap > 0) */
static int lm_head(or_model *m) {
    const int dim = m->dim;
    or_rmsnorm(m->x, m->x, m->norm_out, dim, m->eps);
    /* logits_tied, main.c:1780-1796 (lm_mode 2 is unreachable with softcap > 0) */
    if (or_mm(m->logits, m->x, m->embd.p, dim, m->vocab, m->embd.type, m->q8, 0)) return -1;
    if (m->softcap > 0.0f) {
        const float cap = m->softcap, inv = 1.0f / cap;
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < m->vocab; i++) m->logits[i] = cap * tanhf(m->logits[i] * inv);
    }
    return 0;
}

static int embed_ple(or_model *m, int token, int pos) {
    const int dim = m->dim;
    if (pos < 0 || pos >= m->max_seq || token < 0 || token >= m->vocab) return -1;
    if (or_emb_lookup(m->x, m->embd.p, m->embd.type, token, dim)) return -1;
    const float es = sqrtf((float)dim);
    for (int i = 0; i < dim; i++) m->x[i] = m->x[i] * es;
    build_ple(m, token);
    return 0;
}

/* main.c:1838-2029 (debug dumps replaced by the stats array) */
int or_forward(or_model *m, int token, int pos, int lm_mode) {
    if (embed_ple(m, token, pos)) return -1;
    float *x_before = (float *)malloc((size_t)m->dim * sizeof(float));
    for (int l = 0; l < m->n_layers; l++) {
        if (layer_step(m, l, pos, x_before)) { free(x_before); return -1; }
    }
    free(x_before);
    if (lm_mode == 0) return 0;
    return lm_head(m);
}

/* forward() with every layer's input taken from x_in ((n_layers+1) x dim:
 * row 0 is the input of layer 0, row l+1 the input of layer l+1, row
 * n_layers the input of the final norm).  Layer l's output goes to row l of
 * x_out (n_layers x dim).  The KV cache is written from the injected inputs,
 * so each layer is checked in isolation against a device run that produced
 * x_in.  The embedding of the token is still computed (build_ple uses it). */
int or_forward_inject(or_model *m, int token, int pos, int lm_mode, const float *x_in, float *x_out) {
    const int dim = m->dim;
    if (embed_ple(m, token, pos)) return -1;
    float *x_before = (float *)malloc((size_t)dim * sizeof(float));
    for (int l = 0; l < m->n_layers; l++) {
        memcpy(m->x, x_in + (size_t)l * dim, (size_t)dim * sizeof(float));
        if (layer_step(m, l, pos, x_before)) { free(x_before); return -1; }
        memcpy(x_out + (size_t)l * dim, m->x, (size_t)dim * sizeof(float));
    }
    free(x_before);
    if (lm_mode == 0) return 0;
    memcpy(m->x, x_in + (size_t)m->n_layers * dim, (size_t)dim * sizeof(float));
    return lm_head(m);
}

int or_embed(or_model *m, int token, int pos) { return embed_ple(m, token, pos); }

int or_layer_inject(or_model *m, int token, int pos, int layer, const float *x_in, float *x_out) {
    if (layer < 0 || layer >= m->n_layers || embed_ple(m, token, pos)) return -1;
    float *x_before = (float *)malloc((size_t)m->dim * sizeof(float));
    memcpy(m->x, x_in, (size_t)m->dim * sizeof(float));
    const int rc = layer_step(m, layer, pos, x_before);
    free(x_before);
    if (rc == 0) memcpy(x_out, m->x, (size_t)m->dim * sizeof(float));
    return rc;
}

int or_lm_head_inject(or_model *m, const float *x_in) {
    memcpy(m->x, x_in, (size_t)m->dim * sizeof(float));
    return lm_head(m);
}

float *or_model_state(or_model *m, const char *name) {
    static const char *names[] = {"x", "xb2", "q", "k", "v", "q_out", "ple", "ple_ctx", "ple_gate", "hb", "hb2", "logits"};
    float *bufs[] = {m->x, m->xb2, m->q, m->k, m->v, m->q_out, m->ple, m->ple_ctx, m->ple_gate, m->hb, m->hb2, m->logits};
    for (size_t i = 0; i < sizeof names / sizeof names[0]; i++)
        if (!strcmp(name, names[i])) return bufs[i];
    return NULL;
}

int or_forward_inject_q8(or_model *m, int token, int pos, int lm_mode, const float *x_in, const or_q8K *q8_in,
                         float *x_out) {
    m->q8_inj = q8_in;
    const int rc = or_forward_inject(m, token, pos, lm_mode, x_in, x_out);
    m->q8_inj = NULL;
    return rc;
}

/* The K/V part of forward() for every storing layer, each from its injected
 * input row: attn_norm, Q8_K (main.c:1878-1884), then layer_kv. */
int or_forward_inject_kv(or_model *m, int token, int pos, const float *x_in, const or_q8K *q8_in) {
    const int dim = m->dim;
    if (pos < 0 || pos >= m->max_seq || token < 0 || token >= m->vocab) return -1;
    m->q8_inj = q8_in;
    int rc = 0;
    for (int l = 0; l < m->n_layers && l < OR_N_LAYER_KV && rc == 0; l++) {
        or_rmsnorm(m->xb2, x_in + (size_t)l * dim, m->attn_norm[l], dim, m->eps);
        const int q8_att = q8_point(m, l, OR_Q8_SLOT_ATTN, m->xb2, dim, m->wq[l].type);
        rc = layer_kv(m, l, pos, q8_att);
    }
    m->q8_inj = NULL;
    return rc;
}

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + (double)t.tv_nsec * 1e-9;
}

/* main.c:2335-2488 with temp <= 0 (greedy), no forced tokens, no thinking */
int or_generate_greedy(or_model *m, const int *prompt, int n_prompt, int max_new,
                       int *out_tokens, double *prefill_sec, double *decode_sec) {
    int token = prompt[0], gen = 0;
    const double t0 = now_s();
    double t_dec = t0;
    int decode_timing = 0;
    if (prefill_sec) *prefill_sec = 0.0;
    for (int pos = 0; pos < n_prompt + max_new - 1; pos++) {
        if (pos >= m->max_seq) break;
        const int lm_mode = (pos < n_prompt - 1) ? 0 : 1;
        if (or_forward(m, token, pos, lm_mode)) return -1;
        if (pos == n_prompt - 1) {
            t_dec = now_s();
            if (prefill_sec) *prefill_sec = t_dec - t0;
            decode_timing = 1;
        }
        int next;
        if (pos < n_prompt - 1) {
            next = prompt[pos + 1];
        } else {
            next = or_argmax_first(m->logits, m->vocab);
            if (next == m->eos) break;
            out_tokens[gen++] = next;
        }
        token = next;
    }
    if (decode_sec) *decode_sec = decode_timing ? now_s() - t_dec : 0.0;
    return gen;
}
