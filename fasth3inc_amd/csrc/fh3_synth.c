/*
 * fh3_synth.c -- seeded generators and the Q4_K encoder (see fh3_synth.h).
 * Host C99 + OpenMP; no GPU work happens here.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "fh3/fh3.h"
#include "fh3/fh3_synth.h"

/* ------------------------------------------------------------------------ */
/* Philox4x32-10                                                             */
/* ------------------------------------------------------------------------ */
#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

void fh3_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        const uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Block b of stream s: counter (b_lo, b_hi, s_lo, s_hi), key (seed_lo, seed_hi). */
static void philox_block(uint64_t seed, uint64_t stream, uint64_t b, uint32_t out[4]) {
    const uint32_t ctr[4] = {(uint32_t)b, (uint32_t)(b >> 32), (uint32_t)stream, (uint32_t)(stream >> 32)};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    fh3_philox4x32_10(ctr, key, out);
}

/* Box-Muller on two words: u = (w + 1) / (2^32 + 2) in (0,1). */
static void box_muller(uint32_t a, uint32_t b, float *z0, float *z1) {
    const double u0 = ((double)a + 1.0) / 4294967298.0;
    const double u1 = ((double)b + 1.0) / 4294967298.0;
    const double r = sqrt(-2.0 * log(u0));
    const double th = 6.28318530717958647692 * u1;
    *z0 = (float)(r * cos(th));
    *z1 = (float)(r * sin(th));
}

void fh3_synth_rng_normal(uint64_t seed, uint64_t stream, float *out, size_t n) {
    if (!out || n == 0) return;
    const int64_t nb = (int64_t)((n + 3) / 4);
    #pragma omp parallel for schedule(static) if (nb > 4096)
    for (int64_t b = 0; b < nb; b++) {
        uint32_t w[4];
        float z[4];
        philox_block(seed, stream, (uint64_t)b, w);
        box_muller(w[0], w[1], &z[0], &z[1]);
        box_muller(w[2], w[3], &z[2], &z[3]);
        const size_t base = (size_t)b * 4;
        for (int i = 0; i < 4 && base + (size_t)i < n; i++) out[base + (size_t)i] = z[i];
    }
}

void fh3_rng_uniform(uint64_t seed, uint64_t stream, float *out, size_t n) {
    if (!out || n == 0) return;
    const int64_t nb = (int64_t)((n + 3) / 4);
    #pragma omp parallel for schedule(static) if (nb > 4096)
    for (int64_t b = 0; b < nb; b++) {
        uint32_t w[4];
        philox_block(seed, stream, (uint64_t)b, w);
        const size_t base = (size_t)b * 4;
        for (int i = 0; i < 4 && base + (size_t)i < n; i++)
            out[base + (size_t)i] = (float)(((double)w[i] + 0.5) / 4294967296.0);
    }
}

/* ------------------------------------------------------------------------ */
/* fp16 encode                                                              */
/* ------------------------------------------------------------------------ */
uint16_t fh3_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / NaN */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
    if (ax >= 0x477FF000u) /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        const uint32_t e = ax >> 23;                 /* 102..112 */
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;             /* value = m * 2^(e-150); unit 2^-24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float f16_to_f32_bits(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu, bits;
    if (exp == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);
    else if (exp) bits = sign | ((exp + 112u) << 23) | (man << 13);
    else if (!man) bits = sign;
    else {
        uint32_t e = 113u;
        while (!(man & 0x400u)) { man <<= 1; e--; }
        bits = sign | (e << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Q4_K encoder                                                             */
/* ------------------------------------------------------------------------ */
static int clamp_round(float v, int lo, int hi) {
    const float r = nearbyintf(v);
    if (!(r >= (float)lo)) return lo; /* also NaN */
    if (r > (float)hi) return hi;
    return (int)r;
}

static void q4k_encode_block(const float *w, uint8_t *blk) {
    float step[8], offs[8];
    float smax = 0.f, omax = 0.f;
    for (int g = 0; g < 8; g++) {
        float lo = 0.f, hi = -INFINITY;
        for (int l = 0; l < 32; l++) {
            const float v = w[g * 32 + l];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        if (hi < lo) hi = lo;
        step[g] = (hi - lo) / 15.f;
        offs[g] = -lo;
        if (step[g] > smax) smax = step[g];
        if (offs[g] > omax) omax = offs[g];
    }
    const uint16_t hd = fh3_f32_to_f16(smax / 63.f);
    const uint16_t hm = fh3_f32_to_f16(omax / 63.f);
    const float d = f16_to_f32_bits(hd), dmin = f16_to_f32_bits(hm);
    uint8_t sc[8], mn[8];
    for (int g = 0; g < 8; g++) {
        sc[g] = (uint8_t)(d > 0.f ? clamp_round(step[g] / d, 0, 63) : 0);
        mn[g] = (uint8_t)(dmin > 0.f ? clamp_round(offs[g] / dmin, 0, 63) : 0);
    }
    blk[0] = (uint8_t)(hd & 0xFFu); blk[1] = (uint8_t)(hd >> 8);
    blk[2] = (uint8_t)(hm & 0xFFu); blk[3] = (uint8_t)(hm >> 8);
    uint8_t *s = blk + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63u) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63u) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15u) | ((mn[j + 4] & 15u) << 4));
    }
    uint8_t *qs = blk + 16;
    for (int c = 0; c < 4; c++) {
        const int glo = 2 * c, ghi = 2 * c + 1;
        const float Dlo = d * (float)sc[glo], Mlo = dmin * (float)mn[glo];
        const float Dhi = d * (float)sc[ghi], Mhi = dmin * (float)mn[ghi];
        for (int l = 0; l < 32; l++) {
            const int qlo = Dlo > 0.f ? clamp_round((w[glo * 32 + l] + Mlo) / Dlo, 0, 15) : 0;
            const int qhi = Dhi > 0.f ? clamp_round((w[ghi * 32 + l] + Mhi) / Dhi, 0, 15) : 0;
            qs[c * 32 + l] = (uint8_t)(qlo | (qhi << 4));
        }
    }
}

int fh3_q4k_quantize(const float *src, int64_t rows, int64_t n, uint8_t *dst) {
    if (!src || !dst || rows <= 0 || n <= 0 || n % 256) return FH3_E_INVALID;
    const int64_t nsb = n / 256;
    #pragma omp parallel for schedule(static) if (rows * nsb > 1024)
    for (int64_t i = 0; i < rows * nsb; i++) q4k_encode_block(src + i * 256, dst + i * 144);
    return FH3_OK;
}

/* ------------------------------------------------------------------------ */
/* Workload generators                                                      */
/* ------------------------------------------------------------------------ */
int fh3_synth_q4k_weights(uint64_t seed, uint64_t stream, int64_t rows, int64_t n, float sigma,
                          float spread_decades, uint8_t *dst) {
    if (!dst || rows <= 0 || n <= 0 || n % 256) return FH3_E_INVALID;
    const int64_t nsb = n / 256;
    const int64_t chunk_rows = 256;
    float *buf = (float *)malloc((size_t)chunk_rows * (size_t)n * sizeof(float));
    float *spr = spread_decades > 0.f ? (float *)malloc((size_t)chunk_rows * (size_t)nsb * sizeof(float)) : NULL;
    if (!buf || (spread_decades > 0.f && !spr)) {
        free(buf);
        free(spr);
        return FH3_E_NOMEM;
    }
    for (int64_t r0 = 0; r0 < rows; r0 += chunk_rows) {
        const int64_t nr = rows - r0 < chunk_rows ? rows - r0 : chunk_rows;
        /* the element stream is indexed by (row * n + k): chunking is invisible */
        const size_t cnt = (size_t)(nr * n);
        /* Philox blocks are 4 values; n % 256 == 0 keeps chunks block aligned */
        float *p = buf;
        {
            const int64_t b0 = (r0 * n) / 4, nb = (int64_t)(cnt / 4);
            #pragma omp parallel for schedule(static)
            for (int64_t b = 0; b < nb; b++) {
                uint32_t wv[4];
                float z[4];
                philox_block(seed, stream, (uint64_t)(b0 + b), wv);
                box_muller(wv[0], wv[1], &z[0], &z[1]);
                box_muller(wv[2], wv[3], &z[2], &z[3]);
                for (int i = 0; i < 4; i++) p[b * 4 + i] = sigma * z[i];
            }
        }
        if (spr) {
            const int64_t nsbc = nr * nsb;
            #pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < nsbc; i++) {
                uint32_t wv[4];
                /* one block per super-block on stream ^ 0x5350 ("SP") */
                philox_block(seed, stream ^ 0x5350ull, (uint64_t)(r0 * nsb + i), wv);
                const double u = ((double)wv[0] + 0.5) / 4294967296.0;
                const float f = (float)pow(10.0, spread_decades * (u - 0.5));
                for (int l = 0; l < 256; l++) buf[i * 256 + l] *= f;
            }
        }
        int rc = fh3_q4k_quantize(buf, nr, n, dst + (size_t)r0 * (size_t)nsb * 144u);
        if (rc != FH3_OK) {
            free(buf);
            free(spr);
            return rc;
        }
    }
    free(buf);
    free(spr);
    return FH3_OK;
}

void fh3_synth_x_normal(uint64_t seed, uint64_t stream, float *x, size_t count) {
    fh3_synth_rng_normal(seed, stream, x, count);
}

void fh3_synth_x_outliers(uint64_t seed, uint64_t stream, float *x, size_t count, float frac) {
    if (!x || count == 0) return;
    fh3_synth_rng_normal(seed, stream, x, count);
    const double thr = (double)frac * 4294967296.0;
    const int64_t nb = (int64_t)((count + 1) / 2);
    #pragma omp parallel for schedule(static) if (nb > 4096)
    for (int64_t b = 0; b < nb; b++) {
        uint32_t wv[4];
        /* two entries per block on stream ^ 0x4F55 ("OU"): (select, sign) pairs */
        philox_block(seed, stream ^ 0x4F55ull, (uint64_t)b, wv);
        for (int i = 0; i < 2; i++) {
            const size_t idx = (size_t)b * 2 + (size_t)i;
            if (idx < count && (double)wv[2 * i] < thr) x[idx] = (wv[2 * i + 1] & 1u) ? 8.f : -8.f;
        }
    }
}

void fh3_synth_x_silu_gated(uint64_t seed, uint64_t stream, float *x, size_t count) {
    if (!x || count == 0) return;
    const int64_t nb = (int64_t)((count + 1) / 2);
    #pragma omp parallel for schedule(static) if (nb > 4096)
    for (int64_t b = 0; b < nb; b++) {
        uint32_t wv[4];
        float z[4];
        philox_block(seed, stream, (uint64_t)b, wv);
        box_muller(wv[0], wv[1], &z[0], &z[1]);
        box_muller(wv[2], wv[3], &z[2], &z[3]);
        for (int i = 0; i < 2; i++) {
            const size_t idx = (size_t)b * 2 + (size_t)i;
            if (idx >= count) break;
            const float a = z[2 * i], g = z[2 * i + 1];
            x[idx] = a * (g / (1.f + expf(-g)));
        }
    }
}
