/*
 * fh3_oracle.c -- CPU restatement of fh3's Q4_K path.  TEST INFRASTRUCTURE
 * ONLY (see fh3_oracle.h): the checker and CPU baseline for the HIP product.
 *
 * Build flags follow the reference (CMakeLists.txt:15-26): -O3 -mavx2 -mfma
 * -mf16c -ffp-contract=off -fopenmp.  -ffp-contract=off matters: the
 * reference rounds every product and every sum separately except where it
 * calls fmaf() explicitly.
 */
#include "fh3_oracle.h"

#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <omp.h>

#define ORACLE_Q4_K 12
#define ORACLE_F32 0

/* ------------------------------------------------------------------------ */
/* fp16 decode: src/core/fh3_quant.h:20-41.  The reference build uses F16C    */
/* (_cvtsh_ss), an exact conversion that quiets signalling NaNs; this is the  */
/* same mapping written out on the bit fields.                                */
/* ------------------------------------------------------------------------ */
float fh3_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal half: value = man * 2^-24; shift the leading one up to
         * bit 10 (s shifts) and the value is 1.f * 2^(-14 - s) */
        uint32_t e = 113u; /* fp32 biased exponent of 2^-14 */
        while (!(man & 0x400u)) {
            man <<= 1;
            e -= 1u;
        }
        bits = sign | (e << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* src/core/fh3_quant.c:14-34, restricted to the two types on this path. */
size_t fh3_oracle_row_bytes(int type, int64_t n) {
    if (n <= 0) return 0;
    if (type == ORACLE_F32) return (size_t)n * sizeof(float);
    if (type == ORACLE_Q4_K) return (size_t)((n + 255) / 256) * 144u;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q4_K super-block decode: src/core/fh3_quant.c:154-196.                     */
/*   bytes 0-1 d (fp16), 2-3 dmin (fp16), 4-15 packed 6-bit scales and mins,  */
/*   16-143 four 32-byte chunks of nibbles: chunk c low nibbles are group 2c, */
/*   high nibbles group 2c+1.  w = (d*sc)*q - dmin*m, each op rounded.        */
/* Only whole super-blocks are written (n/256), as in the reference.          */
/* ------------------------------------------------------------------------ */
static void oracle_q4k_scales(const uint8_t *s, uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = (uint8_t)(s[j] & 63u);
        mn[j] = (uint8_t)(s[j + 4] & 63u);
        sc[j + 4] = (uint8_t)((s[j + 8] & 15u) | ((s[j] >> 6) << 4));
        mn[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
}

static void oracle_dequant_q4_k(const uint8_t *src, float *dst, int64_t n) {
    const int64_t nsb = n / 256;
    for (int64_t b = 0; b < nsb; b++) {
        const uint8_t *blk = src + b * 144;
        uint16_t hd = (uint16_t)(blk[0] | (blk[1] << 8));
        uint16_t hm = (uint16_t)(blk[2] | (blk[3] << 8));
        const float d = fh3_oracle_f16_to_f32(hd);
        const float dmin = fh3_oracle_f16_to_f32(hm);
        uint8_t sc[8], mn[8];
        oracle_q4k_scales(blk + 4, sc, mn);
        float scale[8], offs[8];
        for (int g = 0; g < 8; g++) {
            scale[g] = d * (float)sc[g];
            offs[g] = dmin * (float)mn[g];
        }
        const uint8_t *qs = blk + 16;
        float *out = dst + b * 256;
        for (int c = 0; c < 4; c++) {
            const int glo = 2 * c, ghi = 2 * c + 1;
            for (int l = 0; l < 32; l++) {
                const uint8_t byte = qs[c * 32 + l];
                const float qlo = (float)(byte & 15u);
                const float qhi = (float)(byte >> 4);
                float plo = scale[glo] * qlo;
                float phi = scale[ghi] * qhi;
                out[glo * 32 + l] = plo - offs[glo];
                out[ghi * 32 + l] = phi - offs[ghi];
            }
        }
    }
}

/* src/core/fh3_quant.c:284-318: NULL / non-positive n is a silent no-op and an
 * unsupported type writes nothing. */
void fh3_oracle_dequant(int type, const void *src, float *dst, int64_t n) {
    if (!src || !dst || n <= 0) return;
    if (type == ORACLE_F32) {
        memcpy(dst, src, (size_t)n * sizeof(float));
    } else if (type == ORACLE_Q4_K) {
        oracle_dequant_q4_k((const uint8_t *)src, dst, n);
    }
}

/* ------------------------------------------------------------------------ */
/* Dot-product contract: src/core/fh3_ops.c:19-47 (and the AVX2 forms at      */
/* :50-207, which compute the same per-output sequence).  Lane j accumulates  */
/* k = j (mod 8) with fmaf over the first n - n%8 elements; the lanes reduce  */
/* as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)); the tail k >= n8 is folded with    */
/* fmaf; bias is a separate add (:100-105, :184-194).                          */
/* Four weight rows share one pass over x.                                    */
/* ------------------------------------------------------------------------ */
static inline float oracle_tree8(const float a[8]) {
    const float s01 = a[0] + a[1];
    const float s23 = a[2] + a[3];
    const float s45 = a[4] + a[5];
    const float s67 = a[6] + a[7];
    const float s03 = s01 + s23;
    const float s47 = s45 + s67;
    return s03 + s47;
}

static void oracle_dot4(const float *x, const float *w, int64_t n, int rows, float out[4]) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    const int64_t n8 = n - (n % 8);
    for (int64_t k = 0; k < n8; k += 8) {
        for (int r = 0; r < rows; r++) {
            const float *wr = w + (size_t)r * (size_t)n + k;
            for (int j = 0; j < 8; j++) acc[r][j] = fmaf(x[k + j], wr[j], acc[r][j]);
        }
    }
    for (int r = 0; r < rows; r++) {
        float s = oracle_tree8(acc[r]);
        const float *wr = w + (size_t)r * (size_t)n;
        for (int64_t k = n8; k < n; k++) s = fmaf(x[k], wr[k], s);
        out[r] = s;
    }
}

#define ORACLE_TILE 64 /* src/core/fh3_ops.c:16 */

void fh3_oracle_matmul_rows(const Fh3OracleW *w, const float *x, float *y,
                            int n_tok, const float *bias_or_null,
                            int64_t o_begin, int64_t o_end) {
    if (!w || !x || !y || n_tok <= 0 || w->in <= 0 || w->out <= 0) return;
    const size_t row_bytes = fh3_oracle_row_bytes(w->type, w->in);
    if (row_bytes == 0) return;
    if (o_begin < 0) o_begin = 0;
    if (o_end > w->out) o_end = w->out;
    if (o_begin >= o_end) return;
    const int64_t K = w->in, N = w->out;
    const int64_t ntiles = (o_end - o_begin + ORACLE_TILE - 1) / ORACLE_TILE;

    #pragma omp parallel
    {
        float *tile = (float *)malloc((size_t)ORACLE_TILE * (size_t)K * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t ti = 0; ti < ntiles; ti++) {
            if (!tile) continue;
            const int64_t o0 = o_begin + ti * ORACLE_TILE;
            const int64_t rows = (o0 + ORACLE_TILE <= o_end) ? ORACLE_TILE : (o_end - o0);
            /* the reference leaves the K%256 tail of the tile uninitialised
             * (fh3_quant.c:155); this path zero-fills it so results are defined */
            memset(tile, 0, (size_t)rows * (size_t)K * sizeof(float));
            for (int64_t r = 0; r < rows; r++)
                fh3_oracle_dequant(w->type, w->data + (size_t)(o0 + r) * row_bytes,
                                   tile + (size_t)r * (size_t)K, K);
            for (int t = 0; t < n_tok; t++) {
                const float *xt = x + (size_t)t * (size_t)K;
                float *yt = y + (size_t)t * (size_t)N;
                for (int64_t r = 0; r < rows; r += 4) {
                    const int nr = (rows - r >= 4) ? 4 : (int)(rows - r);
                    float d[4];
                    oracle_dot4(xt, tile + (size_t)r * (size_t)K, K, nr, d);
                    for (int i = 0; i < nr; i++) {
                        float v = d[i];
                        if (bias_or_null) v = v + bias_or_null[o0 + r + i];
                        yt[o0 + r + i] = v;
                    }
                }
            }
        }
        free(tile);
    }
}

void fh3_oracle_matmul(const Fh3OracleW *w, const float *x, float *y,
                       int n_tok, const float *bias_or_null) {
    if (!w) return;
    fh3_oracle_matmul_rows(w, x, y, n_tok, bias_or_null, 0, w->out);
}

int fh3_oracle_threads(void) { return omp_get_max_threads(); }
