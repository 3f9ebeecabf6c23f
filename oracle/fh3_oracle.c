/*
 * fh3_oracle.c -- CPU restatement of fh3's linear layer (any decodable weight
 * type), of every block decoder of src/core/fh3_quant.c (F32, F16, BF16, Q8_0,
 * Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) and of the DiT block's elementwise ops around
 * the layer (rmsnorm, modulate, swiglu, gate_residual) and of its attention
 * branch (rope3, dense online-softmax attention).  TEST INFRASTRUCTURE ONLY
 * (see fh3_oracle.h): the checker and CPU baseline for the HIP product.
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

/* src/core/fh3_quant.c:14-34: bytes per row, by (block bytes, block length). */
size_t fh3_oracle_row_bytes(int type, int64_t n) {
    if (n <= 0) return 0;
    int bb, bl;
    switch (type) {
        case 0: bb = 4, bl = 1; break;      /* F32 */
        case 1: bb = 2, bl = 1; break;      /* F16 */
        case 30: bb = 2, bl = 1; break;     /* BF16 */
        case 2: bb = 18, bl = 32; break;    /* Q4_0 */
        case 3: bb = 20, bl = 32; break;    /* Q4_1 */
        case 6: bb = 22, bl = 32; break;    /* Q5_0 */
        case 7: bb = 24, bl = 32; break;    /* Q5_1 */
        case 8: bb = 34, bl = 32; break;    /* Q8_0 */
        case 9: bb = 40, bl = 32; break;    /* Q8_1 */
        case 10: bb = 84, bl = 256; break;  /* Q2_K */
        case 11: bb = 110, bl = 256; break; /* Q3_K */
        case 12: bb = 144, bl = 256; break; /* Q4_K */
        case 13: bb = 176, bl = 256; break; /* Q5_K */
        case 14: bb = 210, bl = 256; break; /* Q6_K */
        case 15: bb = 292, bl = 256; break; /* Q8_K */
        default: return 0;
    }
    return (size_t)((n + bl - 1) / bl) * (size_t)bb;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

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

/* ------------------------------------------------------------------------ */
/* The other block formats of src/core/fh3_quant.c:36-282.  Every value is     */
/* formed with the reference's roundings: scale products first (d*sc,         */
/* dmin*m), then the weight product, then the offset subtraction, each in      */
/* fp32.  Only whole blocks are written (n / block length).                   */
/* ------------------------------------------------------------------------ */

/* F16 (:36-49): exact conversion; BF16 (:51-56, fh3_quant.h:44-49): the 16 bits
 * are the top half of the fp32 word. */
static void oracle_dequant_f16(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = fh3_oracle_f16_to_f32(rd16(src + 2 * i));
}

static void oracle_dequant_bf16(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const uint32_t bits = (uint32_t)rd16(src + 2 * i) << 16;
        memcpy(&dst[i], &bits, sizeof bits);
    }
}

/* Q8_0 (:58-72): 34-byte blocks of 32, fp16 d then 32 int8; w = q * d. */
static void oracle_dequant_q8_0(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = src + b * 34;
        const float d = fh3_oracle_f16_to_f32(rd16(blk));
        for (int i = 0; i < 32; i++) dst[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

/* Q2_K (:74-114): 84-byte super-blocks.  Bytes 0-15: one byte per 16-weight
 * group, scale in the low nibble and min in the high nibble; 16-79: two
 * 32-byte chunks of 2-bit values; 80-81 d, 82-83 dmin.  Weight j of the
 * super-block lives in chunk j/128 at bit pair (j/32)%4, byte (j%32); its
 * group is j/16.  w = (d*sc)*q - dmin*m. */
static void oracle_dequant_q2_k(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 84;
        const float d = fh3_oracle_f16_to_f32(rd16(blk + 80));
        const float dmin = fh3_oracle_f16_to_f32(rd16(blk + 82));
        for (int j = 0; j < 256; j++) {
            const int g = j / 16;
            const uint8_t q = (uint8_t)((blk[16 + (j / 128) * 32 + (j % 32)] >> (2 * ((j / 32) % 4))) & 3u);
            const float dl = d * (float)(blk[g] & 15u);
            const float ml = dmin * (float)(blk[g] >> 4);
            dst[b * 256 + j] = dl * (float)q - ml;
        }
    }
}

/* Q3_K (:116-152): 110-byte super-blocks.  Bytes 0-31 high-bit mask, 32-95
 * two 32-byte chunks of 2-bit values, 96-107 the 16 signed 6-bit group scales
 * (low 4 bits: byte g, low nibble for g < 8, high nibble of byte g-8 after;
 * top 2 bits: bits 2*(g/4).. of byte 8 + g%4; minus 32), 108-109 d.  Weight j:
 * group g = j/16; low bits from chunk g/8, byte (g%2)*16 + j%16 of it, bit
 * pair (g%8)/2; mask bit g/2 of byte (g%2)*16 + j%16; q = low - 4 when the mask
 * bit is clear.  w = (d*sc)*q. */
static void oracle_dequant_q3_k(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 110;
        const uint8_t *hm = blk, *qs = blk + 32, *sc = blk + 96;
        const float d = fh3_oracle_f16_to_f32(rd16(blk + 108));
        for (int j = 0; j < 256; j++) {
            const int g = j / 16, l = j % 16;
            const int lo4 = g < 8 ? (sc[g] & 15) : (sc[g - 8] >> 4);
            const int hi2 = (sc[8 + g % 4] >> (2 * (g / 4))) & 3;
            const int scale = (lo4 | (hi2 << 4)) - 32;
            const int low = (qs[(g / 8) * 32 + (g % 2) * 16 + l] >> (2 * ((g % 8) / 2))) & 3;
            const int hbit = (hm[(g % 2) * 16 + l] >> (g / 2)) & 1;
            const float dl = d * (float)scale;
            dst[b * 256 + j] = dl * (float)(low - (hbit ? 0 : 4));
        }
    }
}

/* Q5_K (:198-236): 176-byte super-blocks.  d, dmin, 12 bytes of 6-bit scales
 * and mins packed as in Q4_K, 16-47 fifth bits (bit g of byte l for element l
 * of group g), 48-175 four 32-byte chunks of nibbles (chunk g/2, low nibble
 * for even g).  w = (d*sc)*q - dmin*m. */
static void oracle_dequant_q5_k(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 176;
        const float d = fh3_oracle_f16_to_f32(rd16(blk));
        const float dmin = fh3_oracle_f16_to_f32(rd16(blk + 2));
        uint8_t sc[8], mn[8];
        oracle_q4k_scales(blk + 4, sc, mn);
        for (int g = 0; g < 8; g++) {
            const float dl = d * (float)sc[g], ml = dmin * (float)mn[g];
            for (int l = 0; l < 32; l++) {
                const int nib = (blk[48 + (g / 2) * 32 + l] >> (4 * (g % 2))) & 15;
                const int bit5 = (blk[16 + l] >> g) & 1;
                dst[b * 256 + g * 32 + l] = dl * (float)(nib | (bit5 << 4)) - ml;
            }
        }
    }
}

/* Q6_K (:238-282): 210-byte super-blocks.  0-127 low nibbles, 128-191 high bit
 * pairs, 192-207 16 int8 group scales, 208-209 d.  Weight j: half h = j/128,
 * r = (j%128)/16, l = j%16; low nibble of byte h*64 + (r%4)*16 + l (high
 * nibble when r >= 4); bit pair r/2 of byte 128 + h*32 + (r%2)*16 + l;
 * q = (nibble | pair << 4) - 32.  w = (d*sc)*q. */
static void oracle_dequant_q6_k(const uint8_t *src, float *dst, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = src + b * 210;
        const float d = fh3_oracle_f16_to_f32(rd16(blk + 208));
        for (int j = 0; j < 256; j++) {
            const int h = j / 128, r = (j % 128) / 16, l = j % 16;
            const int nib = (blk[h * 64 + (r % 4) * 16 + l] >> (4 * (r / 4))) & 15;
            const int pair = (blk[128 + h * 32 + (r % 2) * 16 + l] >> (2 * (r / 2))) & 3;
            const float dl = d * (float)(int8_t)blk[192 + j / 16];
            dst[b * 256 + j] = dl * (float)((nib | (pair << 4)) - 32);
        }
    }
}

/* src/core/fh3_quant.c:284-318: NULL / non-positive n is a silent no-op and an
 * unsupported type writes nothing. */
void fh3_oracle_dequant(int type, const void *src, float *dst, int64_t n) {
    if (!src || !dst || n <= 0) return;
    const uint8_t *s = (const uint8_t *)src;
    switch (type) {
        case ORACLE_F32: memcpy(dst, src, (size_t)n * sizeof(float)); break;
        case 1: oracle_dequant_f16(s, dst, n); break;
        case 30: oracle_dequant_bf16(s, dst, n); break;
        case 8: oracle_dequant_q8_0(s, dst, n); break;
        case 10: oracle_dequant_q2_k(s, dst, n); break;
        case 11: oracle_dequant_q3_k(s, dst, n); break;
        case ORACLE_Q4_K: oracle_dequant_q4_k(s, dst, n); break;
        case 13: oracle_dequant_q5_k(s, dst, n); break;
        case 14: oracle_dequant_q6_k(s, dst, n); break;
        default: break;
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

/* ------------------------------------------------------------------------ */
/* The DiT block's elementwise ops around the linear layer                   */
/* (src/core/fh3_ops.c:410-585), as the reference's AVX2/FMA build computes   */
/* them: rmsnorm sums x*x in 8 fmaf lanes (element d in lane d%8) reduced by  */
/* the fixed tree, then a scalar fmaf tail; modulate and gate_residual fuse   */
/* their multiply-add on the 8-wide part of each 1024-element chunk.          */
/* ------------------------------------------------------------------------ */
void fh3_oracle_rmsnorm(float *x, const float *w, int n, int dim, float eps) {
    if (!x || !w || n <= 0 || dim <= 0) return;
    const int64_t d8 = dim - (dim % 8);
    for (int i = 0; i < n; i++) {
        float *row = x + (size_t)i * (size_t)dim;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int64_t d = 0; d < d8; d++) acc[d % 8] = fmaf(row[d], row[d], acc[d % 8]);
        float sum = oracle_tree8(acc);
        for (int64_t d = d8; d < dim; d++) sum = fmaf(row[d], row[d], sum);
        const float inv_rms = 1.0f / sqrtf(sum / (float)dim + eps);
        for (int64_t d = 0; d < dim; d++) row[d] = row[d] * inv_rms * w[d];
    }
}

/* src/core/fh3_ops.c:529-557: x = x*(1+scale) + shift, fused on the 8-wide
 * part, two roundings on a chunk's tail (the build has -ffp-contract=off). */
void fh3_oracle_modulate(float *x, const float *shift, const float *scale, int n, int dim) {
    if (!x || !shift || !scale || n <= 0 || dim <= 0) return;
    const int64_t total = (int64_t)n * (int64_t)dim;
    for (int64_t k0 = 0; k0 < total; k0 += 1024) {
        const int64_t k1 = k0 + 1024 <= total ? k0 + 1024 : total;
        const int64_t kv = k0 + ((k1 - k0) / 8) * 8;
        for (int64_t k = k0; k < kv; k++) x[k] = fmaf(x[k], 1.0f + scale[k], shift[k]);
        for (int64_t k = kv; k < k1; k++) x[k] = x[k] * (1.0f + scale[k]) + shift[k];
    }
}

/* src/core/fh3_ops.c:507-527: out[j] = val[j] * silu(gate[j]), the input row
 * being [val (F) | gate (F)]; silu(g) = g / (1 + expf(-g)), 0 below -80. */
void fh3_oracle_swiglu(const float *in, float *out, int n, int F) {
    if (!in || !out || n <= 0 || F <= 0) return;
    for (int i = 0; i < n; i++) {
        const float *val = in + (size_t)i * 2 * (size_t)F, *gate = val + F;
        for (int j = 0; j < F; j++) {
            const float g = gate[j];
            const float s = g < -80.0f ? 0.0f : g / (1.0f + expf(-g));
            out[(size_t)i * (size_t)F + j] = val[j] * s;
        }
    }
}

/* src/core/fh3_ops.c:559-585: h = fmaf(gate, y, h) element by element. */
void fh3_oracle_gate_residual(float *h, const float *gate, const float *y, int n, int dim) {
    if (!h || !gate || !y || n <= 0 || dim <= 0) return;
    const int64_t total = (int64_t)n * (int64_t)dim;
    for (int64_t k = 0; k < total; k++) h[k] = fmaf(gate[k], y[k], h[k]);
}

/* ------------------------------------------------------------------------ */
/* The attention branch's ops (src/core/fh3_ops.c:458-505,587-695).          */
/* ------------------------------------------------------------------------ */

/* src/core/fh3_ops.c:458-505: rotate the first rot_dim channels of each head
 * vector in halves, v0 = x[j], v1 = x[rot/2 + j]:
 *   x[j]         = v0*cos[j] - v1*sin[j]
 *   x[rot/2 + j] = v1*cos[rot/2 + j] + v0*sin[rot/2 + j]
 * every product and the add/sub rounded separately; cos/sin are [n][rot_dim]
 * (one row per token, shared by the heads); channels >= rot_dim untouched. */
void fh3_oracle_rope3(float *x, const float *cos, const float *sin, int n, int heads, int head_dim,
                      int rot_dim) {
    if (!x || !cos || !sin || n <= 0 || heads <= 0 || head_dim <= 0 || rot_dim <= 0 || rot_dim > head_dim ||
        (rot_dim % 2) != 0)
        return;
    const int half = rot_dim / 2;
    for (int i = 0; i < n; i++) {
        const float *c = cos + (size_t)i * (size_t)rot_dim, *s = sin + (size_t)i * (size_t)rot_dim;
        for (int h = 0; h < heads; h++) {
            float *v = x + ((size_t)i * (size_t)heads + (size_t)h) * (size_t)head_dim;
            for (int j = 0; j < half; j++) {
                const float v0 = v[j], v1 = v[half + j];
                const float a = v0 * c[j], b = v1 * s[j];
                const float e = v1 * c[half + j], f = v0 * s[half + j];
                v[j] = a - b;
                v[half + j] = e + f;
            }
        }
    }
}

/* The reference's dot_product_avx2 (src/core/fh3_ops.c:50-65): 8 fmaf lanes,
 * the fixed tree, an fmaf tail. */
static float oracle_dot(const float *x, const float *w, int64_t n) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int64_t n8 = n - (n % 8);
    for (int64_t k = 0; k < n8; k++) acc[k % 8] = fmaf(x[k], w[k], acc[k % 8]);
    float s = oracle_tree8(acc);
    for (int64_t k = n8; k < n; k++) s = fmaf(x[k], w[k], s);
    return s;
}

#define ORACLE_ATTN_TILE 64 /* src/core/fh3_ops.c:587 */

/* src/core/fh3_ops.c:589-695, one query at a time: q/o rows [nq][heads][hd],
 * k/v rows [nk][heads][hd] (the reference has nq = nk = n; a query's result
 * depends only on its own row, so a subset of queries is exact).  Scores
 * s = dot(q, k)*(1/sqrtf(hd)) over key tiles of 64; per tile m_new =
 * max(m, tile max), alpha = expf(m - m_new), l *= alpha, acc *= alpha, then
 * for each key p = expf(s - m_new), l += p, acc = fmaf(p, v, acc); finally
 * o = acc * (l > 0 ? 1/l : 0).  m starts at -1e30. */
void fh3_oracle_attention_rows(const float *q, int nq, const float *k, const float *v, int nk, float *o,
                               int heads, int hd) {
    if (!q || !k || !v || !o || nq <= 0 || nk <= 0 || heads <= 0 || hd <= 0) return;
    const float scale = 1.0f / sqrtf((float)hd);
    #pragma omp parallel
    {
        float *acc = (float *)malloc((size_t)hd * sizeof(float));
        float sc[ORACLE_ATTN_TILE];
        #pragma omp for collapse(2) schedule(static)
        for (int h = 0; h < heads; h++) {
            for (int i = 0; i < nq; i++) {
                if (!acc) continue;
                const float *qi = q + ((size_t)i * (size_t)heads + (size_t)h) * (size_t)hd;
                float *oi = o + ((size_t)i * (size_t)heads + (size_t)h) * (size_t)hd;
                float m = -1e30f, l = 0.0f;
                memset(acc, 0, (size_t)hd * sizeof(float));
                for (int j0 = 0; j0 < nk; j0 += ORACLE_ATTN_TILE) {
                    const int B = j0 + ORACLE_ATTN_TILE <= nk ? ORACLE_ATTN_TILE : nk - j0;
                    float mt = -INFINITY;
                    for (int t = 0; t < B; t++) {
                        const float *kj = k + ((size_t)(j0 + t) * (size_t)heads + (size_t)h) * (size_t)hd;
                        sc[t] = oracle_dot(qi, kj, hd) * scale;
                        if (t == 0 || sc[t] > mt) mt = sc[t];
                    }
                    const float mn = m > mt ? m : mt;
                    const float alpha = expf(m - mn);
                    l *= alpha;
                    for (int d = 0; d < hd; d++) acc[d] *= alpha;
                    for (int t = 0; t < B; t++) {
                        const float *vj = v + ((size_t)(j0 + t) * (size_t)heads + (size_t)h) * (size_t)hd;
                        const float p = expf(sc[t] - mn);
                        l += p;
                        for (int d = 0; d < hd; d++) acc[d] = fmaf(p, vj[d], acc[d]);
                    }
                    m = mn;
                }
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
                for (int d = 0; d < hd; d++) oi[d] = acc[d] * inv;
            }
        }
        free(acc);
    }
}

void fh3_oracle_attention(const float *q, const float *k, const float *v, float *o, int n, int heads, int hd) {
    fh3_oracle_attention_rows(q, n, k, v, n, o, heads, hd);
}

/* ------------------------------------------------------------------------ */
/* Video sparse attention (src/core/fh3_vsa.c:31-507).                       */
/* ------------------------------------------------------------------------ */

/* Tile geometry (src/core/fh3_vsa.c:31-163): text tokens, then audio tokens,
 * in runs of `tile`; then the video grid (gt, gh, gw) in 4x4x4 cubes, t-major,
 * tokens of a cube in (t, h, w) order.  Modalities that do not sum to n make
 * every token video; a grid that does not match the video count becomes
 * 1 x 1 x V.  Writes tile_tok[n] (token of each position), tile_off[T + 1]
 * and returns T (or -1); *n_prefix gets the number of text + audio tiles. */
int fh3_oracle_vsa_geometry(int n, int num_text, int num_audio, int num_video, int grid_t, int grid_h,
                            int grid_w, int tile, int *tile_tok, int *tile_off, int max_tiles, int *n_prefix) {
    if (n <= 0) return -1;
    if (tile <= 0) tile = 64;
    int T = num_text > 0 ? num_text : 0, A = num_audio > 0 ? num_audio : 0, V = num_video > 0 ? num_video : 0;
    if (T + A + V != n) T = 0, A = 0, V = n;
    int gt = grid_t, gh = grid_h, gw = grid_w;
    if (gt <= 0 || gh <= 0 || gw <= 0 || gt * gh * gw != V) gt = 1, gh = 1, gw = V;
    int nt = 0, pos = 0;
    tile_off[0] = 0;
    const int seg_len[2] = {T, A}, seg_start[2] = {0, T};
    for (int sgi = 0; sgi < 2; sgi++) {
        for (int s0 = 0; s0 < seg_len[sgi]; s0 += tile) {
            const int sz = seg_len[sgi] - s0 < tile ? seg_len[sgi] - s0 : tile;
            if (nt >= max_tiles) return -1;
            for (int e = 0; e < sz; e++) tile_tok[pos++] = seg_start[sgi] + s0 + e;
            tile_off[++nt] = pos;
        }
    }
    *n_prefix = nt;
    if (V > 0) {
        const int base = T + A;
        for (int t0 = 0; t0 < gt; t0 += 4)
            for (int h0 = 0; h0 < gh; h0 += 4)
                for (int w0 = 0; w0 < gw; w0 += 4) {
                    if (nt >= max_tiles) return -1;
                    for (int t = t0; t < gt && t < t0 + 4; t++)
                        for (int h = h0; h < gh && h < h0 + 4; h++)
                            for (int w = w0; w < gw && w < w0 + 4; w++)
                                tile_tok[pos++] = base + (t * gh + h) * gw + w;
                    tile_off[++nt] = pos;
                }
    }
    return nt;
}

typedef struct {
    float s;
    int j;
} OracleTileScore;

/* descending score, then ascending tile index (src/core/fh3_vsa.c:178-184) */
static int oracle_tile_cmp(const void *a, const void *b) {
    const OracleTileScore *x = (const OracleTileScore *)a, *y = (const OracleTileScore *)b;
    if (x->s > y->s) return -1;
    if (x->s < y->s) return 1;
    return x->j < y->j ? -1 : (x->j > y->j ? 1 : 0);
}

/* src/core/fh3_vsa.c:186-507 on [n][heads][hd] rows.  Per tile: mean-pooled
 * q, k (and v with a gate) accumulated as pool += x * (1/count) in tile order;
 * tile scores dot(qpool, kpool) * (1/sqrtf(hd)) with separate roundings.
 * Query tiles of text/audio attend to every tile; a video query tile attends
 * to every prefix tile plus its top ceil((1 - sparsity) * video tiles) video
 * tiles (all of them when sparsity <= 0 or that count covers them).  Fine
 * attention per query over the selected tiles' tokens in tile order: max,
 * sum of expf, weights p * (1/sum), out += w * v.  With a gate, each tile's
 * softmax over all tile scores mixes the pooled v, and
 * o = fine + coarse * gate.  Returns 0, or -1 when the geometry fails. */
int fh3_oracle_vsa_attention(int tile, float sparsity, const float *q, const float *k, const float *v,
                             const float *gate, float *o, int n, int num_text, int num_audio, int num_video,
                             int grid_t, int grid_h, int grid_w, int heads, int hd) {
    if (!q || !k || !v || !o || n <= 0 || heads <= 0 || hd <= 0) return -1;
    if (tile <= 0) tile = 64;
    const int max_tiles = n + 8;
    int *tok = (int *)malloc((size_t)n * sizeof(int));
    int *off = (int *)malloc((size_t)(max_tiles + 1) * sizeof(int));
    int P = 0;
    const int T = tok && off ? fh3_oracle_vsa_geometry(n, num_text, num_audio, num_video, grid_t, grid_h, grid_w,
                                                       tile, tok, off, max_tiles, &P)
                             : -1;
    if (T <= 0) {
        free(tok);
        free(off);
        return -1;
    }
    const int NV = T - P;
    const size_t TD = (size_t)T * (size_t)hd, HTD = (size_t)heads * TD;
    float *qp = (float *)calloc(HTD, sizeof(float)), *kp = (float *)calloc(HTD, sizeof(float));
    float *vp = gate ? (float *)calloc(HTD, sizeof(float)) : NULL;
    float *sc = (float *)malloc((size_t)heads * (size_t)T * (size_t)T * sizeof(float));
    uint8_t *sel = (uint8_t *)calloc((size_t)heads * (size_t)T * (size_t)T, 1);
    float *fine = (float *)calloc((size_t)n * (size_t)heads * (size_t)hd, sizeof(float));
    int rc = (qp && kp && (!gate || vp) && sc && sel && fine) ? 0 : -1;
    const float scale = 1.0f / sqrtf((float)hd);
    if (rc == 0) {
        /* pooling */
        for (int i = 0; i < T; i++) {
            const int cnt = off[i + 1] - off[i];
            const float inv = 1.0f / (float)cnt;
            for (int r = 0; r < cnt; r++) {
                const int t = tok[off[i] + r];
                for (int h = 0; h < heads; h++) {
                    const size_t src = ((size_t)t * heads + h) * hd, dst = (size_t)h * TD + (size_t)i * hd;
                    for (int d = 0; d < hd; d++) {
                        qp[dst + d] += q[src + d] * inv;
                        kp[dst + d] += k[src + d] * inv;
                        if (gate) vp[dst + d] += v[src + d] * inv;
                    }
                }
            }
        }
        /* tile scores */
        for (int h = 0; h < heads; h++)
            for (int i = 0; i < T; i++)
                for (int j = 0; j < T; j++) {
                    const float *a = qp + (size_t)h * TD + (size_t)i * hd, *b = kp + (size_t)h * TD + (size_t)j * hd;
                    float dot = 0.0f;
                    for (int d = 0; d < hd; d++) dot += a[d] * b[d];
                    sc[((size_t)h * T + i) * T + j] = dot * scale;
                }
        /* tile selection */
        int kv = 0;
        if (NV > 0) {
            kv = (int)ceilf((1.0f - sparsity) * (float)NV);
            if (kv < 1) kv = 1;
            if (kv > NV) kv = NV;
        }
        const int all = sparsity <= 0.0f || kv == NV;
        OracleTileScore *cand = (OracleTileScore *)malloc((size_t)(NV > 0 ? NV : 1) * sizeof(OracleTileScore));
        if (!cand) rc = -1;
        for (int h = 0; h < heads && rc == 0; h++)
            for (int i = 0; i < T; i++) {
                uint8_t *row = sel + ((size_t)h * T + i) * T;
                if (i < P || all) {
                    memset(row, 1, (size_t)T);
                    continue;
                }
                memset(row, 1, (size_t)P);
                for (int j = 0; j < NV; j++) {
                    cand[j].s = sc[((size_t)h * T + i) * T + P + j];
                    cand[j].j = P + j;
                }
                qsort(cand, (size_t)NV, sizeof(OracleTileScore), oracle_tile_cmp);
                for (int e = 0; e < kv; e++) row[cand[e].j] = 1;
            }
        free(cand);
    }
    if (rc == 0) {
        /* fine attention */
        int *kt = (int *)malloc((size_t)n * sizeof(int));
        float *s = (float *)malloc((size_t)n * sizeof(float)), *p = (float *)malloc((size_t)n * sizeof(float));
        if (!kt || !s || !p) rc = -1;
        for (int h = 0; h < heads && rc == 0; h++)
            for (int i = 0; i < T; i++) {
                const uint8_t *row = sel + ((size_t)h * T + i) * T;
                int nk = 0;
                for (int j = 0; j < T; j++)
                    if (row[j])
                        for (int e = off[j]; e < off[j + 1]; e++) kt[nk++] = tok[e];
                for (int e = off[i]; e < off[i + 1] && nk > 0; e++) {
                    const int tq = tok[e];
                    const float *qi = q + ((size_t)tq * heads + h) * hd;
                    float mx = -1e30f;
                    for (int m = 0; m < nk; m++) {
                        const float *kj = k + ((size_t)kt[m] * heads + h) * hd;
                        float dot = 0.0f;
                        for (int d = 0; d < hd; d++) dot += qi[d] * kj[d];
                        s[m] = dot * scale;
                        if (s[m] > mx) mx = s[m];
                    }
                    float sum = 0.0f;
                    for (int m = 0; m < nk; m++) {
                        p[m] = expf(s[m] - mx);
                        sum += p[m];
                    }
                    const float inv = 1.0f / sum;
                    float *out = fine + ((size_t)tq * heads + h) * hd;
                    for (int m = 0; m < nk; m++) {
                        const float w = p[m] * inv;
                        const float *vj = v + ((size_t)kt[m] * heads + h) * hd;
                        for (int d = 0; d < hd; d++) out[d] += w * vj[d];
                    }
                }
            }
        free(kt);
        free(s);
        free(p);
    }
    if (rc == 0) {
        const size_t total = (size_t)n * (size_t)heads * (size_t)hd;
        if (!gate) {
            memcpy(o, fine, total * sizeof(float));
        } else {
            float *oc = (float *)malloc((size_t)hd * sizeof(float));
            if (!oc) rc = -1;
            for (int i = 0; i < T && rc == 0; i++)
                for (int h = 0; h < heads; h++) {
                    const float *srow = sc + ((size_t)h * T + i) * T;
                    float mx = -1e30f;
                    for (int j = 0; j < T; j++)
                        if (srow[j] > mx) mx = srow[j];
                    float sum = 0.0f;
                    for (int j = 0; j < T; j++) sum += expf(srow[j] - mx);
                    const float inv = 1.0f / sum;
                    memset(oc, 0, (size_t)hd * sizeof(float));
                    for (int j = 0; j < T; j++) {
                        const float w = expf(srow[j] - mx) * inv;
                        const float *pv = vp + (size_t)h * TD + (size_t)j * hd;
                        for (int d = 0; d < hd; d++) oc[d] += w * pv[d];
                    }
                    for (int e = off[i]; e < off[i + 1]; e++) {
                        const size_t at = ((size_t)tok[e] * heads + h) * hd;
                        for (int d = 0; d < hd; d++) o[at + d] = fine[at + d] + oc[d] * gate[at + d];
                    }
                }
            free(oc);
        }
    }
    free(tok);
    free(off);
    free(qp);
    free(kp);
    free(vp);
    free(sc);
    free(sel);
    free(fine);
    return rc;
}
