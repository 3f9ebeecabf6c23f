/*
 * fh3_synth.h -- seeded synthetic inputs for the Q4_K linear layer: a Q4_K
 * encoder and the activation/weight distributions the benchmark workloads are
 * defined on.  Host C99 with OpenMP.
 *
 * The reference ships no Q4_K encoder (it only decodes, src/core/fh3_quant.c:
 * 154-196); fh3_q4k_quantize is this library's own.  The GPU path and the CPU
 * checker always consume the same encoded bytes, so parity never depends on
 * the encoder; its own tests check format validity and round-trip error.
 */
#ifndef FH3_SYNTH_H
#define FH3_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Philox4x32-10 block function (Salmon, Moraes, Dror, Shaw, SC'11):
 * out = philox(ctr, key) with 10 rounds and Weyl key schedule. */
void fh3_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Seeded N(0,1) fp32 generator: Philox4x32-10 (Salmon et al., SC'11) with
 * Box-Muller, one counter per 4 outputs; the same stream, bit for bit, as the
 * reference's fh3_rng_normal (src/model/fh3_sched.c:110-159).  Exported under
 * its own name so that it never interposes on the reference's symbol when
 * both are linked into one program. */
void fh3_synth_rng_normal(uint64_t seed, uint64_t stream, float *out, size_t n);

/* Uniform (0,1) fp32 from the same counter stream layout as fh3_synth_rng_normal:
 * block b of stream s yields 4 values (word + 0.5) / 2^32. */
void fh3_rng_uniform(uint64_t seed, uint64_t stream, float *out, size_t n);

/* Encode rows x n fp32 (n % 256 == 0) into Q4_K rows of fh3_row_bytes(Q4_K, n)
 * bytes.  Per 32-weight group: offset = -min(0, min w), step = (max - min')/15;
 * d and dmin = largest step / offset over the super-block / 63 rounded to fp16;
 * 6-bit sc, m = round(step/d), round(offset/dmin); q = round((w + dmin*m)/(d*sc))
 * clamped to 0..15.  Returns FH3_OK or FH3_E_INVALID. */
int fh3_q4k_quantize(const float *src, int64_t rows, int64_t n, uint8_t *dst);

/* fp32 -> fp16 bits, round to nearest even (overflow -> inf, NaN kept). */
uint16_t fh3_f32_to_f16(float f);

/* Seeded workload generators.  `stream` picks an independent Philox stream.
 *   fh3_synth_q4k_weights: rows x n weights ~ N(0, sigma); when
 *     spread_decades > 0 every 256-weight super-block is scaled by
 *     10^U(-spread/2, spread/2) before encoding.  Writes Q4_K rows to dst.
 *   fh3_synth_x_normal:   N(0,1).
 *   fh3_synth_x_outliers: N(0,1) with a fraction `frac` of entries set to
 *     +-8 (sign and position seeded).
 *   fh3_synth_x_silu_gated: a * silu(b), a, b ~ N(0,1) independent -- the
 *     input of a SwiGLU down projection. */
int fh3_synth_q4k_weights(uint64_t seed, uint64_t stream, int64_t rows, int64_t n, float sigma,
                          float spread_decades, uint8_t *dst);
void fh3_synth_x_normal(uint64_t seed, uint64_t stream, float *x, size_t count);
void fh3_synth_x_outliers(uint64_t seed, uint64_t stream, float *x, size_t count, float frac);
void fh3_synth_x_silu_gated(uint64_t seed, uint64_t stream, float *x, size_t count);

#ifdef __cplusplus
}
#endif

#endif /* FH3_SYNTH_H */
