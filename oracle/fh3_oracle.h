/*
 * fh3_oracle.h -- CPU restatement of fh3's block dequantisation (every type
 * src/core/fh3_quant.c decodes) and of its Q4_K weight-stationary matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product in fasth3inc_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or the
 * timed CPU baseline -- never as a compute path of the product.
 *
 * Every function restates the arithmetic of the reference file:line it cites
 * (paths relative to the fh3 repository root).  The restatement is pinned by:
 *   - tests/golden/Q4_K.bin and tests/golden/quant/<TYPE>.bin for F16, BF16,
 *     Q8_0, Q2_K, Q3_K, Q5_K, Q6_K (gguf-py dequantize output, bit-exact)
 *   - tests/golden/matmul_ref.bin (fp64 NumPy product, rel-L2 <= 1e-6)
 *   - tests/golden/ref_vectors.npz and live calls into oracle/_ref (the
 *     reference's own fh3_quant.c + fh3_ops.c compiled by oracle/Makefile),
 *     bitwise, for the matmul and for every decoder on random blocks
 *   - closed-form cases in tests/test_oracle.py (fp16 decode of every bit
 *     pattern, all 64x64 scale/min decodings, brute-force small products).
 * Nothing in this file is "parity unpinned".
 */
#ifndef FH3_ORACLE_H
#define FH3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as the reference's Fh3W (include/fh3/fh3.h:82-87). */
typedef struct Fh3OracleW {
    int type;
    int64_t in;
    int64_t out;
    const uint8_t *data;
} Fh3OracleW;

/* src/core/fh3_quant.h:20-41 -- exact fp16 -> fp32 (F16C semantics). */
float fh3_oracle_f16_to_f32(uint16_t h);

/* src/core/fh3_quant.c:14-34 -- bytes of one weight row, every type id. */
size_t fh3_oracle_row_bytes(int type, int64_t n);

/* src/core/fh3_quant.c:36-282 (per-type decoders) and :284-318 (dispatch):
 * F32, F16, BF16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K; other ids write nothing. */
void fh3_oracle_dequant(int type, const void *src, float *dst, int64_t n);

/* src/core/fh3_ops.c:317-404 -- OpenMP over 64-row output tiles.  Output bits
 * equal the reference's fh3_matmul / _scalar / _avx2 (fh3_ops.c:210-315). */
void fh3_oracle_matmul(const Fh3OracleW *w, const float *x, float *y,
                       int n_tok, const float *bias_or_null);

/* Same arithmetic, restricted to output rows [o_begin, o_end) of W; y keeps
 * the full [n_tok][w->out] layout and only those columns are written.  Used to
 * check large shapes on a seeded subset of outputs (rows are independent). */
void fh3_oracle_matmul_rows(const Fh3OracleW *w, const float *x, float *y,
                            int n_tok, const float *bias_or_null,
                            int64_t o_begin, int64_t o_end);

/* Number of OpenMP threads the oracle runs with (omp_get_max_threads()). */
int fh3_oracle_threads(void);

/* The DiT block's elementwise ops around the linear layer, as the reference's
 * AVX2/FMA build computes them (bitwise):
 *   src/core/fh3_ops.c:410-456 rmsnorm, :529-557 modulate, :507-527 swiglu,
 *   :559-585 gate_residual. */
void fh3_oracle_rmsnorm(float *x, const float *w, int n, int dim, float eps);
void fh3_oracle_modulate(float *x, const float *shift, const float *scale, int n, int dim);
void fh3_oracle_swiglu(const float *in, float *out, int n, int F);
void fh3_oracle_gate_residual(float *h, const float *gate, const float *y, int n, int dim);

/* Attention branch (src/core/fh3_ops.c:458-505,587-695): rope3 in place on
 * x[n][heads][head_dim] with cos/sin [n][rot_dim]; dense attention over
 * [n][heads][hd] rows.  fh3_oracle_attention_rows computes nq queries
 * against nk keys (the reference's result for those query rows). */
void fh3_oracle_rope3(float *x, const float *cos, const float *sin, int n, int heads, int head_dim,
                      int rot_dim);
void fh3_oracle_attention(const float *q, const float *k, const float *v, float *o, int n, int heads, int hd);
void fh3_oracle_attention_rows(const float *q, int nq, const float *k, const float *v, int nk, float *o,
                               int heads, int hd);

/* Video sparse attention (src/core/fh3_vsa.c): the tile geometry and the
 * whole call.  The sequence is given by its counts and video grid (the fields
 * of the reference's Fh3Seq that the call reads). */
int fh3_oracle_vsa_geometry(int n, int num_text, int num_audio, int num_video, int grid_t, int grid_h,
                            int grid_w, int tile, int *tile_tok, int *tile_off, int max_tiles, int *n_prefix);
int fh3_oracle_vsa_attention(int tile, float sparsity, const float *q, const float *k, const float *v,
                             const float *gate, float *o, int n, int num_text, int num_audio, int num_video,
                             int grid_t, int grid_h, int grid_w, int heads, int hd);

#ifdef __cplusplus
}
#endif

#endif /* FH3_ORACLE_H */
