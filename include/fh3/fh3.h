/*
 * fh3.h -- the fh3 entry points of the Q4_K linear-layer path, served by the
 * MI355X (gfx950) library libfh3hip.so.
 *
 * Types and signatures keep the reference's ABI so existing C callers link
 * unchanged; each declaration cites the reference interface it replaces
 * (paths relative to the fh3 repository root).  Every compute entry point
 * here runs on the GPU; there is no CPU fallback in this library.  When no
 * HIP device can be initialised the call prints a diagnostic to stderr, leaves
 * its outputs unwritten, and fh3_hip_last_error() says why.
 */
#ifndef FH3_H
#define FH3_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML/GGUF tensor type ids (reference include/fh3/fh3.h:63-79). */
typedef enum {
    FH3_QUANT_F32  = 0,
    FH3_QUANT_F16  = 1,
    FH3_QUANT_Q4_0 = 2,
    FH3_QUANT_Q4_1 = 3,
    FH3_QUANT_Q5_0 = 6,
    FH3_QUANT_Q5_1 = 7,
    FH3_QUANT_Q8_0 = 8,
    FH3_QUANT_Q8_1 = 9,
    FH3_QUANT_Q2_K = 10,
    FH3_QUANT_Q3_K = 11,
    FH3_QUANT_Q4_K = 12,
    FH3_QUANT_Q5_K = 13,
    FH3_QUANT_Q6_K = 14,
    FH3_QUANT_Q8_K = 15,
    FH3_QUANT_BF16 = 30
} Fh3QuantType;

/* A weight matrix W[out][in] stored row-major in `type` blocks
 * (reference include/fh3/fh3.h:82-87).  For the HIP entry points taking a
 * device matrix, `data` is a device pointer. */
typedef struct Fh3W {
    int type;
    int64_t in;
    int64_t out;
    const uint8_t *data;
} Fh3W;

/* Video sparse attention settings (reference include/fh3/fh3.h:41-44):
 * tile <= 0 means 64; sparsity is the share of video key tiles dropped. */
typedef struct Fh3VsaCfg {
    int tile;
    float sparsity;
} Fh3VsaCfg;

/* The reference's sequence descriptor (src/model/fh3_seq.h:32-45; opaque in
 * its fh3.h).  Laid out identically so a caller's Fh3Seq passes unchanged;
 * the attention calls read only the counts and the video grid. */
typedef struct Fh3Seq {
    int seq_len;     /* N = num_text + num_audio + num_video */
    int num_text;
    int num_audio;
    int num_video;
    int grid_t;      /* video grid (t, h, w) in tokens */
    int grid_h;
    int grid_w;
    int *tags;
    int *pair_index;
    double *pos;
    float *cos;      /* [N][96] rope tables */
    float *sin;
} Fh3Seq;

/* Per-layer tensor views into a packed trunk layer
 * (reference include/fh3/fh3.h:90-100; run order src/io/fh3_pack.h:26-37). */
typedef struct Fh3LayerView {
    Fh3W qkv;
    Fh3W gate_compress;
    Fh3W out;
    Fh3W fc1;
    Fh3W fc2;
    Fh3W norm1;
    Fh3W norm2;
    Fh3W q_norm;
    Fh3W k_norm;
} Fh3LayerView;

/* Return codes (reference include/fh3/fh3.h:218-226). */
#define FH3_OK              0
#define FH3_ERR           (-1)
#define FH3_E_IO          (-2)
#define FH3_E_TRUNCATED   (-3)
#define FH3_E_BAD_MAGIC   (-4)
#define FH3_E_BAD_VERSION (-5)
#define FH3_E_NOT_FOUND   (-6)
#define FH3_E_NOMEM       (-7)
#define FH3_E_INVALID     (-8)

/* Bytes of one row of n elements of `type`; 0 for n <= 0 or an unknown type.
 * Replaces src/core/fh3_quant.c:14-34 (same table, Q4_K = ceil(n/256)*144). */
size_t fh3_row_bytes(int type, int64_t n);

/* Dequantise n elements of one row from host memory to host fp32, on the GPU.
 * F32, F16, BF16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K are decoded
 * bit-identically to the reference; block types write only whole blocks
 * (n/32 for Q8_0, n/256 for the K types), as the reference does.  Other types
 * print "unsupported type" and write nothing.  NULL pointers or n <= 0 are a
 * silent no-op.  Replaces src/core/fh3_quant.c:36-318. */
void fh3_dequant(int type, const void *src, float *dst, int64_t n);

/* y[n_tok][out] = x[n_tok][in] * W^T (+ bias[out]) on host buffers, computed
 * on the GPU (inputs are copied in and y out on every call).  NULL pointers or
 * non-positive sizes are a silent no-op, as in the reference.  Weight types:
 * every type fh3_dequant decodes (Q4_K, Q5_K and Q6_K rows of up to 32768
 * values read in place by the product kernels; F32, F16, BF16, Q8_0, Q2_K,
 * Q3_K and longer rows decoded per call to fp16 rows).  in is any
 * length for F32, F16 and BF16 (e.g. the DiT's 32- and 96-value patch rows),
 * a multiple of 32 for Q8_0 and of 256 for the K types (whole blocks, the
 * rows the reference defines), up to 2^24; other types or in print an error
 * and leave y unwritten.  Results are
 * deterministic run to run; they match the CPU path within rel-Frobenius 2e-3
 * (fp16 or int16 operands, fp32 accumulation).  Replaces
 * src/core/fh3_ops.c:317-404. */
void fh3_matmul(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null);

/* The reference's single-thread variants (src/core/fh3_ops.c:210-315) are
 * bitwise-equal to fh3_matmul by contract; here they run the same GPU path. */
void fh3_matmul_scalar(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null);
void fh3_matmul_avx2(const Fh3W *w, const float *x, float *y, int n_tok, const float *bias_or_null);

/* Dense attention on host buffers q, k, v, o [n][heads][hd], computed on the
 * GPU (copied in and out on every call): softmax(q.k^T / sqrt(hd)) v over all
 * n keys per head, no mask.  NULL pointers or non-positive sizes are a silent
 * no-op, as in the reference; head dims other than 64 and 128 print
 * "not supported" and leave o unwritten.  fp16 operands with fp32
 * accumulation and an fp32 online softmax: within rel-Frobenius 2e-3 of the
 * CPU result.  Replaces src/core/fh3_ops.c:589-695 (declared at
 * include/fh3/fh3.h:117 there). */
void fh3_attention(const float *q, const float *k, const float *v, float *o, int n, int heads, int hd);

/* Video sparse attention on host buffers q, k, v, gate (may be NULL), o
 * [n][heads][head_dim], computed on the GPU (copied in and out on every call):
 * per 64-token tile (text and audio runs, then 4x4x4 video cubes) mean-pooled
 * q/k scores pick each video query tile's top (1 - sparsity) share of video
 * key tiles (text/audio tiles always kept), fine attention runs over the
 * chosen tiles, and with a gate a softmax over all tile scores mixes the
 * pooled v in: o = fine + coarse * gate.  The tile statistics are computed in
 * the reference's order, so the tile choice is the CPU's; the attention itself
 * matches within rel-Frobenius 2e-3.  NULL pointers or non-positive sizes are
 * a silent no-op; head dims other than 64/128, tiles above 64 or more than
 * 4096 tiles print "not supported" and leave o unwritten.  Replaces
 * src/core/fh3_vsa.c:186-507 (declared at include/fh3/fh3.h:118 there). */
void fh3_vsa_attention(const Fh3VsaCfg *c, const float *q, const float *k, const float *v, const float *gate,
                       float *o, const Fh3Seq *seq, int heads, int head_dim);

#ifdef __cplusplus
}
#endif

#endif /* FH3_H */
