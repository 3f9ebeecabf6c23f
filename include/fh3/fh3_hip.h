/*
 * fh3_hip.h -- C-ABI of the MI355X (gfx950) HIP module behind the fh3 Q4_K
 * linear layer.  Plain pointers and sizes only; streams are passed as the
 * opaque `void *` of a hipStream_t (NULL = the module's compute stream).
 *
 * These entry points have no counterpart in the CPU-only reference; they are
 * the device-resident form of src/core/fh3_ops.c:317-404 (fh3_matmul) and
 * src/core/fh3_quant.c:154-196 (dequant_q4_k) that the host wrappers in fh3.h
 * and the trunk streamer in fh3_trunk.h are built on.  All return FH3_OK or a
 * negative FH3_* code; fh3_hip_last_error() describes the last failure.
 */
#ifndef FH3_HIP_H
#define FH3_HIP_H

#include <stddef.h>
#include <stdint.h>
#include "fh3/fh3.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Select and initialise a device; creates the compute stream.  Idempotent for
 * the same device.  Every other entry point initialises device 0 (or the one
 * named by the FH3_HIP_DEVICE environment variable) on first use. */
int fh3_hip_init(int device);
/* Release streams and library-owned device buffers. */
void fh3_hip_shutdown(void);
/* Text of the last error raised in this thread ("" when none). */
const char *fh3_hip_last_error(void);
/* The library's compute stream (a hipStream_t) after initialisation, else NULL. */
void *fh3_hip_stream(void);

/* Device memory helpers (synchronous).  fh3_hip_free called on a thread
 * between fh3_hip_graph_begin and fh3_hip_graph_end is carried out by
 * fh3_hip_graph_end (a free during the capture would end it with an error). */
int fh3_hip_malloc(void **dptr, size_t bytes);
int fh3_hip_free(void *dptr);
int fh3_hip_memcpy_htod(void *dst, const void *src, size_t bytes);
int fh3_hip_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int fh3_hip_memcpy_dtod(void *dst, const void *src, size_t bytes);
int fh3_hip_memset(void *dptr, int value, size_t bytes);
int fh3_hip_synchronize(void);

/* Bit-exact fp32 dequantisation of `rows` rows of n elements each, rows
 * spaced fh3_row_bytes(type, n) apart in d_src, written densely to d_dst
 * [rows][n].  Types F32, F16, BF16, Q8_0 (n % 32 == 0), Q2_K, Q3_K, Q4_K, Q5_K,
 * Q6_K (n % 256 == 0); pointers 16-byte aligned.  Same bits as
 * src/core/fh3_quant.c:36-282.  FH3_E_INVALID for another type or size. */
int fh3_hip_dequant_dev(int type, const void *d_src, float *d_dst, int64_t rows, int64_t n,
                        void *stream);

/* Device-resident fh3_matmul: d_y[n_tok][w->out] = d_x[n_tok][w->in] * W^T
 * (+ d_bias).  w->data is a device pointer to the packed rows (16-byte
 * aligned; d_x 16-byte aligned, d_y and d_bias any float pointer: a 16-byte
 * aligned d_y with out % 4 == 0 takes the faster full-block stores of the
 * large-M kernel).  w->in: any length up to 2^24 for F32, F16 and BF16, a
 * multiple of 32 for Q8_0, of 256 for the K types (FH3_E_INVALID otherwise).
 * Q4_K rows of whole super-blocks up to 32768 values run the kernels described
 * here, and Q5_K / Q6_K rows of that kind are read in place too (the
 * FH3_HIP_PATH_SKINNY kernel up to 64 tokens, FH3_HIP_PATH_GEMM above); the
 * other types fh3_dequant decodes, and rows of any type with in % 256 != 0 or
 * in > 32768, are first decoded to fp16 rows of round_up(in, 256) columns,
 * zero-padded (the exact value rounded once; F16 used as it is where
 * in % 256 == 0), into a library buffer of out * round_up(in, 256) * 2 bytes,
 * then multiplied with the same activation handling (zeros past in) and fp32
 * accumulation.  Work is enqueued on `stream` and the call
 * returns without synchronising.  For one to four tokens (FH3_HIP_PATH_GEMV8
 * below) activations are quantised to int16 inside the product kernel and
 * weights enter an integer MFMA exactly; otherwise activations are converted to
 * fp16 with a per-row power-of-two scale and weights enter an fp16 MFMA (exact
 * sc*q for n_tok <= 64, dequantised in fp32 and rounded once to fp16 above),
 * with fp32 accumulation.  Deterministic: no atomics, fixed reduction order.
 * A NaN or infinity in a token's activations makes every output of that
 * token non-finite (NaN on the GEMV8 path), as in the reference, and leaves
 * the other tokens' outputs as they would be without it.
 * Except on the GEMV8 path, uses a library-owned workspace of about
 * n_tok * in * 2 bytes, plus S * n_tok * out * 4 bytes of partial sums where
 * K is split (the FH3_HIP_PATH_MIDM path, S <= in / 512; the GEMM path when
 * its 256 x 128 tiles number fewer than about 512, S <= in / 512 and
 * S * tiles <= 4096); calls that overlap on different streams race on it.  Q4_K, Q5_K and Q6_K products of more than 64
 * tokens need out * row_bytes < 2^32 (32-bit row offsets; 7.6e9 Q4_K weights). */
int fh3_hip_matmul_dev(const Fh3W *w, const float *d_x, float *d_y, int n_tok,
                       const float *d_bias_or_null, void *stream);

/* The two stages of fh3_hip_matmul_dev, for callers that feed one activation
 * matrix to several weight matrices (the DiT's qkv and gate_compress read the
 * same normalised rows) or that time the product kernel alone.
 *   fh3_hip_prepared_bytes: device bytes a prepared buffer for n_tok x in
 *     needs (fragments of round_up(n_tok, 256) rows by round_up(in, 256)
 *     columns, fp16, plus one fp32 scale per row, plus for n_tok <= 64 and
 *     rows of whole super-blocks one fp32 sum per 32-value group);
 *   fh3_hip_prepare_x_dev: fill d_prep (16-byte aligned) from d_x[n_tok][in];
 *   fh3_hip_matmul_prepared_dev: the product from a prepared buffer; same
 *     results as fh3_hip_matmul_dev.  Its only library workspace is the
 *     partial sums of the split-K kernels: the FH3_HIP_PATH_MIDM path, and
 *     the FH3_HIP_PATH_GEMM path while its 256 x 128 tiles number fewer than
 *     about 512 (roughly 65..2048 tokens; fh3_hip_matmul_workspace_bytes
 *     gives the exact size).  Weights of a type other than Q4_K also use the
 *     fp16-row buffer.  (For the FH3_HIP_PATH_GEMV8 shapes the prepared form
 *     is a copy of x; it is valid only while fh3_hip_set_path keeps the
 *     setting it was prepared under.  The fragment form, with its group sums,
 *     is valid under any setting.) */
size_t fh3_hip_prepared_bytes(int n_tok, int64_t in);
int fh3_hip_prepare_x_dev(const float *d_x, int n_tok, int64_t in, void *d_prep, void *stream);
int fh3_hip_matmul_prepared_dev(const Fh3W *w, const void *d_prep, float *d_y, int n_tok,
                                const float *d_bias_or_null, void *stream);

/* The DiT block around its linears (reference src/model/fh3_dit.c:383-439),
 * fused on the device.
 *
 * Prologue: fh3_hip_prepare_x_norm_dev fills a prepared buffer (as
 * fh3_hip_prepare_x_dev) from rows first normalised by rmsnorm with weight
 * d_norm_w[in] and eps (src/core/fh3_ops.c:410-456), then, when d_shift and
 * d_scale ([n_tok][in]) are both set, AdaLN-modulated
 * x*(1+scale)+shift (src/core/fh3_ops.c:529-557): one launch in place of
 * fh3_rmsnorm + fh3_modulate + the activation preparation.  Sums run in a
 * different order than the CPU's (fp32), then the usual fp16 / int16
 * conversion.  fh3_hip_rownorm_dev writes the same normalised rows as fp32
 * (d_y may equal d_x): the device form of fh3_rmsnorm (+ fh3_modulate).
 *
 * Epilogues, Q4_K weights, on the product fh3_hip_matmul_dev would compute
 * (bias included):
 *   FH3_EPI_GATE_RESIDUAL  d_out[n_tok][out] += d_aux[n_tok][out] * y
 *                          (fh3_gate_residual, src/core/fh3_ops.c:559-585);
 *   FH3_EPI_SWIGLU         the weight's rows are [val (F) | gate (F)],
 *                          out = 2F with out % 128 == 0;
 *                          d_out[n_tok][F] = val * silu(gate)
 *                          (fh3_swiglu, src/core/fh3_ops.c:507-527).
 * Each replaces a product and an elementwise pass over its output. */
#define FH3_EPI_NONE          0
#define FH3_EPI_GATE_RESIDUAL 1
#define FH3_EPI_SWIGLU        2
int fh3_hip_prepare_x_norm_dev(const float *d_x, int n_tok, int64_t in, const float *d_norm_w, float eps,
                               const float *d_shift, const float *d_scale, void *d_prep, void *stream);
int fh3_hip_rownorm_dev(const float *d_x, int n_tok, int64_t in, const float *d_norm_w, float eps,
                        const float *d_shift, const float *d_scale, float *d_y, void *stream);
int fh3_hip_matmul_epi_dev(const Fh3W *w, const float *d_x, int n_tok, const float *d_bias_or_null, int epi,
                           const float *d_aux, float *d_out, void *stream);
int fh3_hip_matmul_prepared_epi_dev(const Fh3W *w, const void *d_prep, int n_tok, const float *d_bias_or_null,
                                    int epi, const float *d_aux, float *d_out, void *stream);

/* The DiT block's attention branch (reference src/model/fh3_dit.c:390-411)
 * on the device.
 *
 * fh3_hip_attention_dev: dense attention over device arrays q, k, v, o
 * [n][heads][hd] (fh3_attention, src/core/fh3_ops.c:589-695).
 *
 * fh3_hip_attention_qkv_dev: the same, reading q, k and v in place from the
 * qkv projection's output d_qkv [n][3 * heads * hd] (no split copies, cf.
 * fh3_dit.c:390-395), with q and k first rmsnorm'ed per head by d_qnorm_w /
 * d_knorm_w [hd] and eps (both or neither; fh3_dit.c:397-398) and rotated by
 * rope3 on their first rot_dim channels with d_cos / d_sin [n][rot_dim] (both
 * or neither; fh3_rope3, src/core/fh3_ops.c:458-505; fh3_dit.c:400-401).
 *
 * hd must be 64 or 128; pointers 16-byte aligned.  Operands are fp16 with
 * fp32 accumulation and an fp32 online softmax (rel-Frobenius <= 2e-3 against
 * the CPU sequence).  The fp16 operands live in a library workspace
 * (6 * heads * round_up(n, 128) * hd bytes): calls that overlap on different
 * streams must not share it. */
int fh3_hip_attention_dev(const float *d_q, const float *d_k, const float *d_v, float *d_o, int n, int heads,
                          int hd, void *stream);
int fh3_hip_attention_qkv_dev(const float *d_qkv, int n, int heads, int hd, const float *d_qnorm_w,
                              const float *d_knorm_w, float eps, const float *d_cos, const float *d_sin, int rot_dim,
                              float *d_o, void *stream);

/* Video sparse attention on the device (fh3_vsa_attention, reference
 * src/core/fh3_vsa.c:186-507): q, k, v, gate (may be NULL), o are device
 * arrays [n][heads][head_dim]; c and seq are host structs (seq's counts and
 * video grid).  The qkv form reads q, k, v from the qkv projection output
 * d_qkv [n][3 * heads * head_dim] and first applies the per-head q/k rmsnorm
 * and rope3 (as fh3_hip_attention_qkv_dev; src/model/fh3_dit.c:390-409).
 * Same limits as fh3_vsa_attention.  The tile geometry of the last sequence
 * shape is kept on the device; a new shape synchronises the device once to
 * replace it.  Workspace (library-owned): the fp16 operands, pooled tiles,
 * heads * T^2 tile scores and the tile lists (T = number of tiles); calls that
 * overlap on different streams must not share it. */
int fh3_hip_vsa_attention_dev(const Fh3VsaCfg *c, const float *d_q, const float *d_k, const float *d_v,
                              const float *d_gate, float *d_o, const Fh3Seq *seq, int heads, int head_dim,
                              void *stream);
int fh3_hip_vsa_attention_qkv_dev(const Fh3VsaCfg *c, const float *d_qkv, const float *d_qnorm_w,
                                  const float *d_knorm_w, float eps, const float *d_cos, const float *d_sin,
                                  int rot_dim, const float *d_gate, float *d_o, const Fh3Seq *seq, int heads,
                                  int head_dim, void *stream);

/* Weight registration (the boundary's "host data -> device pointer" hook).
 * fh3_hip_register_weights uploads [host, host + bytes) once and keeps the
 * copy on the device; the host-pointer wrappers fh3_matmul / fh3_dequant then
 * find any weight lying inside a registered range and use the device copy in
 * place, copying only x in and y out (a registered range is typically a
 * packed layer or an mmapped GGUF tensor region).  *d_out (may be NULL) gets
 * the device address of `host`, usable directly as Fh3W.data with the _dev
 * entry points.  The host bytes must not change while registered:
 * registering the same range again refreshes the device copy.  Ranges may
 * not overlap.  fh3_hip_unregister_weights frees the copy (after the device
 * is idle); fh3_hip_registered_ptr returns the device address of
 * [host, host + bytes) or NULL.  Replaces the per-call weight upload of the
 * wrappers; the reference keeps weights in host memory
 * (src/io/fh3_trunk.c:413-431, src/io/fh3_pack.c:148-158). */
int fh3_hip_register_weights(const void *host, size_t bytes, const void **d_out);
int fh3_hip_unregister_weights(const void *host);
const void *fh3_hip_registered_ptr(const void *host, size_t bytes);

/* HIP graph capture of work enqueued on a stream (NULL = the compute
 * stream), for launch-bound loops such as small-M text-encoder layers:
 * begin, enqueue fh3_hip_* calls on that stream, end -> an executable graph
 * that fh3_hip_graph_launch replays on any stream.  A captured call must not
 * need to grow the library workspace (or, for VSA, see a new sequence
 * shape): it then returns FH3_E_INVALID without enqueuing anything, and the
 * same call run once eagerly first makes its capture succeed.  A workspace
 * that a later eager call grows gets a new buffer; the old one stays
 * allocated while any graph made by fh3_hip_graph_end exists (graphs keep
 * their buffer addresses), and is freed when fh3_hip_graph_destroy destroys
 * the last of them.  A capture begun by the caller's own
 * hipStreamBeginCapture is seen when a call under it reaches its workspace;
 * from then on replaced buffers stay allocated until fh3_hip_shutdown, since
 * the library cannot see when such a graph is destroyed.  Graphs therefore
 * stay valid across workspace growth; replays of graphs that share a
 * workspace buffer must not overlap. */
int fh3_hip_graph_begin(void *stream);
int fh3_hip_graph_end(void *stream, void **graph_exec);
int fh3_hip_graph_launch(void *graph_exec, void *stream);
int fh3_hip_graph_destroy(void *graph_exec);

/* Bytes of library workspace a product allocates (0 when none): the prepared
 * activations of fh3_hip_matmul_dev / fh3_hip_matmul_epi_dev (prepared = 0)
 * plus the partial sums of the split-K kernels; with prepared = 1 the same for
 * fh3_hip_matmul_prepared_dev / _prepared_epi_dev.  epi as below.  Under the
 * current fh3_hip_set_path setting. */
size_t fh3_hip_matmul_workspace_bytes(const Fh3W *w, int n_tok, int epi, int prepared);

/* The no-allocation product, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and bit-identical results as
 * fh3_hip_matmul_dev with Q4_K weights and no epilogue, but its workspace is
 * a fixed array of FH3_HIP_NOALLOC_SCRATCH_BYTES in device memory that the
 * library binds in fh3_hip_init (each device holds its own copy until the
 * process ends).  The call allocates and frees nothing; it returns
 * FH3_E_INVALID when the library is not initialised, for another weight
 * type, or when the shape needs more workspace than the array holds (the
 * message gives the size), or for rows of more than 32768 values.  The need
 * is the prepared activations (about 2 * round_up(n_tok, 256) * in bytes,
 * 16.3 MB at 64 tokens and in = 32768) plus the K-split partial sums
 * (4 * S * n_tok * out bytes, S up to in / 2048 from 33 tokens); see
 * fh3_hip_matmul_workspace_bytes.  Every n_tok <= 64 fits the real DiT and
 * text-encoder shapes (out <= 28672 at in <= 14336, out = 5120 at
 * in = 25600); at in = 32768 and 64 tokens, out up to 12208 fits.  The array
 * keeps the last call's contents; every call on
 * a device shares it, so calls that overlap on one device (different streams,
 * threads, or graph replays) race and must be serialised by the caller. */
#define FH3_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)
int fh3_hip_matmul_noalloc_dev(const Fh3W *w, const float *d_x, float *d_y, int n_tok,
                               const float *d_bias_or_null, void *stream);

/* Kernel selection for fh3_hip_matmul_dev: FH3_HIP_PATH_AUTO picks
 *   - FH3_HIP_PATH_GEMV8 for n_tok <= 4 when its window fits (in <= 20480 for
 *     one or two tokens, in <= 12288 for three or four): activations
 *     quantised to int16 (two int8
 *     planes, one power-of-two scale per token and wavefront window) inside
 *     the kernel, integer MFMA on the raw 4-bit weights, no preparation launch
 *     and no workspace;
 *   - FH3_HIP_PATH_SWEEP for the other n_tok <= 16 when 512 <= in <= 32768,
 *     and n_tok <= 64 when 5120 <= in <= 32768 (forced on shorter rows: in
 *     groups of 32 tokens, each swept by its own workgroups, up to 4096):
 *     fp16 activations with their group sums (prepared), exact fp16 sc*q
 *     weights, persistent workgroups that keep each wavefront's activations in
 *     registers while they sweep the weight rows; rows of more than 5120
 *     weights are split into K slices whose partial sums (library workspace,
 *     see fh3_hip_matmul_workspace_bytes) are added in slice order;
 *   - FH3_HIP_PATH_MIDM only when forced (n_tok <= 64): K split into windows
 *     over 128-row workgroups that share staged activations, partial sums in
 *     a library workspace, then an ordered sum;
 *   - FH3_HIP_PATH_SKINNY (fp16 activations, exact fp16 sc*q weights) for
 *     the other n_tok <= fh3_hip_skinny_max();
 *   - FH3_HIP_PATH_GEMM above.
 * Setting a path forces it where it can take the shape (tests); prepare and
 * product of the two-stage API must run under the same setting. */
#define FH3_HIP_PATH_AUTO   0
#define FH3_HIP_PATH_SKINNY 1
#define FH3_HIP_PATH_GEMM   2
#define FH3_HIP_PATH_GEMV8  3
#define FH3_HIP_PATH_MIDM   4
#define FH3_HIP_PATH_SWEEP  5
int fh3_hip_set_path(int path);
int fh3_hip_skinny_max(void);
/* The kernel family fh3_hip_matmul_dev would use for n_tok tokens of in
 * inputs under the current setting. */
int fh3_hip_matmul_path(int n_tok, int64_t in);

#ifdef __cplusplus
}
#endif

#endif /* FH3_HIP_H */
