// fh3_kernels.h -- launchers of the gfx950 kernels in fh3_kernels.hip.
// Internal to libfh3hip.so; the public C-ABI is include/fh3/fh3_hip.h.
#ifndef FH3_KERNELS_H
#define FH3_KERNELS_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Weight type ids (the values of the reference's FH3_QUANT_* enum).
enum {
    FH3K_F32 = 0, FH3K_F16 = 1, FH3K_Q8_0 = 8, FH3K_Q2_K = 10, FH3K_Q3_K = 11,
    FH3K_Q4_K = 12, FH3K_Q5_K = 13, FH3K_Q6_K = 14, FH3K_BF16 = 30
};

// Elements per block of a decodable type (1 for F32/F16/BF16), 0 otherwise.
int fh3k_dequant_block_len(int type);

// Bit-exact fp32 dequantisation of `rows` rows of n elements (n a multiple of
// the block length), source rows row_bytes apart, output dense [rows][n].
// src 2-byte aligned with row_bytes even (16-byte for Q4_K/Q5_K), dst
// 16-byte aligned.
hipError_t fh3k_dequant_f32(int type, const void *src, int64_t row_bytes, int64_t n, int64_t rows,
                            float *dst, hipStream_t st);

// x[M][K] fp32 -> x16 fragments (Mpad x K fp16, Mpad % 32 == 0, rows >= M zero)
// and xs_inv[Mpad] (per-row inverse power-of-two scale); with xsum set (K <=
// 32768), also xsum[M][K/32]: the sum of each 32-value group of the row's
// fp16 values (the offsets of fh3k_sweep_epi).
hipError_t fh3k_xprep(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv, float *xsum,
                      hipStream_t st);

// y = x * W^T (+bias) from prepared fragments, n_tok <= fh3k_skinny_max_tokens();
// x16 must hold round_up(M, 32) rows.
hipError_t fh3k_skinny(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                       const float *xs_inv, const float *bias, float *y, int M, hipStream_t st);
int fh3k_skinny_max_tokens(void);

// y = x * W^T (+bias) for n_tok = M <= fh3k_gemv8_max_tokens() straight from
// fp32 x[M][K] (16-byte aligned): activations quantised to int16 inside the
// kernel, integer MFMA on the raw weights.  fh3k_gemv8_fits(K, M) says whether
// the kernel takes this shape (its LDS grows with K * M).
hipError_t fh3k_gemv8(const void *W, int64_t row_bytes, int N, int K, const float *x, const float *bias,
                      float *y, int M, hipStream_t st);
int fh3k_gemv8_max_tokens(void);
int fh3k_gemv8_fits(int K, int M);

// Weights of any decodable type as fp16 rows dst[N][Kp] (the exact fp32 value
// rounded once; F16 copied), K a multiple of the type's block length, Kp >= K
// a multiple of 256, columns K..Kp-1 zero; then the fp16-row products, same
// activation fragments and launch rules as fh3k_skinny / fh3k_gemm (with Kp
// as their K).
hipError_t fh3k_weights_f16(int type, const void *src, int64_t row_bytes, int K, int Kp, int N, void *dst,
                            hipStream_t st);
// x[M][K] fp32 with any K and 4-byte alignment -> x16 fragments of
// Kp = round_up(K, 256) columns (zeros at k >= K) and xs_inv[Mpad], with
// fh3k_xprep's scale rule and rounding (the same bits where both apply).
hipError_t fh3k_xprep_any(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv, hipStream_t st);
hipError_t fh3k_skinny16(const void *W16, int N, int K, const void *x16, const float *xs_inv, const float *bias,
                         float *y, int M, hipStream_t st);
hipError_t fh3k_gemm16(const void *W16, int N, int K, const void *x16, const float *xs_inv, const float *bias,
                       float *y, int M, hipStream_t st);
// Q5_K / Q6_K weights (type FH3K_Q5_K / FH3K_Q6_K) read in place by the
// small-M kernel, M <= fh3k_skinny_max_tokens(), same fragments as fh3k_skinny;
// fh3k_skinny_q_takes(type) says whether a type has this kernel.  Rows that
// give fewer row blocks than the chip takes are split into K windows whose raw
// sums go to part (fh3k_skinny_q_part_bytes(N, K, M) bytes; 0 = no split).
hipError_t fh3k_skinny_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                         const float *xs_inv, const float *bias, float *y, int M, float *part, hipStream_t st);
size_t fh3k_skinny_q_part_bytes(int N, int K, int M);
int fh3k_skinny_q_takes(int type);

// Product epilogues (EPI_* of fh3_kernels.hip; FH3_EPI_* of fh3_hip.h): 0 plain
// store, 1 y[t][o] += aux[t][o] * product (gate residual), 2 SwiGLU (weight of
// 2F rows [val | gate], y of width F; N % 128 == 0 for the GEMM, % 16 below).
hipError_t fh3k_skinny_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16, const float *xs_inv,
                           const float *bias, float *y, int M, int epi, const float *aux, hipStream_t st);
hipError_t fh3k_gemv8_epi(const void *W, int64_t row_bytes, int N, int K, const float *x, const float *bias,
                          float *y, int M, int epi, const float *aux, hipStream_t st);
// Up to fh3k_sweep_max_tokens() tokens from prepared fragments and their group
// sums (fh3k_xprep with xsum), when fh3k_sweep_fits(K, M); persistent, the
// activations held in registers.
// K beyond 32 super-blocks is split into slices whose partial sums go to part
// (fh3k_sweep_part_bytes(N, K, M) bytes; 0 = no split, part may be NULL).
hipError_t fh3k_sweep_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16, const float *xs_inv,
                          const float *xsum, const float *bias, float *y, int M, int epi, const float *aux,
                          float *part, hipStream_t st);
size_t fh3k_sweep_part_bytes(int N, int K, int M);
int fh3k_sweep_fits(int K, int M);
int fh3k_sweep_max_tokens(void);
// Q6_K weights read in place by the sweep (fh3k_sweep_q_takes), no epilogue:
// same fragments and launch rules as fh3k_sweep_epi without the group sums;
// partial sums of its K slices in part (fh3k_sweep_q_part_bytes bytes).
hipError_t fh3k_sweep_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                        const float *xs_inv, const float *bias, float *y, int M, float *part, hipStream_t st);
size_t fh3k_sweep_q_part_bytes(int type, int N, int K, int M);
int fh3k_sweep_q_takes(int type);
// Large M.  When the 256 x 128 tiles alone would not fill the chip, K is split
// into windows whose raw sums go to part (fh3k_gemm_part_bytes bytes; 0 = no
// split) and are added in window order with the epilogue; x16 must hold
// round_up(M, fh3k_gemm_row_pad()) rows.
hipError_t fh3k_gemm_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16, const float *xs_inv,
                         const float *bias, float *y, int M, int epi, const float *aux, float *part,
                         hipStream_t st);
size_t fh3k_gemm_part_bytes(int N, int K, int M, int epi);
// Q5_K / Q6_K weights read in place by k_gemm (fh3k_gemm_q_takes), no
// epilogue: same fragments, tiles, K split and partial-sum bytes
// (fh3k_gemm_part_bytes with epi 0) as fh3k_gemm_epi.
hipError_t fh3k_gemm_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                       const float *xs_inv, const float *bias, float *y, int M, float *part, hipStream_t st);
int fh3k_gemm_q_takes(int type);
// Prepared rows k_gemm reads for M tokens (its tiles cover 128 or 256
// tokens; at most round_up(M, fh3k_gemm_row_pad())).
int fh3k_gemm_rows(int M);

// Middle M (1 <= M <= fh3k_midm_max_tokens()): K split into S windows, partial
// sums in part (fh3k_midm_part_bytes(N, K, M) bytes), then an ordered sum with
// the epilogue.  Same prepared fragments as fh3k_skinny (round_up(M, 32) rows).
hipError_t fh3k_midm_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16, const float *xs_inv,
                         const float *bias, float *y, int M, int epi, const float *aux, float *part,
                         hipStream_t st);
size_t fh3k_midm_part_bytes(int N, int K, int M);
int fh3k_midm_max_tokens(void);

// fh3k_xprep with the rows first normalised: rmsnorm with weight norm_w and
// eps, then (shift and scale both set, [M][K]) AdaLN modulate.
hipError_t fh3k_xprep_norm(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv, const float *norm_w,
                           float eps, const float *shift, const float *scale, float *xsum, hipStream_t st);
// The same normalisation into fp32 rows y[M][K] (y may alias x).
hipError_t fh3k_rownorm_f32(const float *x, int M, int K, float *y, const float *norm_w, float eps,
                            const float *shift, const float *scale, hipStream_t st);

// Attention (fh3_attn.hip).  q, k, v: fp32 rows [n][heads][hd] at token
// stride ld (16-byte aligned, ld % 4 == 0), e.g. read in place from a qkv
// projection output; o: [n][heads][hd] at token stride o_ld.  Optional
// per-head rmsnorm of q and k (weights [hd], eps) and rope3 on their first rot
// channels (cos/sin [n][rot]).  ws holds fh3k_attn_ws_bytes(n, heads, hd).
// hd must pass fh3k_attn_head_dim_ok.
int64_t fh3k_attn_pad(int n);
size_t fh3k_attn_ws_bytes(int n, int heads, int hd);
int fh3k_attn_head_dim_ok(int hd);
hipError_t fh3k_attention(const float *q, const float *k, const float *v, int64_t ld, int n, int heads, int hd,
                          const float *qn_w, const float *kn_w, float eps, const float *cosb, const float *sinb,
                          int rot, void *ws, float *o, int64_t o_ld, hipStream_t st);

// Video sparse attention.  q, k at token stride ld, v at ldv; optional per-head
// q/k rmsnorm and rope3 as fh3k_attention; gate and o [n][heads][hd] at stride
// o_ld.  Tile geometry from the host: inv[T] = 1/count, cnt[T], gather[
// round_up(64 T, 128)] (token of each slot, -1 empty); P prefix tiles, kv video
// tiles kept per video query tile (all = 1 keeps every tile), scale =
// 1/sqrt(hd).  T <= fh3k_vsa_max_tiles(); ws holds fh3k_vsa_ws_bytes(T, heads, hd).
int fh3k_vsa_max_tiles(void);
size_t fh3k_vsa_ws_bytes(int T, int heads, int hd);
hipError_t fh3k_vsa_attention(const float *q, const float *k, const float *v, int64_t ld, int64_t ldv,
                              const float *qn_w, const float *kn_w, float eps, const float *cosb, const float *sinb,
                              int rot, const float *gate, float *o, int64_t o_ld, int heads, int hd, const float *inv,
                              const int *gather, const int *cnt, int T, int P, int kv, int all, float scale, void *ws,
                              hipStream_t st);

// Largest in-dimension (K) the activation preparation handles.
int fh3k_max_in(void);

// Device address, on the current device, of the fixed scratch array of
// FH3_HIP_NOALLOC_SCRATCH_BYTES (fh3_hip.h) that the no-allocation entry point
// uses as its workspace.
hipError_t fh3k_scratch_bind(void **ptr);

int fh3k_gemm_row_pad(void);

#ifdef __cplusplus
}
#endif

#endif
