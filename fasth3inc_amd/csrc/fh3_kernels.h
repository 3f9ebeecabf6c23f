// fh3_kernels.h -- launchers of the gfx950 kernels in fh3_kernels.hip.
// Internal to libfh3hip.so; the public C-ABI is include/fh3/fh3_hip.h.
#ifndef FH3_KERNELS_H
#define FH3_KERNELS_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Bit-exact fp32 dequantisation of `rows` Q4_K rows (n % 256 == 0).
hipError_t fh3k_dequant_q4k_f32(const void *src, int64_t row_bytes, int64_t n, int64_t rows,
                                float *dst, hipStream_t st);

// x[M][K] fp32 -> x16 fragments (Mpad x K fp16, Mpad % 32 == 0, rows >= M zero)
// and xs_inv[Mpad] (per-row inverse power-of-two scale).
hipError_t fh3k_xprep(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv,
                      hipStream_t st);

// y = x * W^T (+bias) from prepared fragments, n_tok <= fh3k_skinny_max_tokens();
// x16 must hold round_up(M, 32) rows.
hipError_t fh3k_skinny(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                       const float *xs_inv, const float *bias, float *y, int M, hipStream_t st);
int fh3k_skinny_max_tokens(void);

// Largest in-dimension (K) the activation preparation handles.
int fh3k_max_in(void);

// y = x * W^T (+bias) from prepared fragments; x16 must hold
// round_up(M, fh3k_gemm_row_pad()) rows.
hipError_t fh3k_gemm(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                     const float *xs_inv, const float *bias, float *y, int M, hipStream_t st);
int fh3k_gemm_row_pad(void);

#ifdef __cplusplus
}
#endif

#endif
