// fh3_kernels.hip -- gfx950 kernels of the fh3 Q4_K linear layer.
//
// Q4_K super-block (144 B per 256 weights, reference src/core/fh3_quant.c:154-196):
//   bytes 0-1 d (fp16), 2-3 dmin (fp16), 4-15 packed 6-bit scales/mins,
//   16-143 four 32-byte chunks; chunk c holds group 2c in its low nibbles and
//   group 2c+1 in its high nibbles.  w = (d*sc_g)*q - dmin*m_g.
//
// Kernels
//   k_dequant_q4k_f32   bit-exact fp32 dequantisation (parity / debug path)
//   k_xprep             fp32 activations -> fp16 MFMA fragments, per-row 2^e scale
//   k_skinny<TB,NW>     small n_tok: one wavefront per 16 weight rows per K slice,
//                       v_mfma_f32_16x16x32_f16, K split over NW waves, LDS reduce
//   k_gemm              large n_tok: 256x128 output tile, Q4_K dequantised into LDS
//                       as fp16, v_mfma_f32_32x32x16_f16, fp32 accumulation
//
// Fragment layout shared by k_xprep, k_skinny and k_gemm ("X16"): activations of
// 32 tokens x 16 k form one 1 KiB fragment; lane l (0..63) holds 8 consecutive
// fp16 of token (l % 32) at k offset 8*(l / 32).  Fragment (T, kf) lives at
// X16[(T * (K/16) + kf) * 64 + l], so a wavefront loads one fragment as 1 KiB of
// contiguous memory.  MFMA A and B operands use the same lane -> k mapping, so
// the k order inside one MFMA never needs to match the hardware's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fh3_kernels.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

// ---------------------------------------------------------------------------
// Scalar helpers
// ---------------------------------------------------------------------------

// Exact fp16 -> fp32 on the bit fields (independent of the fp16 denormal mode);
// NaNs come out quiet, as with x86 F16C (reference src/core/fh3_quant.h:20-41).
__device__ __forceinline__ float f16_to_f32_exact(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else if (exp != 0u) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0u) {
        bits = sign;
    } else {
        // subnormal half: man * 2^-24 = 2^(p-24) * 1.f with p the top set bit
        const uint32_t p = 31u - (uint32_t)__builtin_clz(man);
        bits = sign | ((p + 103u) << 23) | ((man << (23u - p)) & 0x7FFFFFu);
    }
    return __builtin_bit_cast(float, bits);
}

// 6-bit scale and min of group g from the 12 packed bytes held in words
// s0 = bytes 0-3, s1 = bytes 4-7, s2 = bytes 8-11 (little endian).
// Reference src/core/fh3_quant.c:168-177.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                              uint32_t &sc, uint32_t &mn) {
    if (g < 4) {
        const int sh = 8 * g;
        sc = (s0 >> sh) & 63u;
        mn = (s1 >> sh) & 63u;
    } else {
        const int sh = 8 * (g - 4);
        sc = ((s2 >> sh) & 15u) | (((s0 >> (sh + 6)) & 3u) << 4);
        mn = ((s2 >> (sh + 4)) & 15u) | (((s1 >> (sh + 6)) & 3u) << 4);
    }
}

// Group scale D = d*sc and offset Mn = dmin*m, each rounded once in fp32 exactly
// as the reference forms dl[] and ml[].
__device__ __forceinline__ void q4k_group(const u32x4 hdr, int g, float &D, float &Mn) {
    uint32_t sc, mn;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, g, sc, mn);
    const float d = f16_to_f32_exact(hdr.x & 0xFFFFu);
    const float dmin = f16_to_f32_exact(hdr.x >> 16);
    D = __fmul_rn(d, (float)sc);
    Mn = __fmul_rn(dmin, (float)mn);
}

// Eight weights of one group from 8 bytes (u0 = bytes 0-3, u1 = bytes 4-7),
// low nibbles (hi == false) or high nibbles, as fp16 for the MFMA B/A operand:
// fma(D, q, -Mn) in fp32 rounded once to fp16 (v_fma_mix).
__device__ __forceinline__ half8 q4k_deq8_f16(uint32_t u0, uint32_t u1, bool hi, float D, float Mn) {
    const uint32_t a = (hi ? (u0 >> 4) : u0) & 0x0F0F0F0Fu;
    const uint32_t b = (hi ? (u1 >> 4) : u1) & 0x0F0F0F0Fu;
    half8 r;
    r[0] = (_Float16)__builtin_fmaf(D, (float)(a & 0xFFu), -Mn);
    r[1] = (_Float16)__builtin_fmaf(D, (float)((a >> 8) & 0xFFu), -Mn);
    r[2] = (_Float16)__builtin_fmaf(D, (float)((a >> 16) & 0xFFu), -Mn);
    r[3] = (_Float16)__builtin_fmaf(D, (float)(a >> 24), -Mn);
    r[4] = (_Float16)__builtin_fmaf(D, (float)(b & 0xFFu), -Mn);
    r[5] = (_Float16)__builtin_fmaf(D, (float)((b >> 8) & 0xFFu), -Mn);
    r[6] = (_Float16)__builtin_fmaf(D, (float)((b >> 16) & 0xFFu), -Mn);
    r[7] = (_Float16)__builtin_fmaf(D, (float)(b >> 24), -Mn);
    return r;
}

__device__ __forceinline__ u32x4 ld16(const uint8_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}

// ---------------------------------------------------------------------------
// Bit-exact fp32 dequantisation.  One thread per (row, super-block, 16-byte
// quarter of the nibbles): 32 outputs, two groups.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_dequant_q4k_f32(const uint8_t *__restrict__ src,
                                                         int64_t row_bytes, int64_t n, int64_t rows,
                                                         float *__restrict__ dst) {
    const int64_t nsb = n / 256;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * nsb * 8) return;
    const int64_t row = gid / (nsb * 8);
    const int64_t rem = gid - row * nsb * 8;
    const int64_t sb = rem >> 3;
    const int piece = (int)(rem & 7);
    const int c = piece >> 1, h = piece & 1;
    const uint8_t *blk = src + row * row_bytes + sb * 144;
    const u32x4 hdr = ld16(blk);
    float Dlo, Mlo, Dhi, Mhi;
    q4k_group(hdr, 2 * c, Dlo, Mlo);
    q4k_group(hdr, 2 * c + 1, Dhi, Mhi);
    const u32x4 qv = ld16(blk + 16 + 32 * c + 16 * h);
    float *out = dst + row * n + sb * 256;
    float lo[16], hi[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t byte = (qv[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        lo[j] = __fsub_rn(__fmul_rn(Dlo, (float)(byte & 15u)), Mlo);
        hi[j] = __fsub_rn(__fmul_rn(Dhi, (float)(byte >> 4)), Mhi);
    }
    f32x4 *olo = reinterpret_cast<f32x4 *>(out + (2 * c) * 32 + 16 * h);
    f32x4 *ohi = reinterpret_cast<f32x4 *>(out + (2 * c + 1) * 32 + 16 * h);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        olo[j] = f32x4{lo[4 * j], lo[4 * j + 1], lo[4 * j + 2], lo[4 * j + 3]};
        ohi[j] = f32x4{hi[4 * j], hi[4 * j + 1], hi[4 * j + 2], hi[4 * j + 3]};
    }
}

// ---------------------------------------------------------------------------
// Activation preparation.  One workgroup per 32-token block T.  Row t gets the
// scale 2^e with e = 15 - E, where max|x_t| = f * 2^E (f in [0.5, 1)), so the
// largest magnitude lands in [2^14, 2^15): fp16 never overflows and small rows
// keep full fp16 precision.  xs_inv[t] = 2^-e undoes it in the epilogue.
// Rows M..Mpad-1 are written as zeros.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_xprep(const float *__restrict__ X, int M, int K,
                                               half8 *__restrict__ X16, float *__restrict__ xs_inv) {
    __shared__ float s_scale[32];
    const int T = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int rr = 0; rr < 8; rr++) {
        const int r = wave * 8 + rr;
        const int t = T * 32 + r;
        float mx = 0.f;
        if (t < M) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(X + (size_t)t * K);
            for (int k4 = lane; k4 < K / 4; k4 += 64) {
                const f32x4 v = xr[k4];
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if (lane == 0) {
            int e = 0;
            if (mx > 0.f && mx <= 3.4028234663852886e38f) {
                int E;
                (void)frexpf(mx, &E);
                e = 15 - E;
                e = e > 126 ? 126 : (e < -126 ? -126 : e);
            }
            s_scale[r] = ldexpf(1.0f, e);
            xs_inv[t] = ldexpf(1.0f, -e);
        }
    }
    __syncthreads();
    const int kf_n = K / 16;
    const int tl = lane & 31;
    const int t = T * 32 + tl;
    const float s = s_scale[tl];
    const int koff = 8 * (lane >> 5);
    for (int kf = wave; kf < kf_n; kf += 4) {
        half8 h = {};
        if (t < M) {
            const f32x4 *p = reinterpret_cast<const f32x4 *>(X + (size_t)t * K + kf * 16 + koff);
            const f32x4 a = p[0], b = p[1];
            h[0] = (_Float16)(a.x * s); h[1] = (_Float16)(a.y * s);
            h[2] = (_Float16)(a.z * s); h[3] = (_Float16)(a.w * s);
            h[4] = (_Float16)(b.x * s); h[5] = (_Float16)(b.y * s);
            h[6] = (_Float16)(b.z * s); h[7] = (_Float16)(b.w * s);
        }
        X16[((size_t)T * kf_n + kf) * 64 + lane] = h;
    }
}

// ---------------------------------------------------------------------------
// Small-M kernel.  Workgroup = NW wavefronts over 16 consecutive weight rows
// o0..o0+15; wavefront w takes super-blocks sb = w, w+NW, ...
// MFMA 16x16x32: B lane l = (row j = l%16, chunk q = l/16) loads the 32 bytes of
// chunk q (both of its groups 2q and 2q+1) plus the 16-byte header, i.e. each
// super-block of a row is read once, 144 B by 4 lanes.  MFMA m (0..7) takes from
// lane (j, q) the 8 weights of group 2q + m/4 at offsets 8*(m%4)..+7; the A
// lane (token i, q) loads the activations of the same k, one 16-byte piece of
// an X16 fragment.  Partial sums of the NW waves are added in wave order
// through LDS (deterministic).
// ---------------------------------------------------------------------------
template <int TB, int NW>
__global__ __launch_bounds__(NW * 64) void k_skinny(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                    int N, int K, const half8 *__restrict__ X16,
                                                    const float *__restrict__ xs_inv,
                                                    const float *__restrict__ bias,
                                                    float *__restrict__ Y, int M) {
    __shared__ f32x4 red[NW][TB][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int o0 = blockIdx.x * 16;
    int orow = o0 + j;
    orow = orow < N ? orow : N - 1;
    const uint8_t *wrow = W + (size_t)orow * row_bytes;
    const int nsb = K / 256;
    const int kf_n = K / 16;

    f32x4 acc[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) acc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // A-operand base per token block: token i = tb*16 + j
    const half8 *xb[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) {
        const int t = tb * 16 + j;
        xb[tb] = X16 + (size_t)(t >> 5) * kf_n * 64 + (t & 31);
    }

    int sb = wave;
    u32x4 h0 = {}, c0a = {}, c0b = {}, h1 = {}, c1a = {}, c1b = {};
    if (sb < nsb) {
        const uint8_t *blk = wrow + (size_t)sb * 144;
        h0 = ld16(blk); c0a = ld16(blk + 16 + 32 * q); c0b = ld16(blk + 32 + 32 * q);
    }
    if (sb + NW < nsb) {
        const uint8_t *blk = wrow + (size_t)(sb + NW) * 144;
        h1 = ld16(blk); c1a = ld16(blk + 16 + 32 * q); c1b = ld16(blk + 32 + 32 * q);
    }
    for (; sb < nsb; sb += NW) {
        float Dlo, Mlo, Dhi, Mhi;
        q4k_group(h0, 2 * q, Dlo, Mlo);
        q4k_group(h0, 2 * q + 1, Dhi, Mhi);
        const u32x4 ca = c0a, cb = c0b;
        // rotate the two-deep prefetch
        h0 = h1; c0a = c1a; c0b = c1b;
        if (sb + 2 * NW < nsb) {
            const uint8_t *blk = wrow + (size_t)(sb + 2 * NW) * 144;
            h1 = ld16(blk); c1a = ld16(blk + 16 + 32 * q); c1b = ld16(blk + 32 + 32 * q);
        }
        const int kf_sb = sb * 16 + 4 * q;  // fragment of group 2q, offset 0
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int part = m & 3;
            const bool hi = m >= 4;
            const u32x4 cv = part < 2 ? ca : cb;
            const uint32_t u0 = (part & 1) ? cv.z : cv.x;
            const uint32_t u1 = (part & 1) ? cv.w : cv.y;
            const half8 b = q4k_deq8_f16(u0, u1, hi, hi ? Dhi : Dlo, hi ? Mhi : Mlo);
            // k = sb*256 + (2q + hi)*32 + 8*part -> fragment kf_sb + 2*hi + part/2,
            // half (part & 1) of it
            const int kf = kf_sb + (hi ? 2 : 0) + (part >> 1);
            const int lsel = (part & 1) * 32;
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {
                const half8 a = xb[tb][(size_t)kf * 64 + lsel];
                acc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[tb], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++) red[wave][tb][lane] = acc[tb];
    __syncthreads();
    // output D of 16x16: lane l holds column (weight row) l%16, rows (tokens)
    // 4*(l/16) + v
    if (threadIdx.x < TB * 64) {
        const int tb = threadIdx.x >> 6, l = threadIdx.x & 63;
        f32x4 s = red[0][tb][l];
#pragma unroll
        for (int w = 1; w < NW; w++) s += red[w][tb][l];
        const int o = o0 + (l & 15);
        if (o < N) {
            const float bo = bias ? bias[o] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = tb * 16 + 4 * (l >> 4) + v;
                if (t < M) Y[(size_t)t * N + o] = s[v] * xs_inv[t] + bo;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-M kernel.  Output tile 256 tokens x 128 weight rows, 4 wavefronts, each
// owning 64 tokens x all 128 rows (2 x 4 tiles of 32x32, 128 fp32 accumulators
// per lane).  Per K step of 64 (one Q4_K chunk: groups 2c and 2c+1):
//   - thread (r = tid%128, h = tid/128) loads 16 bytes of row r's chunk and
//     writes 32 dequantised fp16 weights into the LDS B-fragments;
//   - each wavefront loads its X16 fragments straight from global memory
//     (1 KiB contiguous per load), one step ahead;
//   - LDS is double buffered, one barrier per step.
// Workgroup ids are remapped so that the 8 XCDs each run a contiguous run of
// tiles in token-major order: concurrent tiles on one XCD share the same 256
// activation rows in that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int GEMM_BM = 256;
constexpr int GEMM_BN = 128;

__global__ __launch_bounds__(256, 2) void k_gemm(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                 int N, int K, const half8 *__restrict__ X16,
                                                 const float *__restrict__ xs_inv,
                                                 const float *__restrict__ bias,
                                                 float *__restrict__ Y, int M, int m_tiles,
                                                 int n_tiles) {
    __shared__ half8 lds[2][16][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const int total = m_tiles * n_tiles;
    const int id = blockIdx.x;
    const int per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int mt = L / n_tiles, nt = L - mt * n_tiles;
    const int m0 = mt * GEMM_BM, n0 = nt * GEMM_BN;

    // weight-loader role
    const int r = tid & 127, h = tid >> 7;
    int orow = n0 + r;
    orow = orow < N ? orow : N - 1;
    const uint8_t *wrow = W + (size_t)orow * row_bytes;
    const int wf = (r >> 5) * 4;   // first LDS fragment of this row's 32-row block
    const int wl = r & 31;

    // activation fragments of this wavefront: token blocks T0, T0+1
    const int kf_n = K / 16;
    const half8 *xa0 = X16 + ((size_t)(m0 / 32 + 2 * wave) * kf_n) * 64 + lane;
    const half8 *xa1 = xa0 + (size_t)kf_n * 64;

    const int S = K / 64;
    f32x16 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    u32x4 hv = ld16(wrow);
    u32x4 qv = ld16(wrow + 16 + 16 * h);
    half8 xf[2][4];
#pragma unroll
    for (int k = 0; k < 4; k++) { xf[0][k] = xa0[k * 64]; xf[1][k] = xa1[k * 64]; }

    for (int s = 0; s < S; s++) {
        const int buf = s & 1;
        const int c = s & 3;
        {
            float Dlo, Mlo, Dhi, Mhi;
            q4k_group(hv, 2 * c, Dlo, Mlo);
            q4k_group(hv, 2 * c + 1, Dhi, Mhi);
            lds[buf][wf + h][wl] = q4k_deq8_f16(qv.x, qv.y, false, Dlo, Mlo);
            lds[buf][wf + h][wl + 32] = q4k_deq8_f16(qv.z, qv.w, false, Dlo, Mlo);
            lds[buf][wf + 2 + h][wl] = q4k_deq8_f16(qv.x, qv.y, true, Dhi, Mhi);
            lds[buf][wf + 2 + h][wl + 32] = q4k_deq8_f16(qv.z, qv.w, true, Dhi, Mhi);
        }
        half8 xn[2][4];
        if (s + 1 < S) {
            const int s1 = s + 1;
            const uint8_t *blk = wrow + (size_t)(s1 >> 2) * 144;
            if ((s1 & 3) == 0) hv = ld16(blk);
            qv = ld16(blk + 16 + 32 * (s1 & 3) + 16 * h);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                xn[0][k] = xa0[(size_t)(s1 * 4 + k) * 64];
                xn[1][k] = xa1[(size_t)(s1 * 4 + k) * 64];
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            half8 bfr[4];
#pragma unroll
            for (int ob = 0; ob < 4; ob++) bfr[ob] = lds[buf][ob * 4 + k][lane];
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                acc[0][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xf[0][k], bfr[ob], acc[0][ob], 0, 0, 0);
                acc[1][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xf[1][k], bfr[ob], acc[1][ob], 0, 0, 0);
            }
        }
        if (s + 1 < S) {
#pragma unroll
            for (int k = 0; k < 4; k++) { xf[0][k] = xn[0][k]; xf[1][k] = xn[1][k]; }
        }
    }

    // epilogue: 32x32 output D, lane l holds column l%32 (weight row) and rows
    // 8*(v/4) + 4*(l/32) + v%4 (tokens)
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
        const int tbase = m0 + 64 * wave + 32 * tb + 4 * (lane >> 5);
#pragma unroll
        for (int ob = 0; ob < 4; ob++) {
            const int o = n0 + 32 * ob + (lane & 31);
            if (o >= N) continue;
            const float bo = bias ? bias[o] : 0.f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int t = tbase + 8 * (v >> 2) + (v & 3);
                if (t < M) Y[(size_t)t * N + o] = acc[tb][ob][v] * xs_inv[t] + bo;
            }
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers (host side, called by fh3_hip.cpp)
// ---------------------------------------------------------------------------
extern "C" hipError_t fh3k_dequant_q4k_f32(const void *src, int64_t row_bytes, int64_t n, int64_t rows,
                                           float *dst, hipStream_t st) {
    const int64_t threads = rows * (n / 256) * 8;
    if (threads <= 0) return hipSuccess;
    const int64_t blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(k_dequant_q4k_f32, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint8_t *)src, row_bytes, n, rows, dst);
    return hipGetLastError();
}

extern "C" hipError_t fh3k_xprep(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv,
                                 hipStream_t st) {
    hipLaunchKernelGGL(k_xprep, dim3((unsigned)(Mpad / 32)), dim3(256), 0, st, x, M, K, (half8 *)x16,
                       xs_inv);
    return hipGetLastError();
}

template <int TB>
static hipError_t launch_skinny(const void *W, int64_t rb, int N, int K, const void *x16,
                                const float *xs_inv, const float *bias, float *y, int M, hipStream_t st) {
    const unsigned blocks = (unsigned)((N + 15) / 16);
    hipLaunchKernelGGL((k_skinny<TB, 4>), dim3(blocks), dim3(256), 0, st, (const uint8_t *)W, rb, N, K,
                       (const half8 *)x16, xs_inv, bias, y, M);
    return hipGetLastError();
}

extern "C" hipError_t fh3k_skinny(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                  const float *xs_inv, const float *bias, float *y, int M, hipStream_t st) {
    const int tb = (M + 15) / 16;
    switch (tb) {
        case 1: return launch_skinny<1>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, st);
        case 2: return launch_skinny<2>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, st);
        case 3: return launch_skinny<3>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, st);
        case 4: return launch_skinny<4>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" int fh3k_skinny_max_tokens(void) { return 64; }

extern "C" hipError_t fh3k_gemm(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                const float *xs_inv, const float *bias, float *y, int M, hipStream_t st) {
    const int m_tiles = (M + GEMM_BM - 1) / GEMM_BM;
    const int n_tiles = (N + GEMM_BN - 1) / GEMM_BN;
    hipLaunchKernelGGL(k_gemm, dim3((unsigned)(m_tiles * n_tiles)), dim3(256), 0, st,
                       (const uint8_t *)W, row_bytes, N, K, (const half8 *)x16, xs_inv, bias, y, M,
                       m_tiles, n_tiles);
    return hipGetLastError();
}

extern "C" int fh3k_gemm_row_pad(void) { return GEMM_BM; }
