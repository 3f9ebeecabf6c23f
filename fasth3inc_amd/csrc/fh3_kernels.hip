// fh3_kernels.hip -- gfx950 kernels of the fh3 Q4_K linear layer.
//
// Q4_K super-block (144 B per 256 weights, reference src/core/fh3_quant.c:154-196):
//   bytes 0-1 d (fp16), 2-3 dmin (fp16), 4-15 packed 6-bit scales/mins,
//   16-143 four 32-byte chunks; chunk c holds group 2c in its low nibbles and
//   group 2c+1 in its high nibbles.  w = (d*sc_g)*q - dmin*m_g.
//
// Kernels
//   k_dequant_blocks<T> bit-exact fp32 dequantisation of Q8_0/Q2_K/Q3_K/Q4_K/Q5_K/Q6_K
//   k_dequant_half<BF>  bit-exact fp32 from F16 / BF16
//   k_xprep             fp32 activations -> fp16 MFMA fragments, per-row 2^e scale
//   k_skinny<QT,TB,C>   small n_tok: one wavefront per 16 weight rows per K slice of
//                       C super-blocks, exact weights (sc*q in fp16), two
//                       v_mfma_f32_16x16x32_f16 chains, LDS reduce over the slices;
//                       Q4_K, Q5_K or Q6_K blocks read in place
//   k_sweep<C,TB>       up to 64 tokens: k_skinny's exact weights, persistent
//                       workgroups with the activations held in registers, the
//                       offsets from precomputed group sums (f32 MFMA); long
//                       rows in K slices added by k_midm_sum
//   k_gemv8<MT,C>       up to 4 tokens: integer MFMA on the raw nibbles, fp32
//                       activations quantised in the kernel, persistent
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

#include <type_traits>

#include "fh3/fh3_hip.h"
#include "fh3_kernels.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Product-path group constants.  The hardware fp16 -> fp32 conversion is exact;
// D = d*sc and Mn = dmin*m are rounded once as in the reference, and the
// offset is folded with the magic bias of q4k_deq8_f16: C = -(Mn + 1024*D).
__device__ __forceinline__ void q4k_group_fast(const u32x4 hdr, int g, float &D, float &C) {
    uint32_t sc, mn;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, g, sc, mn);
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
    D = d * (float)sc;
    C = -(dmin * (float)mn + 1024.0f * D);
}

// Two nibble bytes (q0, q1 in bytes sel-picked from a) as the fp16 pair
// (1024 + q0, 1024 + q1): exponent byte 0x64 above each nibble (v_perm_b32).
__device__ __forceinline__ half2v q4k_magic_pair(uint32_t a, uint32_t sel) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, a, sel));
}

// Eight weights of one group from 8 bytes (u0 = bytes 0-3, u1 = bytes 4-7),
// low nibbles (hi == false) or high nibbles, as fp16 for an MFMA operand:
// fma(D, 1024 + q, C) = D*q - Mn evaluated in fp32 and rounded once to fp16
// (v_fma_mix).  C carries an fp32 rounding of at most 2^-24 * 1024 * D, far
// below the fp16 rounding of the result.
// fp16(D*p + C) for both halves of a pair p of fp16 values, with an fp32
// fused multiply-add: v_fma_mixlo/mixhi_f16 take the f16 operand and the f32
// operands as they are and write one half of the result each, so a pair costs
// two instructions instead of two conversions in, two FMAs and one pack.
__device__ __forceinline__ uint32_t fma_mix_pair(float D, uint32_t p, float C) {
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
        : "=&v"(r)
        : "v"(D), "v"(p), "v"(C));
    return r;
}

__device__ __forceinline__ half8 q4k_deq8_f16(uint32_t u0, uint32_t u1, bool hi, float D, float C) {
    const uint32_t a = (hi ? (u0 >> 4) : u0) & 0x0F0F0F0Fu;
    const uint32_t b = (hi ? (u1 >> 4) : u1) & 0x0F0F0F0Fu;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
    const u32x4 r = {fma_mix_pair(D, p0, C), fma_mix_pair(D, p1, C), fma_mix_pair(D, p2, C), fma_mix_pair(D, p3, C)};
    return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ u32x4 ld16(const uint8_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}

// ---------------------------------------------------------------------------
// Bit-exact fp32 dequantisation of every block format the reference decodes
// (src/core/fh3_quant.c:58-282).  One thread per 16 consecutive outputs of a
// block ("piece" G): 16 pieces per 256-weight super-block, 2 per Q8_0 block,
// so a wavefront writes 4 KiB of contiguous fp32 with 16-byte stores.  Every
// value is formed with the reference's roundings (__fmul_rn / __fsub_rn keep
// the compiler from contracting them into an fma): the group scale product
// first, then the weight product, then the offset subtraction.
//
// Block starts are only as aligned as the block size allows (Q5_K 16 B, Q2_K
// 4 B, Q3_K / Q6_K / Q8_0 2 B), so each format loads with its own guaranteed
// alignment and never wider.
// ---------------------------------------------------------------------------
template <int A>
__device__ __forceinline__ u32x4 ld16_al(const uint8_t *p) {
    if constexpr (A >= 16) {
        return ld16(p);
    } else if constexpr (A >= 4) {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
        return u32x4{q[0], q[1], q[2], q[3]};
    } else {
        const uint16_t *q = reinterpret_cast<const uint16_t *>(p);
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 16);
        return r;
    }
}

__device__ __forceinline__ uint32_t byte_of(const u32x4 v, int i) {
    return (v[i >> 2] >> (8 * (i & 3))) & 0xFFu;
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);
}

// Per-format geometry: block length, block bytes, pieces (threads) per block.
template <int T> struct Fmt;
template <> struct Fmt<FH3K_Q8_0> { static constexpr int BL = 32, BB = 34, P = 2; };
template <> struct Fmt<FH3K_Q2_K> { static constexpr int BL = 256, BB = 84, P = 16; };
template <> struct Fmt<FH3K_Q3_K> { static constexpr int BL = 256, BB = 110, P = 16; };
template <> struct Fmt<FH3K_Q4_K> { static constexpr int BL = 256, BB = 144, P = 16; };
template <> struct Fmt<FH3K_Q5_K> { static constexpr int BL = 256, BB = 176, P = 16; };
template <> struct Fmt<FH3K_Q6_K> { static constexpr int BL = 256, BB = 210, P = 16; };

// Outputs 16G..16G+15 of one block.
template <int T>
__device__ __forceinline__ void deq_piece(const uint8_t *blk, int G, float o[16]) {
    if constexpr (T == FH3K_Q8_0) {
        // fh3_quant.c:58-72: d (fp16) then 32 int8; w = q * d
        const float d = f16_to_f32_exact(ld_u16(blk));
        const u32x4 q = ld16_al<2>(blk + 2 + 16 * G);
#pragma unroll
        for (int l = 0; l < 16; l++) o[l] = __fmul_rn((float)(int8_t)byte_of(q, l), d);
    } else if constexpr (T == FH3K_Q2_K) {
        // fh3_quant.c:74-114: bytes 0-15 scale|min<<4 per 16-group, 16-79 two
        // 32-byte chunks of 2-bit values (chunk G/8, half G%2, bit pair (G/2)%4),
        // 80 d, 82 dmin; w = (d*sc)*q - dmin*m
        const float d = f16_to_f32_exact(ld_u16(blk + 80));
        const float dmin = f16_to_f32_exact(ld_u16(blk + 82));
        const uint32_t sm = blk[G];
        const float dl = __fmul_rn(d, (float)(sm & 15u)), ml = __fmul_rn(dmin, (float)(sm >> 4));
        const u32x4 q = ld16_al<4>(blk + 16 + (G >> 3) * 32 + (G & 1) * 16);
        const int sh = 2 * ((G >> 1) & 3);
#pragma unroll
        for (int l = 0; l < 16; l++)
            o[l] = __fsub_rn(__fmul_rn(dl, (float)((byte_of(q, l) >> sh) & 3u)), ml);
    } else if constexpr (T == FH3K_Q3_K) {
        // fh3_quant.c:116-152: 0-31 high-bit mask, 32-95 2-bit values, 96-107
        // signed 6-bit scales (low 4 bits from nibbles of bytes 96-103, top 2
        // from bytes 104-107, minus 32), 108 d.  q = low2 - 4 where the mask
        // bit G/2 is clear; w = (d*sc)*q
        const float d = f16_to_f32_exact(ld_u16(blk + 108));
        const uint32_t lo4 = G < 8 ? (blk[96 + G] & 15u) : (blk[88 + G] >> 4);
        const uint32_t hi2 = (blk[104 + (G & 3)] >> (2 * (G >> 2))) & 3u;
        const float dl = __fmul_rn(d, (float)((int)(lo4 | (hi2 << 4)) - 32));
        const u32x4 q = ld16_al<2>(blk + 32 + (G >> 3) * 32 + (G & 1) * 16);
        const u32x4 hm = ld16_al<2>(blk + (G & 1) * 16);
        const int shl = 2 * ((G & 7) >> 1), shh = G >> 1;
#pragma unroll
        for (int l = 0; l < 16; l++) {
            const int v = (int)((byte_of(q, l) >> shl) & 3u) - (((byte_of(hm, l) >> shh) & 1u) ? 0 : 4);
            o[l] = __fmul_rn(dl, (float)v);
        }
    } else if constexpr (T == FH3K_Q4_K || T == FH3K_Q5_K) {
        // fh3_quant.c:154-236: d, dmin, 12 bytes of packed 6-bit scales/mins;
        // group g = G/2 has its nibbles in chunk g/2 (low nibble for even g);
        // Q5_K adds bit g of byte 16 + l' (l' = index inside the group) as the
        // fifth bit.  w = (d*sc)*q - dmin*m
        const u32x4 hdr = ld16(blk);
        const int g = G >> 1, h = G & 1;
        float D, Mn;
        q4k_group(hdr, g, D, Mn);
        constexpr int QS = T == FH3K_Q4_K ? 16 : 48;
        const u32x4 q = ld16(blk + QS + (g >> 1) * 32 + 16 * h);
        u32x4 qh = u32x4{0u, 0u, 0u, 0u};
        if constexpr (T == FH3K_Q5_K) qh = ld16(blk + 16 + 16 * h);
        const int sh = 4 * (g & 1);
#pragma unroll
        for (int l = 0; l < 16; l++) {
            uint32_t v = (byte_of(q, l) >> sh) & 15u;
            if constexpr (T == FH3K_Q5_K) v |= ((byte_of(qh, l) >> g) & 1u) << 4;
            o[l] = __fsub_rn(__fmul_rn(D, (float)v), Mn);
        }
    } else {
        // fh3_quant.c:238-282 (Q6_K): 0-127 low nibbles, 128-191 high bit
        // pairs, 192-207 int8 scales, 208 d.  Half h = G/8, r = G%8: nibble
        // r/4 of byte h*64 + (r%4)*16 + l, pair r/2 of byte 128 + h*32 +
        // (r%2)*16 + l; q = (nibble | pair << 4) - 32; w = (d*sc)*q
        const float d = f16_to_f32_exact(ld_u16(blk + 208));
        const int h = G >> 3, r = G & 7;
        const u32x4 ql = ld16_al<2>(blk + h * 64 + (r & 3) * 16);
        const u32x4 qh = ld16_al<2>(blk + 128 + h * 32 + (r & 1) * 16);
        const float dl = __fmul_rn(d, (float)(int8_t)blk[192 + G]);
        const int shl = 4 * (r >> 2), shh = 2 * (r >> 1);
#pragma unroll
        for (int l = 0; l < 16; l++) {
            const int v = (int)(((byte_of(ql, l) >> shl) & 15u) | (((byte_of(qh, l) >> shh) & 3u) << 4)) - 32;
            o[l] = __fmul_rn(dl, (float)v);
        }
    }
}

template <int T>
__global__ __launch_bounds__(256) void k_dequant_blocks(const uint8_t *__restrict__ src, int64_t row_bytes,
                                                        int64_t nblk, int64_t rows, float *__restrict__ dst) {
    constexpr int BL = Fmt<T>::BL, BB = Fmt<T>::BB, P = Fmt<T>::P;
    const int64_t per_row = nblk * P;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * per_row) return;
    const int64_t row = gid / per_row;
    const int64_t rem = gid - row * per_row;
    const int64_t b = rem / P;
    const int G = (int)(rem - b * P);
    float o[16];
    deq_piece<T>(src + row * row_bytes + b * BB, G, o);
    f32x4 *out = reinterpret_cast<f32x4 *>(dst + row * nblk * BL + b * BL + 16 * G);
#pragma unroll
    for (int j = 0; j < 4; j++) out[j] = f32x4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
}

// F16 (fh3_quant.c:36-49, exact, F16C NaN quieting) and BF16 (:51-56, the bits
// are the top half of the fp32 word): one thread per element.
template <bool BF>
__global__ __launch_bounds__(256) void k_dequant_half(const uint8_t *__restrict__ src, int64_t row_bytes,
                                                      int64_t n, int64_t rows, float *__restrict__ dst) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * n) return;
    const int64_t row = gid / n;
    const int64_t i = gid - row * n;
    const uint32_t h = ld_u16(src + row * row_bytes + 2 * i);
    dst[gid] = BF ? __builtin_bit_cast(float, h << 16) : f16_to_f32_exact(h);
}

// ---------------------------------------------------------------------------
// Activation preparation.  One 256-thread workgroup per token row t, the whole
// row held in registers (V4 float4 per thread, K <= 1024 * V4).  Row t gets
// the scale 2^e with e = 15 - E, where max|x_t| = f * 2^E (f in [0.5, 1)), so
// its largest magnitude lands in [2^14, 2^15): fp16 never overflows and small
// rows keep full fp16 precision.  xs_inv[t] = 2^-e undoes it in the epilogue.
// Rows M..Mpad-1 are written as zeros.  Thread i owns float4 i, i+256, ...;
// float4 k4 is half (k4 & 1) of the 8 fp16 lane slot (t%32 + 32*((k4/2)&1))
// of fragment (t/32, k4/4).
// ---------------------------------------------------------------------------
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// Optional row normalisation applied before the scaling (the DiT block's
// rmsnorm + AdaLN modulate in front of its qkv and fc1 products, reference
// src/model/fh3_dit.c:383-386 and 430-433): when w is set,
//   x = (x * inv_rms) * w,  inv_rms = 1 / sqrt(sum(x*x) / K + eps)
// (src/core/fh3_ops.c:410-456), then, when shift is set,
//   x = fma(x, 1 + scale[t], shift[t])   (src/core/fh3_ops.c:529-557),
// shift / scale being [M][K] rows.
// Sum over each aligned group of 8 lanes (every lane of the group gets it).
// DPP read of v from another lane of its row of 16 (every lane is written:
// full row and bank masks), with no old operand, so the move folds into the
// VALU op that consumes it
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float sum8_f32(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    return v;
}

struct RowNorm {
    const float *w;
    float eps;
    const float *shift, *scale;
};

// Sum over the 256 threads of a workgroup, returned to every thread.
__device__ __forceinline__ float block_sum256(float v, float *s_red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    v = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    __syncthreads();
    return v;
}

template <int V4>
__device__ __forceinline__ void row_norm(f32x4 (&v)[V4], const RowNorm &nm, int t, int K, float *s_red) {
    const int tid = threadIdx.x, n4 = K / 4;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V4; i++)
        ss = __builtin_fmaf(v[i].w, v[i].w, __builtin_fmaf(v[i].z, v[i].z,
             __builtin_fmaf(v[i].y, v[i].y, __builtin_fmaf(v[i].x, v[i].x, ss))));
    ss = block_sum256(ss, s_red);
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)K + nm.eps);
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(nm.w);
    const f32x4 *sh4 = reinterpret_cast<const f32x4 *>(nm.shift ? nm.shift + (size_t)t * K : nullptr);
    const f32x4 *sc4 = reinterpret_cast<const f32x4 *>(nm.scale ? nm.scale + (size_t)t * K : nullptr);
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int k4 = tid + 256 * i;
        if (k4 < n4) {
            const f32x4 w = w4[k4];
            f32x4 y = {(v[i].x * inv) * w.x, (v[i].y * inv) * w.y, (v[i].z * inv) * w.z, (v[i].w * inv) * w.w};
            if (sh4) {
                const f32x4 a = sh4[k4], c = sc4[k4];
                y = f32x4{__builtin_fmaf(y.x, 1.0f + c.x, a.x), __builtin_fmaf(y.y, 1.0f + c.y, a.y),
                          __builtin_fmaf(y.z, 1.0f + c.z, a.z), __builtin_fmaf(y.w, 1.0f + c.w, a.w)};
            }
            v[i] = y;
        }
    }
}

template <int V4>
__global__ __launch_bounds__(256) void k_xprep(const float *__restrict__ X, int M, int K,
                                               half8 *__restrict__ X16, float *__restrict__ xs_inv, RowNorm nm,
                                               float *__restrict__ xsum) {
    __shared__ float s_red[4];
    // Consecutive workgroup ids go to different XCDs; give each XCD a
    // contiguous run of rows instead, so that neighbouring rows, which share
    // 32-byte pieces of the same fragments, are written through one L2 and
    // merge there (gridDim.x = Mpad, a multiple of 8).
    const int t = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n4 = K / 4;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(X + (size_t)t * K);
    f32x4 v[V4];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int k4 = tid + 256 * i;
        v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (t < M && k4 < n4) v[i] = xr[k4];
    }
    if (nm.w && t < M) row_norm<V4>(v, nm, t, K, s_red);  // uniform per workgroup
#pragma unroll
    for (int i = 0; i < V4; i++)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    int e = 0;
    if (mx > 0.f && mx <= 3.4028234663852886e38f) {
        int E;
        (void)frexpf(mx, &E);
        e = 15 - E;
        e = e > 126 ? 126 : (e < -126 ? -126 : e);
    }
    const float s = ldexpf(1.0f, e);
    if (tid == 0) xs_inv[t] = ldexpf(1.0f, -e);
    const int kf_n = K / 16;
    half4 *dst = reinterpret_cast<half4 *>(X16 + (size_t)(t >> 5) * kf_n * 64 + (t & 31));
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int k4 = tid + 256 * i;
        if (k4 < n4) {  // uniform per wavefront: n4 is a multiple of 64
            const half4 h = {(_Float16)(v[i].x * s), (_Float16)(v[i].y * s), (_Float16)(v[i].z * s),
                             (_Float16)(v[i].w * s)};
            // fragment k4/4, lane half (k4/2)&1, 8-byte half k4&1
            dst[(size_t)(k4 >> 2) * 128 + ((k4 >> 1) & 1) * 64 + (k4 & 1)] = h;
            if (xsum) {
                // sums of the 32 fp16 values of each group (the 8 aligned
                // lanes around this one), as the sweep kernel's offset term
                // multiplies them
                const float gs = sum8_f32(((float)h.x + (float)h.y) + ((float)h.z + (float)h.w));
                if (t < M && (lane & 7) == 0) xsum[(size_t)t * (K / 32) + (k4 >> 3)] = gs;
            }
        }
    }
}

// Activations of any row length K and alignment (rows of the run-once
// projections: 32, 96, 64 or 128 values, or more than 32768) -> X16 fragments
// of Kp = round_up(K, 256) columns, zeros at k >= K.  The scale rule and the
// rounding are k_xprep's, so for a K that k_xprep takes the output is the
// same bit for bit.  The row is read twice (its maximum, then the
// fragments), so K is not bounded by one workgroup's registers.  Rows
// M..gridDim.x-1 are written as zeros with scale 1.
__global__ __launch_bounds__(256) void k_xprep_any(const float *__restrict__ X, int M, int K, int Kp,
                                                   half8 *__restrict__ X16, float *__restrict__ xs_inv) {
    __shared__ float s_red[4];
    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *xr = X + (size_t)t * K;
    const int kv = t < M ? K : 0;
    float mx = 0.f;
    for (int k = tid; k < kv; k += 256) mx = fmaxf(mx, fabsf(xr[k]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    int e = 0;
    if (mx > 0.f && mx <= 3.4028234663852886e38f) {
        int E;
        (void)frexpf(mx, &E);
        e = 15 - E;
        e = e > 126 ? 126 : (e < -126 ? -126 : e);
    }
    const float s = ldexpf(1.0f, e);
    if (tid == 0) xs_inv[t] = ldexpf(1.0f, -e);
    const int kf_n = Kp / 16;
    half4 *dst = reinterpret_cast<half4 *>(X16 + (size_t)(t >> 5) * kf_n * 64 + (t & 31));
    for (int k4 = tid; k4 < Kp / 4; k4 += 256) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = 4 * k4 + i < kv ? xr[4 * k4 + i] : 0.f;
        const half4 h = {(_Float16)(v[0] * s), (_Float16)(v[1] * s), (_Float16)(v[2] * s), (_Float16)(v[3] * s)};
        // fragment k4/4, lane half (k4/2)&1, 8-byte half k4&1 (as k_xprep)
        dst[(size_t)(k4 >> 2) * 128 + ((k4 >> 1) & 1) * 64 + (k4 & 1)] = h;
    }
}

// Large-M preparation: RW = 8 (or 4) consecutive rows per 1024-thread
// workgroup.  Thread (r = lane % RW, cc = tid / RW) owns row t0 + r and its
// 8-float chunks c = cc + (1024/RW) i (V per thread, K <= 8 V (1024/RW)).  The
// 8 lanes that share a chunk hold the 8 rows' 16-byte slots of fragment c/2,
// lane half c%2: one aligned 128-byte line per store (64 bytes with RW = 4, used
// at K > 8192, where 8 rows would need 112 VGPRs of activations per thread), where k_xprep's rows each write 16 of a line's 128
// bytes and rely on the L2 to merge them (measured at M = 32768: 5.2 against
// 3.5 TB/s at K = 5120, 4.4 against 3.0 at K = 13824).  Same scale rule and
// rounding as k_xprep; with NORM the row sum of squares is added in another
// order (lanes, then the 16 wavefronts).
template <int V, bool NORM, int RW = 8>
__global__ __launch_bounds__(1024) void k_xprep_r8(const float *__restrict__ X, int M, int K,
                                                   half8 *__restrict__ X16, float *__restrict__ xs_inv, RowNorm nm) {
    constexpr int CPI = 1024 / RW;  // chunks per pass
    __shared__ float s_red[16][RW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & (RW - 1), cc = tid / RW;
    const int t = (int)blockIdx.x * RW + r;
    const int n8 = K / 8;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(X + (size_t)t * K);
    f32x4 v[V][2];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = cc + CPI * i;
        v[i][0] = v[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (t < M && c < n8) {
            v[i][0] = xr[2 * c];
            v[i][1] = xr[2 * c + 1];
        }
    }
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < V; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                ss = __builtin_fmaf(v[i][j].w, v[i][j].w, __builtin_fmaf(v[i][j].z, v[i][j].z,
                     __builtin_fmaf(v[i][j].y, v[i][j].y, __builtin_fmaf(v[i][j].x, v[i][j].x, ss))));
#pragma unroll
        for (int o = RW; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
        if (lane < RW) s_red[wave][lane] = ss;
        __syncthreads();
        ss = s_red[0][r];
#pragma unroll
        for (int w = 1; w < 16; w++) ss += s_red[w][r];
        __syncthreads();  // s_red is reused for the maximum
        const float inv = 1.0f / __builtin_sqrtf(ss / (float)K + nm.eps);
        if (t < M) {
            const f32x4 *w4 = reinterpret_cast<const f32x4 *>(nm.w);
            const f32x4 *sh4 = reinterpret_cast<const f32x4 *>(nm.shift ? nm.shift + (size_t)t * K : nullptr);
            const f32x4 *sc4 = reinterpret_cast<const f32x4 *>(nm.scale ? nm.scale + (size_t)t * K : nullptr);
#pragma unroll
            for (int i = 0; i < V; i++) {
                const int c = cc + CPI * i;
                if (c < n8) {
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const f32x4 w = w4[2 * c + j], x = v[i][j];
                        f32x4 y = {(x.x * inv) * w.x, (x.y * inv) * w.y, (x.z * inv) * w.z, (x.w * inv) * w.w};
                        if (sh4) {
                            const f32x4 a = sh4[2 * c + j], b = sc4[2 * c + j];
                            y = f32x4{__builtin_fmaf(y.x, 1.0f + b.x, a.x), __builtin_fmaf(y.y, 1.0f + b.y, a.y),
                                      __builtin_fmaf(y.z, 1.0f + b.z, a.z), __builtin_fmaf(y.w, 1.0f + b.w, a.w)};
                        }
                        v[i][j] = y;
                    }
                }
            }
        }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i][j].x), fabsf(v[i][j].y)), fmaxf(fabsf(v[i][j].z), fabsf(v[i][j].w))));
#pragma unroll
    for (int o = RW; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane < RW) s_red[wave][lane] = mx;
    __syncthreads();
    mx = s_red[0][r];
#pragma unroll
    for (int w = 1; w < 16; w++) mx = fmaxf(mx, s_red[w][r]);
    int e = 0;
    if (mx > 0.f && mx <= 3.4028234663852886e38f) {
        int E;
        (void)frexpf(mx, &E);
        e = 15 - E;
        e = e > 126 ? 126 : (e < -126 ? -126 : e);
    }
    const float s = ldexpf(1.0f, e);
    if (cc == 0) xs_inv[t] = ldexpf(1.0f, -e);
    half8 *dst = X16 + (size_t)(t >> 5) * (K / 16) * 64 + (t & 31);
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = cc + CPI * i;
        if (c < n8) {
            const f32x4 a = v[i][0], b = v[i][1];
            const half8 h = {(_Float16)(a.x * s), (_Float16)(a.y * s), (_Float16)(a.z * s), (_Float16)(a.w * s),
                             (_Float16)(b.x * s), (_Float16)(b.y * s), (_Float16)(b.z * s), (_Float16)(b.w * s)};
            dst[(size_t)(c >> 1) * 64 + (c & 1) * 32] = h;
        }
    }
}

// The same normalisation into fp32 rows (the prepared form of the one- and
// two-token kernel, and the device form of rmsnorm / modulate): one
// workgroup per row, Y may alias X.
template <int V4>
__global__ __launch_bounds__(256) void k_rownorm_f32(const float *X, int K, float *Y,
                                                     RowNorm nm) {
    __shared__ float s_red[4];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = K / 4;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(X + (size_t)t * K);
    f32x4 v[V4];
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int k4 = tid + 256 * i;
        v[i] = k4 < n4 ? xr[k4] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    row_norm<V4>(v, nm, t, K, s_red);
    f32x4 *yr = reinterpret_cast<f32x4 *>(Y + (size_t)t * K);
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int k4 = tid + 256 * i;
        if (k4 < n4) yr[k4] = v[i];
    }
}

// ---------------------------------------------------------------------------
// Product epilogues (runtime, uniform per launch): the DiT block's operations
// right after its linears, reference src/model/fh3_dit.c:416, 436, 439.
//   EPI_NONE      Y[t][o] = y
//   EPI_GATE_RES  Y[t][o] = fma(aux[t][o], y, Y[t][o])      (fh3_gate_residual,
//                 src/core/fh3_ops.c:559-585; Y is the residual stream h)
//   EPI_SWIGLU    the weight has 2F rows [val | gate]; Y[t][j] = val_j * silu(gate_j)
//                 with Y of width F (fh3_swiglu, src/core/fh3_ops.c:507-527);
//                 a workgroup then owns output columns and takes rows j and
//                 F + j together.
// y is the product value with bias, exactly what fh3_matmul would store.
// ---------------------------------------------------------------------------
constexpr int EPI_NONE = 0, EPI_GATE_RES = 1, EPI_SWIGLU = 2;

// silu(g) = g / (1 + exp(-g)), 0 below -80 (src/core/fh3_ops.c:515-520)
__device__ __forceinline__ float silu_f32(float g) { return g < -80.0f ? 0.0f : g / (1.0f + expf(-g)); }

__device__ __forceinline__ void epi_store(float *Y, const float *aux, int epi, size_t idx, float y) {
    if (epi == EPI_GATE_RES) Y[idx] = __builtin_fmaf(aux[idx], y, Y[idx]);
    else Y[idx] = y;
}

// ---------------------------------------------------------------------------
// Small-M helpers
// ---------------------------------------------------------------------------
// Lane-constant field positions of the 6-bit scale/min of group g
// (reference src/core/fh3_quant.c:168-177): low 4 bits come from byte g of the
// scale (min) word pair when g < 4, else from the low (high) nibble of byte
// 8 + g%4; the top 2 bits from bits 4-5 of byte g (g < 4) or bits 6-7 of byte
// g%4 of the scale (min) word.
struct Q4kField {
    int lo_sh;   // shift of the 4 low bits in the selected word
    int hi_sh;   // shift of the 2 high bits in the scale / min word
    bool upper;  // g >= 4: low bits live in word s2
};

__device__ __forceinline__ Q4kField q4k_field(int g) {
    Q4kField f;
    const int j = g & 3;
    f.upper = g >= 4;
    f.lo_sh = 8 * j;
    f.hi_sh = 8 * j + (f.upper ? 6 : 4);
    return f;
}

__device__ __forceinline__ uint32_t q4k_sc(const u32x4 h, const Q4kField f) {
    const uint32_t lo = f.upper ? (h.w >> f.lo_sh) : (h.y >> f.lo_sh);
    return (lo & 15u) | (((h.y >> f.hi_sh) & 3u) << 4);
}

__device__ __forceinline__ uint32_t q4k_mn(const u32x4 h, const Q4kField f) {
    const uint32_t lo = f.upper ? (h.w >> (f.lo_sh + 4)) : (h.z >> f.lo_sh);
    return (lo & 15u) | (((h.z >> f.hi_sh) & 3u) << 4);
}

__device__ __forceinline__ half2v splat2(uint32_t v) {
    const _Float16 h = (_Float16)(float)v;
    return half2v{h, h};
}

// Eight exact integer weights sc*q (<= 945) of one group as fp16, from 8 bytes
// of nibbles: (1024 + q) * sc - 1024 * sc in one fused fp16 op per pair
// (v_pk_fma_f16; the fused result is an integer below 2048, hence exact).
__device__ __forceinline__ half8 q4k_scq8_f16(uint32_t u0, uint32_t u1, bool hi, half2v sc2, half2v nsc2) {
    const uint32_t a = (hi ? (u0 >> 4) : u0) & 0x0F0F0F0Fu;
    const uint32_t b = (hi ? (u1 >> 4) : u1) & 0x0F0F0F0Fu;
    const half2v p0 = __builtin_elementwise_fma(q4k_magic_pair(a, 0x04010400u), sc2, nsc2);
    const half2v p1 = __builtin_elementwise_fma(q4k_magic_pair(a, 0x04030402u), sc2, nsc2);
    const half2v p2 = __builtin_elementwise_fma(q4k_magic_pair(b, 0x04010400u), sc2, nsc2);
    const half2v p3 = __builtin_elementwise_fma(q4k_magic_pair(b, 0x04030402u), sc2, nsc2);
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Activation fragments of super-block s0 + i for MFMA m = 0..7 of lane
// (token, q): k = sb*256 + (2q + m/4)*32 + 8*(m%4) -> fragment
// sb*16 + 4q + 2*(m/4) + (m%4)/2, lane half (m % 2) of it.  xq[tb] already
// points at fragment s0*16 + 4q of the lane's token, so with i a compile-time
// constant every offset below is one too.  HI is the fragment distance of the
// MFMAs m >= 4 from the first four: 2 for Q4_K / Q5_K (groups 2q and 2q+1),
// 4 for Q6_K (k ranges 64 apart, see sk6_superblock).
template <int TB, int HI = 2>
__device__ __forceinline__ void skinny_load_a(const half8 *const xq[TB], int i, half8 (&a)[8][TB]) {
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int off = (i * 16 + (m >= 4 ? HI : 0) + ((m & 3) >> 1)) * 64 + (m & 1) * 32;
#pragma unroll
        for (int tb = 0; tb < TB; tb++) a[m][tb] = xq[tb][off];
    }
}

// One super-block of the small-M product with exact weights.  With
// w = d*sc_g*q - dmin*m_g, the super-block contributes
//   d * sum_k (sc_g q)_k x_k - dmin * sum_k m_g(k) x_k,
// two MFMA chains over the same activation fragments (B = sc*q, and B = m
// broadcast over each group), scaled by d and dmin in fp32 afterwards.
// `valid` false (a padding super-block) contributes zero.
// With next >= 0 (one activation buffer: two or more token blocks), each MFMA
// step's fragments a[m][*] are reloaded with super-block `next` of the window
// (xq as in skinny_load_a) as soon as the step has used them, so the next
// super-block's activations arrive while this one computes.
template <int TB, int HI = 2>
__device__ __forceinline__ void skinny_superblock(const u32x4 hv, const u32x4 ca, const u32x4 cb, bool valid,
                                                  const Q4kField flo, const Q4kField fhi, half8 (&a)[8][TB],
                                                  f32x4 acc[TB], const half8 *const *xq = nullptr, int next = -1) {
    const float d = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(hv.x & 0xFFFFu)) : 0.f;
    const float dmin = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(hv.x >> 16)) : 0.f;
    const uint32_t sclo = q4k_sc(hv, flo), schi = q4k_sc(hv, fhi);
    const half2v sc_lo = splat2(sclo), sc_hi = splat2(schi);
    const half2v nsc_lo = splat2(sclo) * (_Float16)-1024.0f, nsc_hi = splat2(schi) * (_Float16)-1024.0f;
    const half2v m_lo = splat2(q4k_mn(hv, flo)), m_hi = splat2(q4k_mn(hv, fhi));
    const half8 bm_lo = half8{m_lo[0], m_lo[1], m_lo[0], m_lo[1], m_lo[0], m_lo[1], m_lo[0], m_lo[1]};
    const half8 bm_hi = half8{m_hi[0], m_hi[1], m_hi[0], m_hi[1], m_hi[0], m_hi[1], m_hi[0], m_hi[1]};
    f32x4 aq[TB], am[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) aq[tb] = am[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int part = m & 3;
        const bool hi = m >= 4;
        const u32x4 cv = part < 2 ? ca : cb;
        const uint32_t u0 = (part & 1) ? cv.z : cv.x;
        const uint32_t u1 = (part & 1) ? cv.w : cv.y;
        const half8 b = q4k_scq8_f16(u0, u1, hi, hi ? sc_hi : sc_lo, hi ? nsc_hi : nsc_lo);
#pragma unroll
        for (int tb = 0; tb < TB; tb++) {
            aq[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], b, aq[tb], 0, 0, 0);
            am[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], hi ? bm_hi : bm_lo, am[tb], 0, 0, 0);
        }
        if (next >= 0) {
            const int off = (next * 16 + (m >= 4 ? HI : 0) + ((m & 3) >> 1)) * 64 + (m & 1) * 32;
#pragma unroll
            for (int tb = 0; tb < TB; tb++) a[m][tb] = xq[tb][off];
        }
    }
    // d and dmin belong to the weight row j = lane % 16, which is the output
    // column this lane holds
#pragma unroll
    for (int tb = 0; tb < TB; tb++)
#pragma unroll
        for (int v = 0; v < 4; v++)
            acc[tb][v] = __builtin_fmaf(d, aq[tb][v], __builtin_fmaf(-dmin, am[tb][v], acc[tb][v]));
}

// Raw bytes one lane holds for one super-block in k_skinny, per weight type,
// and their loads.  wh points at the super-block, wa / wb at this lane's
// pieces of it (set once per launch, so every load has a compile-time offset).
//   Q4_K (144 B): header (d, dmin, 12 B of scales/mins), chunk q (32 B).
//   Q5_K (176 B, src/core/fh3_quant.c:198-237): the same header, the 32
//     high-bit bytes qh (bit g of byte l = bit 4 of element l of group g),
//     chunk q of the low nibbles (at 48 + 32q).
//   Q6_K (210 B, src/core/fh3_quant.c:239-282): ql bytes 32q..32q+31, the 32
//     qh bytes of half q/2, the 16 int8 scales and d.  Q6_K super-blocks are
//     only 2-byte aligned; the 16-byte loads of these pieces are unaligned
//     global loads (supported on this GPU), every byte inside the block.
template <int QT> struct SkRaw { u32x4 hv, ca, cb; };
template <> struct SkRaw<FH3K_Q5_K> { u32x4 hv, h0, h1, ca, cb; };
template <> struct SkRaw<FH3K_Q6_K> { u32x4 l0, l1, h0, h1, sc; uint32_t d; };

template <int QT>
constexpr int sk_bytes() { return QT == FH3K_Q5_K ? 176 : (QT == FH3K_Q6_K ? 210 : 144); }

typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ u32x4 ld16u(const uint8_t *p) {
    return *reinterpret_cast<const u32x4u *>(p);
}

// lane pointers of super-block s0 for chunk / quarter q
template <int QT>
__device__ __forceinline__ void sk_lane_ptrs(const uint8_t *wh, int q, const uint8_t *&wa, const uint8_t *&wb) {
    if constexpr (QT == FH3K_Q6_K) {
        wa = wh + 32 * q;                  // ql
        wb = wh + 128 + 32 * (q >> 1);     // qh of this half
    } else {
        wa = wh + (QT == FH3K_Q5_K ? 48 : 16) + 32 * q;  // the chunk
        wb = wh;
    }
}

template <int QT>
__device__ __forceinline__ void sk_load(SkRaw<QT> &r, const uint8_t *wh, const uint8_t *wa, const uint8_t *wb,
                                        int s) {
    constexpr int B = sk_bytes<QT>();
    if constexpr (QT == FH3K_Q6_K) {
        r.l0 = ld16u(wa + s * B);
        r.l1 = ld16u(wa + s * B + 16);
        r.h0 = ld16u(wb + s * B);
        r.h1 = ld16u(wb + s * B + 16);
        r.sc = ld16u(wh + s * B + 192);
        r.d = ld_u16(wh + s * B + 208);
    } else {
        r.hv = ld16(wh + s * B);
        r.ca = ld16(wa + s * B);
        r.cb = ld16(wa + s * B + 16);
        if constexpr (QT == FH3K_Q5_K) {
            r.h0 = ld16(wh + s * B + 16);
            r.h1 = ld16(wh + s * B + 32);
        }
    }
}

// Eight fp16 from 8 bytes of small unsigned integers v (a = bytes 0-3, b =
// bytes 4-7): fma(1024 + v, s, ns) per pair, one rounding.
__device__ __forceinline__ half8 magic8_fma(uint32_t a, uint32_t b, half2v s, half2v ns) {
    const half2v p0 = __builtin_elementwise_fma(q4k_magic_pair(a, 0x04010400u), s, ns);
    const half2v p1 = __builtin_elementwise_fma(q4k_magic_pair(a, 0x04030402u), s, ns);
    const half2v p2 = __builtin_elementwise_fma(q4k_magic_pair(b, 0x04010400u), s, ns);
    const half2v p3 = __builtin_elementwise_fma(q4k_magic_pair(b, 0x04030402u), s, ns);
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Q5_K super-block: as skinny_superblock with q = low nibble | (high bit << 4)
// (0..31), so sc*q <= 63*31 = 1953 stays an exact fp16 integer.  MFMA m takes
// elements 8*(m%4)..+7 of group g = 2q + m/4 of lane (row j, q): chunk bytes
// and qh bytes 8*(m%4)..+7, bit g of the latter.
template <int TB>
__device__ __forceinline__ void sk5_superblock(const SkRaw<FH3K_Q5_K> &r, bool valid, int q, const Q4kField flo,
                                               const Q4kField fhi, const half8 (&a)[8][TB], f32x4 acc[TB]) {
    const u32x4 hv = r.hv;
    const float d = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(hv.x & 0xFFFFu)) : 0.f;
    const float dmin = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(hv.x >> 16)) : 0.f;
    const uint32_t sclo = q4k_sc(hv, flo), schi = q4k_sc(hv, fhi);
    const half2v sc_lo = splat2(sclo), sc_hi = splat2(schi);
    const half2v nsc_lo = splat2(sclo) * (_Float16)-1024.0f, nsc_hi = splat2(schi) * (_Float16)-1024.0f;
    const half2v m_lo = splat2(q4k_mn(hv, flo)), m_hi = splat2(q4k_mn(hv, fhi));
    const half8 bm_lo = half8{m_lo[0], m_lo[1], m_lo[0], m_lo[1], m_lo[0], m_lo[1], m_lo[0], m_lo[1]};
    const half8 bm_hi = half8{m_hi[0], m_hi[1], m_hi[0], m_hi[1], m_hi[0], m_hi[1], m_hi[0], m_hi[1]};
    f32x4 aq[TB], am[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) aq[tb] = am[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int part = m & 3;
        const bool hi = m >= 4;
        const u32x4 cv = part < 2 ? r.ca : r.cb, hq = part < 2 ? r.h0 : r.h1;
        const uint32_t u0 = (part & 1) ? cv.z : cv.x, u1 = (part & 1) ? cv.w : cv.y;
        const uint32_t h0 = (part & 1) ? hq.z : hq.x, h1 = (part & 1) ? hq.w : hq.y;
        const int g = 2 * q + (hi ? 1 : 0);
        const uint32_t b0 = ((hi ? u0 >> 4 : u0) & 0x0F0F0F0Fu) | (((h0 >> g) & 0x01010101u) << 4);
        const uint32_t b1 = ((hi ? u1 >> 4 : u1) & 0x0F0F0F0Fu) | (((h1 >> g) & 0x01010101u) << 4);
        const half8 b = magic8_fma(b0, b1, hi ? sc_hi : sc_lo, hi ? nsc_hi : nsc_lo);
#pragma unroll
        for (int tb = 0; tb < TB; tb++) {
            aq[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], b, aq[tb], 0, 0, 0);
            am[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], hi ? bm_hi : bm_lo, am[tb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++)
#pragma unroll
        for (int v = 0; v < 4; v++)
            acc[tb][v] = __builtin_fmaf(d, aq[tb][v], __builtin_fmaf(-dmin, am[tb][v], acc[tb][v]));
}

// Q6_K super-block, w = d * sc_g * (q - 32) with q the 6-bit value and sc_g
// the signed scale of 16-element sub-group g.  Lane (row j, q) holds ql bytes
// 32q..32q+31 of its row: in half h = q/2 of the block (elements 128h..),
// low nibbles are elements 128h + 32(q%2) + b and high nibbles elements
// 128h + 64 + 32(q%2) + b, b = 0..31, whose 2 high bits are bits 2s..2s+1 of
// qh byte 32h + b (s = (element % 128) / 32).  MFMA m takes b = 8*(m%4)..+7 of
// the low (m < 4) or high nibbles: k = 128h + 32(q%2) + 64(m/4) + 8(m%4),
// fragment 8h + 2(q%2) + 4(m/4) + (m%4)/2 (skinny_load_a with HI = 4), and
// sub-group 8h + 2(q%2) + 4(m/4) + (m%4)/2, i.e. byte 2(q%2) + (m%4)/2 of
// scale word 2h + m/4.
// B = sc * (q - 32) per pair as one fused op on exact fp16 operands:
// q sits in mantissa bits 4-9 of 0x6400 | q << 4 = 1024 + 16q (the nibble in
// bits 4-7 of the low byte, the 2 high bits in bits 0-1 of the high byte, one
// v_perm per pair), and fma(1024 + 16q, sc/16, -96 sc) = sc * (q - 32) with
// sc/16 and -96 sc exact (|96 sc| <= 12288), rounded once: exact while
// |sc * (q - 32)| <= 2048 (the same single rounding k_gemm applies to every
// Q4_K weight), then scaled by d in fp32.  One token block after another
// reads the same B.
struct Sk6Ops { half2v s16[4], c96[4]; };

__device__ __forceinline__ Sk6Ops sk6_scale_ops(const SkRaw<FH3K_Q6_K> &r, int q) {
    const uint32_t w0 = (q >> 1) ? r.sc.z : r.sc.x, w1 = (q >> 1) ? r.sc.w : r.sc.y;
    const int sb = 16 * (q & 1);
    Sk6Ops o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = i < 2 ? w0 : w1;
        const float sv = (float)(int)(int8_t)(uint8_t)((w >> (sb + 8 * (i & 1))) & 0xFFu);
        const _Float16 a = (_Float16)(sv * 0.0625f), c = (_Float16)(sv * -96.0f);
        o.s16[i] = half2v{a, a};
        o.c96[i] = half2v{c, c};
    }
    return o;
}

// B operand of MFMA m (see above): 8 fp16 sc * (q - 32)
__device__ __forceinline__ half8 sk6_b(const SkRaw<FH3K_Q6_K> &r, int q, const Sk6Ops &o, int m) {
    const int part = m & 3;
    const bool hi = m >= 4;
    const u32x4 lq = part < 2 ? r.l0 : r.l1, hq = part < 2 ? r.h0 : r.h1;
    const uint32_t u0 = (part & 1) ? lq.z : lq.x, u1 = (part & 1) ? lq.w : lq.y;
    const uint32_t h0 = (part & 1) ? hq.z : hq.x, h1 = (part & 1) ? hq.w : hq.y;
    const int hs = 2 * (q & 1) + (hi ? 4 : 0);
    // nibble in bits 4-7 of each byte; 0x64 | high bits in each byte
    const uint32_t n0 = hi ? (u0 & 0xF0F0F0F0u) : ((u0 << 4) & 0xF0F0F0F0u);
    const uint32_t n1 = hi ? (u1 & 0xF0F0F0F0u) : ((u1 << 4) & 0xF0F0F0F0u);
    const uint32_t e0 = ((h0 >> hs) & 0x03030303u) | 0x64646464u, e1 = ((h1 >> hs) & 0x03030303u) | 0x64646464u;
    const half2v s = o.s16[(hi ? 2 : 0) + (part >> 1)], c = o.c96[(hi ? 2 : 0) + (part >> 1)];
    // pair (2i, 2i + 1) of a word: bytes [n.b2i, e.b2i, n.b2i+1, e.b2i+1]
    auto pair = [&](uint32_t e, uint32_t n, uint32_t sel) {
        return __builtin_elementwise_fma(__builtin_bit_cast(half2v, __builtin_amdgcn_perm(e, n, sel)), s, c);
    };
    const half2v p0 = pair(e0, n0, 0x05010400u), p1 = pair(e0, n0, 0x07030602u);
    const half2v p2 = pair(e1, n1, 0x05010400u), p3 = pair(e1, n1, 0x07030602u);
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int TB>
__device__ __forceinline__ void sk6_superblock(const SkRaw<FH3K_Q6_K> &r, bool valid, int q,
                                               const half8 (&a)[8][TB], f32x4 acc[TB]) {
    const float d = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(r.d & 0xFFFFu)) : 0.f;
    const Sk6Ops o = sk6_scale_ops(r, q);
    f32x4 aq[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) aq[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const half8 b = sk6_b(r, q, o, m);
#pragma unroll
        for (int tb = 0; tb < TB; tb++) aq[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], b, aq[tb], 0, 0, 0);
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[tb][v] = __builtin_fmaf(d, aq[tb][v], acc[tb][v]);
}

// ---------------------------------------------------------------------------
// Small-M kernel.  Workgroup = NW wavefronts (blockDim.x / 64, at most 8) over
// 16 consecutive weight rows o0..o0+15; wavefront w owns the C contiguous
// super-blocks [w*C, w*C + C) of those rows (NW*C >= K/256 >= C).  The last
// wavefront's window is moved back to [K/256 - C, K/256) so that every load
// stays inside the row; the super-blocks it shares with the previous
// wavefront count as padding (zero).  C is a compile-time constant, so the
// code is straight-line and every load has a compile-time offset from one
// per-lane pointer: a ring of min(C, RMAX) super-blocks of weights is in
// flight (loads pinned ahead of the compute with sched_barrier) and, for one
// token block, the activation fragments of the next super-block are loaded
// while the current one computes.
// MFMA 16x16x32: B lane l = (row j = l%16, chunk q = l/16) holds the 32 bytes of
// chunk q (groups 2q and 2q+1) plus the 16-byte header: each super-block of a
// row is read once, 144 B by 4 lanes.  MFMA m (0..7) takes from lane (j, q) the
// 8 weights of group 2q + m/4 at offsets 8*(m%4)..+7; the A lane (token i, q)
// holds the activations of the same k (one 16-byte piece of an X16
// fragment).  Partial sums of the NW waves are added in wave order through LDS
// (deterministic).
// QT selects the weight type: Q4_K, or Q5_K / Q6_K read in place (the lane
// pieces and products of SkRaw, sk5_superblock, sk6_superblock).
// Q5_K / Q6_K rows may also be split into K windows of L super-blocks
// (blockIdx.y = window; windows are what a workgroup's wavefronts divide, a
// short last window borrows super-blocks of the one before it as padding):
// each workgroup then writes its raw sums to part[window][t][o] and
// k_midm_sum adds the windows in order.  part = nullptr: one window, the
// epilogue here.
// ---------------------------------------------------------------------------
template <int QT, int TB, int C, int MAXT = 512, int RMAX = (TB == 1 ? 5 : 3)>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_skinny(
    const uint8_t *__restrict__ W, int64_t row_bytes, int N, int K, const half8 *__restrict__ X16,
    const float *__restrict__ xs_inv, const float *__restrict__ bias, float *__restrict__ Y, int M, int epi,
    const float *__restrict__ aux, int L = 0, float *__restrict__ part = nullptr) {
    constexpr bool KW = QT != FH3K_Q4_K;  // K windows available
    extern __shared__ f32x4 red[];  // [NW][TB][64]
    constexpr int RING = C < RMAX ? C : RMAX;
    constexpr int AB = TB == 1 ? 2 : 1;  // activation buffers
    const int NW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    // rows o0..o0+15, or (SwiGLU) rows o0..o0+7 and F+o0..F+o0+7
    const int F = N >> 1;
    const int o0 = epi == EPI_SWIGLU ? blockIdx.x * 8 : blockIdx.x * 16;
    const int orow = epi == EPI_SWIGLU ? (j < 8 ? o0 + j : F + o0 + j - 8) : (o0 + j < N ? o0 + j : N - 1);
    const int nsb = K / 256;
    const int kf_n = K / 16;
    // the K window [kb, kb + kn): the whole row, or window blockIdx.y
    const int kb = KW ? (int)blockIdx.y * L : 0;
    const int kn = KW && part ? (L < nsb - kb ? L : nsb - kb) : nsb;
    const int own = kb + wave * C;                         // first super-block this wave owns
    const int s0 = own < kb + kn - C ? own : kb + kn - C;  // its super-blocks, inside the row
    constexpr int SB = sk_bytes<QT>();
    const uint8_t *wh = W + (size_t)orow * row_bytes + (size_t)s0 * SB;  // super-block s0
    const uint8_t *wa, *wb;                                              // this lane's pieces of it
    sk_lane_ptrs<QT>(wh, q, wa, wb);
    constexpr int AHI = QT == FH3K_Q6_K ? 4 : 2;       // skinny_load_a's high-half distance

    f32x4 acc[TB];
    const half8 *xq[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) {
        acc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        // A-operand token of this lane; padding tokens re-read the last real
        // row (their output rows are never stored)
        int t = tb * 16 + j;
        t = t < M ? t : M - 1;
        // fragment of this lane's first k in super-block s0: 4q (Q4_K, Q5_K: chunk
        // q), 8(q/2) + 2(q%2) (Q6_K: see sk6_superblock)
        const int qf = QT == FH3K_Q6_K ? 8 * (q >> 1) + 2 * (q & 1) : 4 * q;
        xq[tb] = X16 + ((size_t)(t >> 5) * kf_n + (size_t)s0 * 16 + qf) * 64 + (t & 31);
    }
    const Q4kField flo = q4k_field(2 * q), fhi = q4k_field(2 * q + 1);

    SkRaw<QT> raw[RING];
#pragma unroll
    for (int s = 0; s < RING; s++) sk_load<QT>(raw[s], wh, wa, wb, s);
    half8 a[AB][8][TB];
    skinny_load_a<TB, AHI>(xq, 0, a[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < C; i++) {
        const int s = i % RING;
        const int ab = AB == 2 ? (i & 1) : 0;
        // Q4_K with one buffer and short windows (longer ones spill): the
        // fragments of super-block i were loaded during super-block i - 1
        // (skinny_superblock's next)
        constexpr bool PF = AB == 1 && QT == FH3K_Q4_K && C <= 4;
        if (AB == 2 && i + 1 < C) {
            skinny_load_a<TB, AHI>(xq, i + 1, a[(i + 1) & 1]);
        } else if (AB == 1 && i > 0 && !PF) {
            skinny_load_a<TB, AHI>(xq, i, a[0]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PF)
            skinny_superblock<TB, AHI>(raw[s].hv, raw[s].ca, raw[s].cb, s0 + i >= own, flo, fhi, a[0], acc, xq,
                                       i + 1 < C ? i + 1 : -1);
        else if constexpr (QT == FH3K_Q5_K)
            sk5_superblock<TB>(raw[s], s0 + i >= own, q, flo, fhi, a[ab], acc);
        else if constexpr (QT == FH3K_Q6_K)
            sk6_superblock<TB>(raw[s], s0 + i >= own, q, a[ab], acc);
        else
            skinny_superblock<TB>(raw[s].hv, raw[s].ca, raw[s].cb, s0 + i >= own, flo, fhi, a[ab], acc);
        if (i + RING < C) sk_load<QT>(raw[s], wh, wa, wb, i + RING);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++) red[(wave * TB + tb) * 64 + lane] = acc[tb];
    __syncthreads();
    // output D of 16x16: lane l holds column (weight row) l%16, rows (tokens)
    // 4*(l/16) + v; the workgroup may have fewer threads than TB*64
    for (int idx = threadIdx.x; idx < TB * 64; idx += blockDim.x) {
        const int tb = idx >> 6, l = idx & 63;
        if (KW && part) {  // this window's raw sums
            f32x4 s = red[tb * 64 + l];
            for (int w = 1; w < NW; w++) s += red[(w * TB + tb) * 64 + l];
            const int o = o0 + (l & 15);
            if (o < N) {
                float *pp = part + (size_t)blockIdx.y * M * N + o;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int t = tb * 16 + 4 * (l >> 4) + v;
                    if (t < M) pp[(size_t)t * N] = s[v];
                }
            }
            continue;
        }
        if (epi == EPI_SWIGLU) {
            if ((l & 15) >= 8) continue;  // the gate column of l is l + 8
            f32x4 sv = red[tb * 64 + l], sg = red[tb * 64 + l + 8];
            for (int w = 1; w < NW; w++) sv += red[(w * TB + tb) * 64 + l], sg += red[(w * TB + tb) * 64 + l + 8];
            const int o = o0 + (l & 15);
            const float bv = bias ? bias[o] : 0.f, bg = bias ? bias[F + o] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = tb * 16 + 4 * (l >> 4) + v;
                if (t < M) Y[(size_t)t * F + o] = (sv[v] * xs_inv[t] + bv) * silu_f32(sg[v] * xs_inv[t] + bg);
            }
            continue;
        }
        f32x4 s = red[tb * 64 + l];
        for (int w = 1; w < NW; w++) s += red[(w * TB + tb) * 64 + l];
        const int o = o0 + (l & 15);
        if (o < N) {
            const float bo = bias ? bias[o] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = tb * 16 + 4 * (l >> 4) + v;
                if (t < M) epi_store(Y, aux, epi, (size_t)t * N + o, s[v] * xs_inv[t] + bo);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Small-M sweep (k_sweep): TB token blocks (M <= 16 TB), persistent.  k_skinny
// reads a wavefront's activation fragments again for every 16-row block (as
// many bytes of fp16 activations per super-block as the Q4_K weights it
// multiplies, 16 tokens x 256 k x 2 B against 144 B x 16 rows); here each
// wavefront loads the fragments of its window once and keeps them in
// registers while its workgroup sweeps row blocks blockIdx.x, +gridDim.x, ...
// Work split and weight ring as k_gemv8: NW = ceil(nsb / C) wavefronts, window
// [s0, s0 + C) per wavefront (the last one moved back inside the row, shared
// super-blocks are padding), one ring slot per super-block of the window,
// refilled with the next block's super-block as soon as it is consumed.
//
// Arithmetic.  With w = d*sc*q - dmin*m, a super-block contributes
//   d * sum_k (sc*q)_k x_k  -  sum_g dmin*m_g * X_g,
// X_g the sum of the group's fp16 activations (made by the preparation).
// The first term is eight v_mfma_f32_16x16x32_f16 on B = sc*q, exact in fp16:
// low nibbles as (1024 + q)*sc - 1024*sc, high nibbles left in place as
// (1024 + 16q)*(sc/16) - 64*sc, one fused v_pk_fma_f16 per pair (the result is
// an integer below 2048, hence exact).  The second is two
// v_mfma_f32_16x16x4_f32 per super-block (A = X_g, B = dmin*m_g of groups c
// and c+4 for lane (row j, k-block c)), accumulated over the block.  The NW
// partial sums are added in wave order through LDS (deterministic).  On this
// GPU the VALU and the matrix core of a SIMD mostly take turns, so both the
// B-operand VALU work (per weight) and the MFMA count (per super-block) set
// the time: the offsets cost 2 MFMAs instead of 8.
// ---------------------------------------------------------------------------
__device__ __forceinline__ half2v magic_fma2(uint32_t a, uint32_t sel, half2v s, half2v ns) {
    return __builtin_elementwise_fma(q4k_magic_pair(a, sel), s, ns);
}

// sum_k (sc*q)_k x_k of one super-block for TB blocks of 16 tokens x 16
// weight rows (A: skinny_load_a's fragments; lane (row j, chunk c) holds chunk
// c of row j); each B operand is built once and used by every token block
// The 6-bit scales of groups 2q and 2q + 1 (the lane's chunk q) as exact fp16
// (sc_lo, sc_hi).  Byte g of {sc_b : scales[0..3]} is group g's scale once
// masked to 6 bits (groups 0-3 are the low bits of scales[0..3], sc_b holds
// groups 4-7; reference src/core/fh3_quant.c:168-177), so one v_perm with the
// lane's selector ssel = (2q, zero, 2q + 1, zero) takes both, and 0x6400 in
// each half makes it the fp16 value 1024 + sc.
__device__ __forceinline__ half2v q4k_sc_pair(const u32x4 h, uint32_t ssel) {
    const uint32_t sc_b = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t x = (__builtin_amdgcn_perm(sc_b, h.y, ssel) & 0x003F003Fu) | 0x64006400u;
    return __builtin_bit_cast(half2v, x) - half2v{(_Float16)1024.0f, (_Float16)1024.0f};
}

// The 6-bit mins of groups q and q + 4 in bytes 0 and 2: byte g of
// {m_b : scales[4..7]} is group g's min once masked (m_b holds groups 4-7),
// msel = (q, zero, 4 + q, zero).
__device__ __forceinline__ uint32_t q4k_mn_pair(const u32x4 h, uint32_t msel) {
    const uint32_t m_b = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    return __builtin_amdgcn_perm(m_b, h.z, msel) & 0x003F003Fu;
}

// The lane's scale operands, (1024 + q) * s - 1024 * s for the low nibbles and
// (1024 + 16q) * (s/16) - 64 * s for the high ones, all products exact in fp16
// (63 * 1024 < 65504).  One token block: both scales from one v_perm
// (q4k_sc_pair).  More token blocks: the two field decodes, which measured
// faster there (17-24 tokens at N = 17408: 21.8 against 24.5 us).
template <int TB>
__device__ __forceinline__ void sweep_scale_ops(const u32x4 hv, uint32_t ssel, const Q4kField flo,
                                                const Q4kField fhi, half2v &s_lo, half2v &ns_lo, half2v &s_hi,
                                                half2v &ns_hi) {
    if constexpr (TB == 1) {
        const half2v sc = q4k_sc_pair(hv, ssel);
        const half2v m = sc * half2v{(_Float16)1.0f, (_Float16)0.0625f};
        const half2v n = sc * half2v{(_Float16)-1024.0f, (_Float16)-64.0f};
        s_lo = __builtin_shufflevector(m, m, 0, 0), s_hi = __builtin_shufflevector(m, m, 1, 1);
        ns_lo = __builtin_shufflevector(n, n, 0, 0), ns_hi = __builtin_shufflevector(n, n, 1, 1);
    } else {
        const uint32_t sclo = q4k_sc(hv, flo), schi = q4k_sc(hv, fhi);
        s_lo = splat2(sclo), ns_lo = s_lo * (_Float16)-1024.0f;
        s_hi = splat2(schi) * (_Float16)0.0625f, ns_hi = splat2(schi) * (_Float16)-64.0f;
    }
}

template <int TB>
__device__ __forceinline__ void sweep_scq(const u32x4 hv, const u32x4 ca, const u32x4 cb, uint32_t ssel,
                                          const Q4kField flo, const Q4kField fhi, const half8 (&a)[8][TB],
                                          f32x4 (&aq)[TB]) {
    half2v s_lo, ns_lo, s_hi, ns_hi;
    sweep_scale_ops<TB>(hv, ssel, flo, fhi, s_lo, ns_lo, s_hi, ns_hi);
#pragma unroll
    for (int tb = 0; tb < TB; tb++) aq[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int part = m & 3;
        const bool hi = m >= 4;
        const u32x4 cv = part < 2 ? ca : cb;
        const uint32_t msk = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        const uint32_t u0 = ((part & 1) ? cv.z : cv.x) & msk, u1 = ((part & 1) ? cv.w : cv.y) & msk;
        const half2v s = hi ? s_hi : s_lo, ns = hi ? ns_hi : ns_lo;
        const half2v p0 = magic_fma2(u0, 0x04010400u, s, ns), p1 = magic_fma2(u0, 0x04030402u, s, ns);
        const half2v p2 = magic_fma2(u1, 0x04010400u, s, ns), p3 = magic_fma2(u1, 0x04030402u, s, ns);
        const half8 b = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
#pragma unroll
        for (int tb = 0; tb < TB; tb++) aq[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m][tb], b, aq[tb], 0, 0, 0);
    }
}

// QT: Q4_K, or Q6_K read in place (the ring holds SkRaw<Q6_K> pieces, the
// activation fragments follow sk6_superblock's k order, and there is no min
// term, so no group sums).
template <int C, int TB, int LB, int EPI, int QT = FH3K_Q4_K>
__global__ __launch_bounds__(LB) void k_sweep(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int K,
                                              const half8 *__restrict__ X16, const float *__restrict__ xs_inv,
                                              const float *__restrict__ xsum, const float *__restrict__ bias,
                                              float *__restrict__ Y, int M, const float *__restrict__ aux, int nblk,
                                              int S, float *__restrict__ part) {
    extern __shared__ f32x4 red[];  // [2][NW][TB][64]
    const int NW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int F = N >> 1;
    constexpr int ROWS = EPI == EPI_SWIGLU ? 8 : 16;  // output columns per block
    // K in S slices of SL super-blocks (S = 1: all of K): workgroup g takes
    // slice g % S and the row blocks g / S, + gridDim.x / S, ...; window
    // offsets below are relative to the slice's first super-block sbb
    const int nsb_all = K >> 8, kf_n = K >> 4;
    const int SL = (nsb_all + S - 1) / S;
    // Token groups: M above 16 TB tokens (rows of at most 16 super-blocks)
    // is split into TG groups of 16 TB tokens, each swept by its own
    // workgroups, which then hold only their group's activations.
    const int TG = (M + 16 * TB - 1) / (16 * TB);
    const int ks = (int)blockIdx.x % S, rs = (int)blockIdx.x / S;
    const int tg = rs % TG, gw = rs / TG, GW = (int)gridDim.x / (S * TG);
    const int t0 = tg * 16 * TB;  // first token of this workgroup's group
    const int sbb = ks * SL;
    const int nsb = SL < nsb_all - sbb ? SL : nsb_all - sbb;
    const int own = wave * C;
    const int s0 = own < nsb - C ? own : nsb - C;
    const int nit = (nblk - gw + GW - 1) / GW;

    // weight row of this lane in block it: rows o0..o0+15, or (SwiGLU) value
    // rows o0..o0+7 and gate rows F+o0..F+o0+7
    auto wptr = [&](int it) {
        const int o0 = (gw + it * GW) * ROWS;
        int orow = EPI == EPI_SWIGLU ? (j < 8 ? o0 + j : F + o0 + j - 8) : o0 + j;
        orow = orow < N ? orow : N - 1;
        return W + (size_t)orow * row_bytes + (size_t)(sbb + s0) * sk_bytes<QT>();
    };
    constexpr bool Q6 = QT == FH3K_Q6_K;
    u32x4 hv[C], ca[C], cb[C];
    SkRaw<FH3K_Q6_K> r6[Q6 ? C : 1];
    if constexpr (Q6) {
        const uint8_t *wh = wptr(0), *wa, *wb;
        sk_lane_ptrs<FH3K_Q6_K>(wh, q, wa, wb);
#pragma unroll
        for (int s = 0; s < C; s++) sk_load<FH3K_Q6_K>(r6[s], wh, wa, wb, s);
    } else {
        const uint8_t *wh = wptr(0), *wc = wh + 16 + 32 * q;
#pragma unroll
        for (int s = 0; s < C; s++) {
            hv[s] = ld16(wh + s * 144);
            ca[s] = ld16(wc + s * 144);
            cb[s] = ld16(wc + s * 144 + 16);
        }
    }
    // A fragments and group sums of the window for tokens 16 tb + j (padding
    // tokens re-read the last real row; their outputs are never stored)
    half8 a[C][8][TB];
    float xg[C][TB][2];
    {
        const half8 *xq[TB];
        const float *xs[TB];
#pragma unroll
        for (int tb = 0; tb < TB; tb++) {
            const int t = t0 + 16 * tb + j < M ? t0 + 16 * tb + j : M - 1;
            const int qf = Q6 ? 8 * (q >> 1) + 2 * (q & 1) : 4 * q;  // see skinny_load_a
            xq[tb] = X16 + ((size_t)(t >> 5) * kf_n + (size_t)(sbb + s0) * 16 + qf) * 64 + (t & 31);
            xs[tb] = Q6 ? nullptr : xsum + (size_t)t * (K >> 5) + (size_t)(sbb + s0) * 8 + q;
        }
#pragma unroll
        for (int i = 0; i < C; i++) {
            skinny_load_a<TB, Q6 ? 4 : 2>(xq, i, a[i]);
            if constexpr (!Q6) {
#pragma unroll
                for (int tb = 0; tb < TB; tb++) {
                    xg[i][tb][0] = xs[tb][i * 8];
                    xg[i][tb][1] = xs[tb][i * 8 + 4];
                }
            }
        }
    }
    // the scales of groups 2q (low nibbles) and 2q + 1 and the mins of groups
    // q and q + 4 (the offset MFMA's k): byte selectors (one token block) or
    // field positions
    const uint32_t ssel = (uint32_t)(2 * q) | 0x0C00u | ((uint32_t)(2 * q + 1) << 16) | 0x0C000000u;
    const uint32_t msel = (uint32_t)q | 0x0C00u | ((uint32_t)(4 + q) << 16) | 0x0C000000u;
    const Q4kField flo = q4k_field(2 * q), fhi = q4k_field(2 * q + 1);
    const Q4kField fm0 = q4k_field(q), fm1 = q4k_field(q + 4);

    // the output this thread stores after each block, if any: lane st_l of
    // the 16x16 result holds column st_l % 16 and tokens 4 (st_l / 16) + v.
    // The four storing wavefronts (one per v) are 0-3, one per SIMD, except
    // with ten: waves w and w + 4 share a SIMD, so ten put three on SIMDs 0
    // and 1 and two on SIMDs 2 and 3, and the stores go to waves 2, 3, 6 and
    // 7, off the path to the next barrier (16 tokens, N = 17408: 16.7-17.0
    // against 17.3-17.5 us; the same bits).  With fewer than four wavefronts
    // (in <= 1536), or two token blocks, the threads of the workgroup take the
    // TB x 256 outputs in turn (st_all).
    const bool st_all = blockDim.x < 256 || part || TB > 1;
    const int sw = (int)threadIdx.x >> 6;
    const int st_v = NW == 10 ? (sw == 2 ? 0 : sw == 3 ? 1 : sw == 6 ? 2 : sw == 7 ? 3 : -1) : (sw < 4 ? sw : -1);
    const int st_l = (int)threadIdx.x & 63;
    const int st_t = t0 + 4 * (st_l >> 4) + (st_v < 0 ? 0 : st_v), st_j = st_l & 15;
    const bool storer = !st_all && st_v >= 0 && st_t < M && (EPI != EPI_SWIGLU || st_j < 8);
    const size_t mn = (size_t)M * N;
    const float st_xs = storer ? xs_inv[st_t] : 0.f;
    // one output (token t, column o = o0 + jj) from the NW partial sums of
    // result lane l, register v (rb: this token block's [NW][TB][64] slice)
    // (the partial sums are read as floats: register v of lane l is float
    // 4 l + v, one 4-byte LDS read each instead of a 16-byte read and a select)
    auto store = [&](const f32x4 *rb, int l, int v, int t, int o, float xs, float b, float bg, float ax, float y0) {
        const float *rf = reinterpret_cast<const float *>(rb) + v;
        float s = rf[4 * l];
        for (int w = 1; w < NW; w++) s += rf[4 * (w * TB * 64 + l)];
        if (EPI == EPI_SWIGLU) {  // the gate of column l % 16 is row l % 16 + 8 of the block
            float sg = rf[4 * (l + 8)];
            for (int w = 1; w < NW; w++) sg += rf[4 * (w * TB * 64 + l + 8)];
            Y[(size_t)t * F + o] = (s * xs + b) * silu_f32(sg * xs + bg);
        } else if (EPI == EPI_GATE_RES) {
            Y[(size_t)t * N + o] = __builtin_fmaf(ax, s * xs + b, y0);
        } else {
            Y[(size_t)t * N + o] = s * xs + b;
        }
    };

    auto block = [&](int it, auto more_tag) {
        constexpr bool MORE = decltype(more_tag)::value;
        const int o0 = (gw + it * GW) * ROWS;
        const int st_o = o0 + st_j;
        const bool st_ok = storer && st_o < N;
        float e_b = 0.f, e_bg = 0.f, e_aux = 0.f, e_y = 0.f;
        if (st_ok) {
            if (bias) {
                e_b = bias[st_o];
                if (EPI == EPI_SWIGLU) e_bg = bias[F + st_o];
            }
            if (EPI == EPI_GATE_RES) {
                e_aux = aux[(size_t)st_t * N + st_o];
                e_y = Y[(size_t)st_t * N + st_o];
            }
        }
        f32x4 acc[TB], accm[TB];
#pragma unroll
        for (int tb = 0; tb < TB; tb++) acc[tb] = accm[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const uint8_t *nh = wptr(MORE ? it + 1 : it), *nc = nh + 16 + 32 * q;
        if constexpr (Q6) {
            const uint8_t *na, *nb;
            sk_lane_ptrs<FH3K_Q6_K>(nh, q, na, nb);
#pragma unroll
            for (int i = 0; i < C; i++) {
                sk6_superblock<TB>(r6[i], s0 + i >= own, q, a[i], acc);
                if (MORE) sk_load<FH3K_Q6_K>(r6[i], nh, na, nb, i);
            }
        }
#pragma unroll
        for (int i = 0; i < (Q6 ? 0 : C); i++) {
            const u32x4 h = hv[i];
            const bool valid = s0 + i >= own;
            const float d = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xFFFFu)) : 0.f;
            const float dmin = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16)) : 0.f;
            f32x4 aq[TB];
            sweep_scq<TB>(h, ca[i], cb[i], ssel, flo, fhi, a[i], aq);
            float bm0, bm1;
            if constexpr (TB == 1) {
                const uint32_t mp = q4k_mn_pair(h, msel);
                bm0 = dmin * (float)(mp & 0xFFu), bm1 = dmin * (float)(mp >> 16);
            } else {
                bm0 = dmin * (float)q4k_mn(h, fm0), bm1 = dmin * (float)q4k_mn(h, fm1);
            }
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {
#pragma unroll
                for (int v = 0; v < 4; v++) acc[tb][v] = __builtin_fmaf(d, aq[tb][v], acc[tb][v]);
                accm[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xg[i][tb][0], bm0, accm[tb], 0, 0, 0);
                accm[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xg[i][tb][1], bm1, accm[tb], 0, 0, 0);
            }
            if (MORE) {
                hv[i] = ld16(nh + i * 144);
                ca[i] = ld16(nc + i * 144);
                cb[i] = ld16(nc + i * 144 + 16);
            }
        }
        f32x4 *rb = red + (it & 1) * NW * TB * 64;  // alternate buffers: one barrier per block
#pragma unroll
        for (int tb = 0; tb < TB; tb++) rb[(wave * TB + tb) * 64 + lane] = acc[tb] - accm[tb];
        __syncthreads();
        if (st_ok) store(rb, st_l, st_v, st_t, st_o, st_xs, e_b, e_bg, e_aux, e_y);
        if (part) {  // K slices: this slice's raw sums of every row of the block
            for (int idx = (int)threadIdx.x; idx < TB * 256; idx += (int)blockDim.x) {
                const int tb = idx >> 8, l = idx & 63, v = (idx >> 6) & 3, jj = l & 15;
                const int t = t0 + 16 * tb + 4 * (l >> 4) + v;
                const int col = EPI == EPI_SWIGLU ? o0 + (jj & 7) : o0 + jj;
                if (t >= M || col >= (EPI == EPI_SWIGLU ? F : N)) continue;
                const float *rt = reinterpret_cast<const float *>(rb + tb * 64) + v;
                float sv = rt[4 * l];
                for (int w = 1; w < NW; w++) sv += rt[4 * (w * TB * 64 + l)];
                part[(size_t)ks * mn + (size_t)t * N + (EPI == EPI_SWIGLU && jj >= 8 ? F + col : col)] = sv;
            }
        } else if (st_all) {
            for (int idx = (int)threadIdx.x; idx < TB * 256; idx += (int)blockDim.x) {
                const int tb = idx >> 8, l = idx & 63, v = (idx >> 6) & 3;
                const int t = t0 + 16 * tb + 4 * (l >> 4) + v, o = o0 + (l & 15);
                if (t >= M || o >= N || (EPI == EPI_SWIGLU && (l & 15) >= 8)) continue;
                const float b = bias ? bias[o] : 0.f, bg = (bias && EPI == EPI_SWIGLU) ? bias[F + o] : 0.f;
                const float ax = EPI == EPI_GATE_RES ? aux[(size_t)t * N + o] : 0.f;
                const float y0 = EPI == EPI_GATE_RES ? Y[(size_t)t * N + o] : 0.f;
                store(rb + tb * 64, l, v, t, o, xs_inv[t], b, bg, ax, y0);
            }
        }
    };
    // every block but the last refills the ring with the next block's weights
    for (int it = 0; it + 1 < nit; it++) block(it, std::integral_constant<bool, true>());
    block(nit - 1, std::integral_constant<bool, false>());
}

// ---------------------------------------------------------------------------
// One- to four-token kernel (k_gemv8): integer MFMA on the raw 4-bit weights,
// activations quantised inside the kernel (no preparation launch).
//
// Activations.  Each wavefront quantises the fp32 activations of its own
// window of C super-blocks once: x_q = rne(x * 2^e), e per (token, wavefront)
// so that max|x| * 2^e lies in [2^13, 2^14) (subnormal windows included), split as x_q = 256*hi + lo with
// hi, lo signed bytes (two int8 planes).  x * 2^e + (1.5*2^23 + 128) puts
// x_q + 128 in the low 16 bits of the fp32 result (round to nearest even):
// byte 1 is hi, byte 0 xor 0x80 is lo, and the float minus the constant is x_q
// itself, so the exact group sums X_g = sum of x_q over each 32-weight group
// come from the same values (a DPP sum over the 8 lanes of a group).
// Non-finite activations in a window make that token's outputs NaN.
//
// LDS record of (super-block, token, plane): the 256 x_q bytes in k order,
// then 32 zero bytes; then the 8 group sums (int32) of each (super-block,
// token).  The records stay for the whole launch.
//
// Products.  v_mfma_i32_16x16x64_i8, B = 16 weight rows; lane (row r = l%16,
// k-block qd = l/16) holds chunk qd of its row (groups 2qd and 2qd+1), and
// one MFMA "piece" (part pt, half hs) takes from it the nibbles hs of bytes
// 16pt..16pt+15: elements 16pt..16pt+15 of group 2qd+hs, as bytes.  A = group
// slots: for the pieces of parity hs, A row i = (token slot i/4, j = i%4) is
// the 16 activation bytes of group 2j + hs of that token in k-block j, zero
// in the other k-blocks (the lane reads the record's zero bytes), so output
// row i collects sum_k q_k x_q over exactly one group of one token, exact in
// int32, and all 16 rows of every MFMA carry a (token, group) pair: four
// token slots cost the same eight MFMAs per super-block as one.  Output
// register v of the parity-hs accumulators of lane l is group 2v + hs of
// token l/16 for row r, so each lane holds all eight groups of its (token,
// row):
//   T_hs = sum over the groups of parity hs of sc_g * (256*S_hi + S_lo),
//   Mt = sum_g m_g * X_g
// in 24-bit integer multiply-adds (|S| < 2^23, |T_hs| < 2^31), then
//   acc += d * T_0 + d * T_1 - dmin * Mt   in fp32,
// the reference's w = (d*sc)*q - dmin*m with all integer parts exact.
//
// Work.  A workgroup of NW wavefronts covers the K/256 super-blocks of 16
// weight rows, wavefront w its window of C (the last window moved back inside
// the row; super-blocks it shares with its neighbour count as padding, zero);
// partial sums are added in wave order through LDS: deterministic.  The
// workgroup walks row blocks blockIdx.x, +gridDim.x, ... and its weight ring
// (one slot per super-block of the window) is refilled with the next block's
// super-block as soon as a slot is consumed, so weight loads stay in flight
// across blocks; the operands of each block's epilogue are loaded before that
// block's refills (a load issued after them would make its wait cover them).
// ---------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int G8_REC = 288;        // x_q bytes of one (super-block, token, plane) + 32 zero bytes
constexpr int G8_XS = 32;          // eight int32 group sums per (super-block, token)
constexpr int G8_MAX_TOKENS = 4;

// Maximum over the wavefront of v >= 0 or NaN (DPP within rows of 16, then
// row broadcasts), read from lane 63.  On such floats the bit patterns
// order as the values do, NaN above Inf, so this is an unsigned integer
// maximum; 0, its identity, stands in the lanes a row broadcast leaves
// unwritten, and every move folds into the v_max_u32 that consumes it.
__device__ __forceinline__ float wave_max_abs_f32(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
#define FH3_DPP_MAX(ctrl, rows) u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, ctrl, rows, 0xF, false));
    FH3_DPP_MAX(0xB1, 0xF)   // quad_perm [1,0,3,2]
    FH3_DPP_MAX(0x4E, 0xF)   // quad_perm [2,3,0,1]
    FH3_DPP_MAX(0x141, 0xF)  // row_half_mirror
    FH3_DPP_MAX(0x140, 0xF)  // row_mirror
    FH3_DPP_MAX(0x142, 0xA)  // row_bcast:15 into rows 1, 3
    FH3_DPP_MAX(0x143, 0xC)  // row_bcast:31 into rows 2, 3
#undef FH3_DPP_MAX
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)u, 63));
}

template <int MT, int C, int LB, int EPI>
__global__ __launch_bounds__(LB) void k_gemv8(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int K,
                                              const float *__restrict__ X, const float *__restrict__ bias,
                                              float *__restrict__ Y, int M, const float *__restrict__ aux, int nblk) {
    constexpr int WAVE_LDS = C * MT * (2 * G8_REC + G8_XS);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    const int NW = blockDim.x >> 6;
    float *red = reinterpret_cast<float *>(lds8 + NW * WAVE_LDS);  // [2][NW][64]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, qd = lane >> 4;
    const int F = N >> 1;
    const int nsb = K >> 8;
    const int own = wave * C;
    const int s0 = own < nsb - C ? own : nsb - C;
    uint8_t *my = lds8 + wave * WAVE_LDS;
    uint8_t *xsb = my + C * MT * 2 * G8_REC;  // group sums [C][MT][8]
    const int nit = (nblk - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    constexpr int ROWS = EPI == EPI_SWIGLU ? 8 : 16;  // output columns per block

    // weight row of this lane in block it: rows o0..o0+15, or (SwiGLU) val
    // rows o0..o0+7 and gate rows F+o0..F+o0+7
    auto wptr = [&](int it) {
        const int o0 = ((int)blockIdx.x + it * (int)gridDim.x) * ROWS;
        int orow = EPI == EPI_SWIGLU ? (r < 8 ? o0 + r : F + o0 + r - 8) : o0 + r;
        orow = orow < N ? orow : N - 1;
        return W + (size_t)orow * row_bytes + (size_t)s0 * 144;
    };

    // activations of the window first: the quantisation waits only for them,
    // not for the weights issued after them (loads complete in order)
    f32x4 xv[MT][C];
#pragma unroll
    for (int t = 0; t < MT; t++)
        if (t < M) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(X + (size_t)t * K + (size_t)s0 * 256) + lane;
#pragma unroll
            for (int i = 0; i < C; i++) xv[t][i] = xr[i * 64];
        }
    u32x4 hv[C], ca[C], cb[C];
    {
        const uint8_t *wh = wptr(0), *wc = wh + 16 + 32 * qd;
#pragma unroll
        for (int s = 0; s < C; s++) {
            hv[s] = ld16(wh + s * 144);
            ca[s] = ld16(wc + s * 144);
            cb[s] = ld16(wc + s * 144 + 16);
        }
    }

    // quantise into the records: lane l holds k = 4l..4l+3 of a super-block
    // (group l/8)
    float inv[MT], inv2[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        inv[t] = 0.f;
        inv2[t] = 1.f;
        if (t < M) {
            // window maximum of |x| with NaN propagated (v_maximum3_f32), so
            // that one value also flags a non-finite window; the wavefront
            // maximum then runs on the bit patterns, which order as the
            // values do on |x| (Inf and NaN above every finite value)
            float mx = 0.f;
#pragma unroll
            for (int i = 0; i < C; i++) {
                const f32x4 v = xv[t][i];
                mx = __builtin_elementwise_maximum(
                    mx, __builtin_elementwise_maximum(
                            __builtin_elementwise_maximum(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                            __builtin_elementwise_maximum(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
            }
            mx = wave_max_abs_f32(mx);
            const bool bad = !(mx <= 3.4028234663852886e38f);
            // 2^e = 2^e1 * 2^e2, both factors normal: e <= 162 for subnormal
            // windows, e >= -114 (largest finite max)
            int e = 0;
            if (mx > 0.f && !bad) {
                int E;
                (void)frexpf(mx, &E);
                e = 14 - E;
            }
            const int e1 = e < 126 ? e : 126, e2 = e - e1;
            const float sc = ldexpf(1.0f, e1), sc2 = ldexpf(1.0f, e2);
            inv[t] = bad ? __builtin_nanf("") : ldexpf(1.0f, -e1);
            inv2[t] = ldexpf(1.0f, -e2);
            // x_q + (1.5*2^23 + 128) = rne(x * 2^e1 * 2^e2 + 1.5*2^23 + 128); x * 2^e1
            // is exact unless it is below 2^-126 in magnitude, where both forms
            // round to the constant itself, so with e2 = 0, the usual case, one
            // fma with 2^e1 gives the same value
            auto quantise = [&](auto two_factors) {
#pragma unroll
                for (int i = 0; i < C; i++) {
                    // scalars, not vector elements: __builtin_bit_cast of an
                    // element expression reads element 0 with this compiler
                    float f0, f1, f2, f3;
                    if constexpr (decltype(two_factors)::value) {
                        const f32x4 v = xv[t][i] * sc;  // exact
                        f0 = __builtin_fmaf(v.x, sc2, 12583040.0f), f1 = __builtin_fmaf(v.y, sc2, 12583040.0f);
                        f2 = __builtin_fmaf(v.z, sc2, 12583040.0f), f3 = __builtin_fmaf(v.w, sc2, 12583040.0f);
                    } else {
                        const f32x4 v = xv[t][i];
                        f0 = __builtin_fmaf(v.x, sc, 12583040.0f), f1 = __builtin_fmaf(v.y, sc, 12583040.0f);
                        f2 = __builtin_fmaf(v.z, sc, 12583040.0f), f3 = __builtin_fmaf(v.w, sc, 12583040.0f);
                    }
                    const uint32_t v0 = __builtin_bit_cast(uint32_t, f0), v1 = __builtin_bit_cast(uint32_t, f1);
                    const uint32_t v2 = __builtin_bit_cast(uint32_t, f2), v3 = __builtin_bit_cast(uint32_t, f3);
                    const uint32_t p01 = __builtin_amdgcn_perm(v1, v0, 0x05040100u);  // v0.b0 v0.b1 v1.b0 v1.b1
                    const uint32_t p23 = __builtin_amdgcn_perm(v3, v2, 0x05040100u);
                    uint8_t *rec = my + (i * MT + t) * 2 * G8_REC + 4 * lane;
                    *reinterpret_cast<uint32_t *>(rec) = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
                    *reinterpret_cast<uint32_t *>(rec + G8_REC) =
                        __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;
                    // f - (1.5*2^23 + 128) = x_q exactly; a group's 32 of them sum
                    // to less than 2^19 in magnitude, exact in fp32
                    const float gs = sum8_f32(((f0 - 12583040.0f) + (f1 - 12583040.0f)) +
                                              ((f2 - 12583040.0f) + (f3 - 12583040.0f)));
                    if ((lane & 7) == 0) reinterpret_cast<int *>(xsb)[(i * MT + t) * 8 + (lane >> 3)] = (int)gs;
                }
            };
            if (e2 == 0)
                quantise(std::false_type{});
            else
                quantise(std::true_type{});
        } else {  // padding token of the tile: zero records (its outputs are not stored)
#pragma unroll
            for (int i = 0; i < C; i++) {
                uint8_t *rec = my + (i * MT + t) * 2 * G8_REC + 4 * lane;
                *reinterpret_cast<uint32_t *>(rec) = 0u;
                *reinterpret_cast<uint32_t *>(rec + G8_REC) = 0u;
                if (lane < 8) reinterpret_cast<int *>(xsb)[(i * MT + t) * 8 + lane] = 0;
            }
        }
    }
    for (int z = lane; z < C * MT * 2 * 2; z += 64)  // the 32 zero bytes after every record
        *reinterpret_cast<u32x4 *>(my + (z >> 1) * G8_REC + 256 + 16 * (z & 1)) = u32x4{0u, 0u, 0u, 0u};
    // the records are read back by lanes of the same wavefront only: LDS
    // operations of a wavefront execute in order
    __builtin_amdgcn_wave_barrier();

    // A operand of lane (row i, k-block qd).  Four token slots (MT == 4):
    // row i = (token slot i/4, j = i%4) holds, for the pieces of parity hs,
    // group 2j + hs of its token when qd == j (that group's chunk is k-block
    // j), so all 16 rows of every MFMA carry a (token, group) pair.  One or two
    // tokens: row i = (token i/8, group g = i%8) holds group g for the pieces
    // with hs == g%2 when qd == g/2 (half the rows of a piece are zero, but
    // each lane then combines only four groups).  Other rows read the
    // record's zero bytes.
    constexpr bool WIDE = MT == 4;
    int aoff[2];
    if constexpr (WIDE) {
        const int a_tok = r >> 2, a_j = r & 3;
#pragma unroll
        for (int hs = 0; hs < 2; hs++)
            aoff[hs] = (qd == a_j && a_tok < MT) ? a_tok * 2 * G8_REC + 32 * (2 * a_j + hs)
                                                 : (a_tok < MT ? a_tok : 0) * 2 * G8_REC + 256;
    } else {
        const int g = r & 7, tt = r >> 3;
        const bool in = qd == (g >> 1) && tt < MT;
#pragma unroll
        for (int hs = 0; hs < 2; hs++)
            aoff[hs] = (in && (g & 1) == hs) ? tt * 2 * G8_REC + 32 * g : (tt < MT ? tt : 0) * 2 * G8_REC + 256;
    }
    // result lane l, weight row r: WIDE, token slot l/16, register v of the
    // parity-hs accumulators is group 2v + hs (all eight groups in the lane);
    // otherwise token l/32, register v is group 4*((l/16)&1) + v, and lanes l
    // and l + 16 hold the two halves
    const int hh = qd & 1;
    const int otok = WIDE ? qd : lane >> 5;
    const int otc = otok < MT ? otok : 0;
    float my_inv = 0.f, my_inv2 = 1.f;
#pragma unroll
    for (int t = 0; t < MT; t++)
        if (otok == t) my_inv = inv[t], my_inv2 = inv2[t];
    // the output (token, column) this thread stores after each block, if any,
    // and the result lane that holds it
    const int st_t = (int)threadIdx.x >> 4, st_rr = (int)threadIdx.x & 15;
    const int st_l = WIDE ? (int)threadIdx.x : 32 * st_t + st_rr;
    const bool storer = (int)threadIdx.x < (WIDE ? 64 : 32) && st_t < M && (EPI != EPI_SWIGLU || st_rr < 8);

    auto block = [&](int it, auto more_tag) {
        constexpr bool MORE = decltype(more_tag)::value;
        const int o0 = ((int)blockIdx.x + it * (int)gridDim.x) * ROWS;
        const int st_o = o0 + st_rr;
        const bool st_ok = storer && st_o < N;
        float e_b = 0.f, e_bg = 0.f, e_aux = 0.f, e_y = 0.f;
        if (st_ok) {
            if (bias) {
                e_b = bias[st_o];
                if (EPI == EPI_SWIGLU) e_bg = bias[F + st_o];
            }
            if (EPI == EPI_GATE_RES) {
                e_aux = aux[(size_t)st_t * N + st_o];
                e_y = Y[(size_t)st_t * N + st_o];
            }
        }
        float acc = 0.f;
        const uint8_t *nh = wptr(MORE ? it + 1 : it), *nc = nh + 16 + 32 * qd;
#pragma unroll
        for (int i = 0; i < C; i++) {
            const u32x4 h = hv[i];
            i32x4 dh[2], dl[2];
#pragma unroll
            for (int hs = 0; hs < 2; hs++) dh[hs] = dl[hs] = i32x4{0, 0, 0, 0};
#pragma unroll
            for (int pc = 0; pc < 4; pc++) {
                const int pt = pc >> 1, hs = pc & 1;
                const u32x4 src = pt ? cb[i] : ca[i];
                const i32x4 b = hs ? i32x4{(int)((src.x >> 4) & 0x0F0F0F0Fu), (int)((src.y >> 4) & 0x0F0F0F0Fu),
                                           (int)((src.z >> 4) & 0x0F0F0F0Fu), (int)((src.w >> 4) & 0x0F0F0F0Fu)}
                                   : i32x4{(int)(src.x & 0x0F0F0F0Fu), (int)(src.y & 0x0F0F0F0Fu),
                                           (int)(src.z & 0x0F0F0F0Fu), (int)(src.w & 0x0F0F0F0Fu)};
                const uint8_t *ap = my + i * MT * 2 * G8_REC + aoff[hs] + 16 * pt;
                const i32x4 ah = *reinterpret_cast<const i32x4 *>(ap);
                const i32x4 al = *reinterpret_cast<const i32x4 *>(ap + G8_REC);
                // one accumulator pair per parity (WIDE), or one for all pieces
                const int ax = WIDE ? hs : 0;
                dh[ax] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, b, dh[ax], 0, 0, 0);
                dl[ax] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, b, dl[ax], 0, 0, 0);
            }
            // 6-bit scales and mins of row r, one per byte: groups 0-3 and 4-7
            // (reference src/core/fh3_quant.c:168-177)
            const uint32_t sc_a = h.y & 0x3F3F3F3Fu, sc_b = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
            const uint32_t m_a = h.z & 0x3F3F3F3Fu, m_b = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
            const bool valid = s0 + i >= own;
            const float d = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xFFFFu)) : 0.f;
            const float dmin = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16)) : 0.f;
            const i32x4 *xs = reinterpret_cast<const i32x4 *>(xsb + (i * MT + otc) * G8_XS);
            // four groups per sum: |T| <= 4 * 63 * 32 * 15 * 2^14 < 2^31
            int T[2] = {0, 0}, Mt = 0;
            if constexpr (WIDE) {
                const i32x4 xa = xs[0], xb = xs[1];
#pragma unroll
                for (int hs = 0; hs < 2; hs++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int gg = 2 * v + hs;
                        const uint32_t scw = gg < 4 ? sc_a : sc_b;
                        const int S = (dh[hs][v] << 8) + dl[hs][v];
                        T[hs] += __mul24((int)((scw >> (8 * (gg & 3))) & 0xFFu), S);
                    }
#pragma unroll
                for (int gg = 0; gg < 8; gg++) {
                    const uint32_t mw = gg < 4 ? m_a : m_b;
                    Mt += __mul24((int)((mw >> (8 * (gg & 3))) & 0xFFu), gg < 4 ? xa[gg] : xb[gg - 4]);
                }
            } else {
                const uint32_t scw = hh ? sc_b : sc_a, mw = hh ? m_b : m_a;
                const i32x4 xv4 = xs[hh];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int S = (dh[0][v] << 8) + dl[0][v];
                    T[0] += __mul24((int)((scw >> (8 * v)) & 0xFFu), S);
                    Mt += __mul24((int)((mw >> (8 * v)) & 0xFFu), xv4[v]);
                }
            }
            acc = __builtin_fmaf(d, (float)T[1], __builtin_fmaf(d, (float)T[0], __builtin_fmaf(-dmin, (float)Mt, acc)));
            if (MORE) {
                hv[i] = ld16(nh + i * 144);
                ca[i] = ld16(nc + i * 144);
                cb[i] = ld16(nc + i * 144 + 16);
            }
        }
        if constexpr (!WIDE) acc += __shfl_down(acc, 16);  // the other four groups
        float *rb = red + (it & 1) * NW * 64;  // alternate buffers: one barrier per block
        rb[wave * 64 + lane] = (acc * my_inv) * my_inv2;
        __syncthreads();
        if (st_ok) {
            float sum = 0.f;
            for (int w = 0; w < NW; w++) sum += rb[w * 64 + st_l];
            if (EPI == EPI_SWIGLU) {  // the gate of column st_rr is row st_rr + 8 of the block
                float sg = 0.f;
                for (int w = 0; w < NW; w++) sg += rb[w * 64 + st_l + 8];
                Y[(size_t)st_t * F + st_o] = (sum + e_b) * silu_f32(sg + e_bg);
            } else if (EPI == EPI_GATE_RES) {
                Y[(size_t)st_t * N + st_o] = __builtin_fmaf(e_aux, sum + e_b, e_y);
            } else {
                Y[(size_t)st_t * N + st_o] = sum + e_b;
            }
        }
    };
    // every block but the last refills the ring with the next block's weights
    for (int it = 0; it + 1 < nit; it++) block(it, std::integral_constant<bool, true>());
    block(nit - 1, std::integral_constant<bool, false>());
}

// ---------------------------------------------------------------------------
// Large-M kernel.  Output tile 256 tokens x 128 weight rows, 4 wavefronts, each
// owning 64 tokens x all 128 rows (2 x 4 tiles of 32x32, 128 fp32 accumulators
// per lane).  Per K step s of 64 (one Q4_K chunk: groups 2c and 2c+1):
//   - thread (r = tid/2, h = tid%2) holds 16 raw bytes of row r's chunk
//     and writes 32 dequantised fp16 weights into the LDS B-fragments;
//   - each wavefront loads its X16 fragments straight from global memory
//     (1 KiB contiguous per load);
//   - software pipelined: in the interval between two barriers the MFMAs of
//     step s read lds[s&1] while step s+1 is dequantised into lds[(s+1)&1],
//     so the dequant VALU work overlaps the matrix work; the loop is unrolled
//     by two so that activation and raw-weight registers ping-pong.
// Workgroup ids are remapped so that the 8 XCDs each run a contiguous run of
// tiles in token-major order: concurrent tiles on one XCD share the same 256
// activation rows in that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int GEMM_BM = 256;
constexpr int GEMM_BN = 128;

// Raw bytes one thread needs for K step s (chunk c = s%4 of a super-block),
// per weight type; what does not change within a super-block (or, for Q6_K,
// within one of its halves) is loaded once and carried from step to step.
//   Q4_K (144 B): the 16-byte header and 16 bytes of chunk c.
//   Q5_K (176 B, src/core/fh3_quant.c:198-237): the same header, qh bytes
//     16h..16h+15 (the high bits of this thread's element positions, one bit
//     per group) and 16 bytes of chunk c of the low nibbles at 48.
//   Q6_K (210 B, src/core/fh3_quant.c:239-282): 16 ql bytes of chunk c (see
//     gemm_dequant), the 16 qh bytes of the chunk's half, that half's eight
//     int8 scales and d.
template <int QT> struct GemmRaw { u32x4 hv, qv; };
template <> struct GemmRaw<FH3K_Q5_K> { u32x4 hv, hb, qv; };
template <> struct GemmRaw<FH3K_Q6_K> { u32x4 hb, qv; u32x2 sc; uint32_t d; };

// CH (the chunk, s % 4) is a compile-time constant, so the header load of
// chunk 0 is not a branch and a K step is one basic block.
// k_gemm reads through buffer resources: wr covers the workgroup's weight
// rows from its first one, woff is the byte offset of this thread's row and
// woffq that offset plus the thread's 16-byte piece of a chunk; the super-block
// offset goes in the scalar offset.  No per-lane address arithmetic per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Q6_K super-blocks are only 2-byte aligned, so its pieces are read with
// unaligned global loads (as k_skinny reads them) from wbase, the workgroup's
// first weight row, plus the super-block offset (uniform) plus the thread's
// 32-bit offset; every byte read lies inside the super-block.
typedef uint32_t u32x2u __attribute__((ext_vector_type(2), aligned(2)));
template <int QT, int CH>
__device__ __forceinline__ void gemm_load_raw(__amdgpu_buffer_rsrc_t wr, const uint8_t *wbase, uint32_t woff,
                                              uint32_t woffq, int sb, GemmRaw<QT> &r, const GemmRaw<QT> &prev) {
    if constexpr (QT == FH3K_Q6_K) {
        // woffq = woff + 16h: ql bytes 64(c/2) + 32(c%2) + 16h, qh bytes
        // 128 + 32(c/2) + 16h, scales 192 + 8(c/2)
        const uint8_t *b = wbase + (size_t)sb * 210;
        r.qv = ld16u(b + woffq + (64 * (CH >> 1) + 32 * (CH & 1)));
        if constexpr ((CH & 1) == 0) {
            r.hb = ld16u(b + woffq + (128 + 32 * (CH >> 1)));
            r.sc = *reinterpret_cast<const u32x2u *>(b + woff + (192 + 8 * (CH >> 1)));
        } else {
            r.hb = prev.hb;
            r.sc = prev.sc;
        }
        r.d = CH == 0 ? ld_u16(b + woff + 208) : prev.d;
    } else {
        const int so = sb * (QT == FH3K_Q5_K ? 176 : 144);
        r.hv = CH == 0 ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)woff, so, 0))
                       : prev.hv;
        r.qv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)woffq + 32 * CH, so, 0));
        if constexpr (QT == FH3K_Q5_K)  // qh bytes 16 + 16h = woffq - 32
            r.hb = CH == 0 ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)woffq - 32, so,
                                                                                              0))
                           : prev.hb;
    }
}

// B-fragment layout: fragment rb*4 + kk holds rows 32rb..32rb+31 x k 16kk..16kk+15
// of the step; lane l holds row l%32 at k offset 8*(l/32).
// Group scale of group 4*upper + j (upper uniform, j in 0..3 may differ per
// lane): the same D and C as q4k_group_fast.
__device__ __forceinline__ void q4k_group_j(const u32x4 hdr, bool upper, int j, float &D, float &C) {
    const int sh = 8 * j;
    uint32_t sc, mn;
    if (!upper) {
        sc = (hdr.y >> sh) & 63u;
        mn = (hdr.z >> sh) & 63u;
    } else {
        sc = ((hdr.w >> sh) & 15u) | (((hdr.y >> (sh + 6)) & 3u) << 4);
        mn = ((hdr.w >> (sh + 4)) & 15u) | (((hdr.z >> (sh + 6)) & 3u) << 4);
    }
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
    D = d * (float)sc;
    C = -(dmin * (float)mn + 1024.0f * D);
}

// Eight fp16 fma(D, 1024 + v, C) from eight byte values v (a = bytes 0-3, b =
// bytes 4-7), each rounded once.
__device__ __forceinline__ half8 deq8_bytes(uint32_t a, uint32_t b, float D, float C) {
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
    const u32x4 q = {fma_mix_pair(D, p0, C), fma_mix_pair(D, p1, C), fma_mix_pair(D, p2, C), fma_mix_pair(D, p3, C)};
    return __builtin_bit_cast(half8, q);
}

// q4k_deq8_f16 with the nibble half as a shift (0 low, 4 high) that may
// differ per lane.
__device__ __forceinline__ half8 q4k_deq8_sh(uint32_t u0, uint32_t u1, int sh, float D, float C) {
    const uint32_t a = (u0 >> sh) & 0x0F0F0F0Fu;
    const uint32_t b = (u1 >> sh) & 0x0F0F0F0Fu;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
    const u32x4 q = {fma_mix_pair(D, p0, C), fma_mix_pair(D, p1, C), fma_mix_pair(D, p2, C), fma_mix_pair(D, p3, C)};
    return __builtin_bit_cast(half8, q);
}

// Value of the neighbouring lane (lane ^ 1), one DPP move (quad_perm 1,0,3,2).
__device__ __forceinline__ float lane_swap1(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
}

// Chunk c of a super-block: 32 quant bytes per row, low nibbles group 2c,
// high nibbles group 2c + 1.  The two threads of a row are adjacent lanes
// (h = lane & 1) holding 16 bytes each; each decodes the scale of group
// 2c + h only and takes the other group's (D, C) from its neighbour, then
// writes its own nibble half first: low nibbles to fragment wf + h, high
// nibbles to wf + 2 + h.
// Q5_K: the same with bit g of each qh byte (h0, h1: the qh bytes of the same
// element positions) as bit 4 of q, q <= 31.
__device__ __forceinline__ half8 q5k_deq8_sh(uint32_t u0, uint32_t u1, uint32_t h0, uint32_t h1, int sh, int g,
                                             float D, float C) {
    return deq8_bytes(((u0 >> sh) & 0x0F0F0F0Fu) | (((h0 >> g) & 0x01010101u) << 4),
                      ((u1 >> sh) & 0x0F0F0F0Fu) | (((h1 >> g) & 0x01010101u) << 4), D, C);
}

// Q6_K: q = nibble (shift SH) | bits HS..HS+1 of the qh byte << 4, weight
// D * (q - 32) with D = d * sc.  fma(D, 1024 + q, -1056 D) is that value
// exactly in fp32 (D = fp16 * int8 has at most 18 significant bits, 1056 D and
// D * (q - 32) at most 24), so each weight is the reference's fp32 value
// rounded once to fp16.
template <int SH, int HS>
__device__ __forceinline__ half8 q6k_deq8(uint32_t u0, uint32_t u1, uint32_t h0, uint32_t h1, float D) {
    auto hi2 = [](uint32_t h) { return (HS >= 4 ? h >> (HS - 4) : h << (4 - HS)) & 0x30303030u; };
    return deq8_bytes(((u0 >> SH) & 0x0F0F0F0Fu) | hi2(h0), ((u1 >> SH) & 0x0F0F0F0Fu) | hi2(h1), D, -1056.0f * D);
}

template <int QT, int CH>
__device__ __forceinline__ void gemm_dequant(half8 (*ldsb)[64], const GemmRaw<QT> &r, int wf, int wl, int h) {
    constexpr int c = CH;
    if constexpr (QT == FH3K_Q6_K) {
        // chunk c = (half c/2, quarter c%2) holds ql bytes 64(c/2) + 32(c%2) +
        // b, b = 0..31: low nibble = element 128(c/2) + 32(c%2) + b (k step
        // offset b), high nibble = element 128(c/2) + 64 + 32(c%2) + b (offset
        // 32 + b); their 2 high bits are bits 2(c%2) and 4 + 2(c%2) of qh
        // byte 32(c/2) + b and their scales sub-groups 8(c/2) + 2(c%2) + b/16
        // and that + 4.  This thread has b = 16h..16h+15: low nibbles to
        // fragment wf + h, high nibbles to wf + 2 + h.
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.d & 0xFFFFu));
        const int sb8 = 8 * (2 * (c & 1) + h);
        const float Dl = d * (float)(int)(int8_t)(uint8_t)(r.sc.x >> sb8);
        const float Dh = d * (float)(int)(int8_t)(uint8_t)(r.sc.y >> sb8);
        constexpr int hs = 2 * (c & 1);
        ldsb[wf + h][wl] = q6k_deq8<0, hs>(r.qv.x, r.qv.y, r.hb.x, r.hb.y, Dl);
        ldsb[wf + h][wl + 32] = q6k_deq8<0, hs>(r.qv.z, r.qv.w, r.hb.z, r.hb.w, Dl);
        ldsb[wf + 2 + h][wl] = q6k_deq8<4, hs + 4>(r.qv.x, r.qv.y, r.hb.x, r.hb.y, Dh);
        ldsb[wf + 2 + h][wl + 32] = q6k_deq8<4, hs + 4>(r.qv.z, r.qv.w, r.hb.z, r.hb.w, Dh);
    } else {
        float Dm, Cm;
        q4k_group_j(r.hv, c >= 2, ((2 * c) & 3) + h, Dm, Cm);
        const float Do = lane_swap1(Dm), Co = lane_swap1(Cm);
        const int own = wf + 3 * h, oth = wf + 2 - h;
        const int sho = 4 * h, sht = 4 - 4 * h;
        if constexpr (QT == FH3K_Q5_K) {
            // the high bit of group 2c + h (own) / 2c + 1 - h (other)
            const int go = 2 * c + h, gt = 2 * c + 1 - h;
            ldsb[own][wl] = q5k_deq8_sh(r.qv.x, r.qv.y, r.hb.x, r.hb.y, sho, go, Dm, Cm);
            ldsb[own][wl + 32] = q5k_deq8_sh(r.qv.z, r.qv.w, r.hb.z, r.hb.w, sho, go, Dm, Cm);
            ldsb[oth][wl] = q5k_deq8_sh(r.qv.x, r.qv.y, r.hb.x, r.hb.y, sht, gt, Do, Co);
            ldsb[oth][wl + 32] = q5k_deq8_sh(r.qv.z, r.qv.w, r.hb.z, r.hb.w, sht, gt, Do, Co);
        } else {
            ldsb[own][wl] = q4k_deq8_sh(r.qv.x, r.qv.y, sho, Dm, Cm);
            ldsb[own][wl + 32] = q4k_deq8_sh(r.qv.z, r.qv.w, sho, Dm, Cm);
            ldsb[oth][wl] = q4k_deq8_sh(r.qv.x, r.qv.y, sht, Do, Co);
            ldsb[oth][wl + 32] = q4k_deq8_sh(r.qv.z, r.qv.w, sht, Do, Co);
        }
    }
}

// Activation fragments of K step s for k_gemm: xr covers the wavefront's two
// token blocks, xoff is the lane's byte offset, tbs the byte stride of a token
// block.
// The step's fragment k is X16 fragment 4s + k (Q4_K, Q5_K: the step is 64
// consecutive k), or for Q6_K (see gemm_dequant) 16(s/4) + 8(c/2) + 2(c%2) +
// k%2 + 4(k/2), c = s%4.
template <int TBW, int QT = FH3K_Q4_K>
__device__ __forceinline__ void gemm_load_xs(__amdgpu_buffer_rsrc_t xr, uint32_t xoff, int tbs, int s,
                                             half8 (&xf)[TBW][4]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int f = QT == FH3K_Q6_K ? 16 * (s >> 2) + 8 * ((s >> 1) & 1) + 2 * (s & 1) + (k & 1) + 4 * (k >> 1)
                                      : s * 4 + k;
        const int so = f * 1024;
#pragma unroll
        for (int a = 0; a < TBW; a++)
            xf[a][k] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)xoff, so + a * tbs, 0));
    }
}

__device__ __forceinline__ void gemm_load_x(const half8 *xa0, const half8 *xa1, int s, half8 (&xf)[2][4]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xf[0][k] = xa0[(size_t)(s * 4 + k) * 64];
        xf[1][k] = xa1[(size_t)(s * 4 + k) * 64];
    }
}

template <int TBW>
__device__ __forceinline__ void gemm_mfma(half8 (*ldsb)[64], int lane, const half8 (&xf)[TBW][4],
                                          f32x16 (&acc)[TBW][4]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        half8 bfr[4];
#pragma unroll
        for (int ob = 0; ob < 4; ob++) bfr[ob] = ldsb[ob * 4 + k][lane];
#pragma unroll
        for (int ob = 0; ob < 4; ob++)
#pragma unroll
            for (int a = 0; a < TBW; a++)
                acc[a][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xf[a][k], bfr[ob], acc[a][ob], 0, 0, 0);
    }
}

// Within a K step the wavefront runs at raised priority (s_setprio 2) from its
// first MFMA to the barrier, so that of the two wavefronts on a SIMD the one
// with matrix work issues first (measured +1.7 % on the DiT shapes).
// Instruction order of one K step, given to the scheduler: the 32 MFMAs each
// followed by up to four VALU (the next step's dequant), the B-fragment reads
// of k-slice k+1 spread over the MFMAs of slice k, the next step's loads one
// per three MFMAs and the LDS writes after MFMA 20 (the best of a sweep of
// these counts on the DiT shapes).  Without it the compiler clusters the
// loads and the dequant into runs that stall the matrix pipe.
// With one token block per wavefront (TBW = 1: 16 MFMAs and 6 loads per step)
// the same pattern is compressed: eight VALU per MFMA, the 12 remaining
// B-fragment reads on three of every four MFMAs, a load every third MFMA and
// the LDS writes after MFMA 10.
template <int TBW, int I>
__device__ __forceinline__ void gemm_pipe_slot() {
    constexpr int NM = 16 * TBW;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 128 / NM, 0);        // VALU
    if constexpr (TBW == 2 ? (I % 2 == 1 && I < 24) : (I % 4 != 0))  // DS read
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if constexpr (I % 3 == 0 && I < 3 * (2 + 4 * TBW)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    if constexpr (I >= 10 * TBW && I < 10 * TBW + 4) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
    if constexpr (I + 1 < NM) gemm_pipe_slot<TBW, I + 1>();
}

template <int TBW>
__device__ __forceinline__ void gemm_pipe() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // B fragments of the first k-slice
    gemm_pipe_slot<TBW, 0>();
}

// TBW: 32-token blocks per wavefront; the workgroup's tile is 128 * TBW tokens
// x 128 weight rows (TBW = 1 for at most 128 tokens: half the matrix work of
// the 256-token tile per K step, whose lower half such products leave empty).
// QT: the weight type, Q4_K, or Q5_K / Q6_K read in place (GemmRaw,
// gemm_dequant); the tile, pipeline and epilogue are the same.
template <int TBW, int QT = FH3K_Q4_K>
__global__ __launch_bounds__(256, 2) void k_gemm(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                 int N, int K, const half8 *__restrict__ X16,
                                                 const float *__restrict__ xs_inv,
                                                 const float *__restrict__ bias,
                                                 float *__restrict__ Y, int M, int m_tiles,
                                                 int n_tiles, int epi, const float *__restrict__ aux, int C,
                                                 float *__restrict__ part) {
    __shared__ half8 lds[2][16][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // grid = tiles x S windows of C super-blocks (S = 1: the whole of K)
    const int tiles = m_tiles * n_tiles;
    const int total = gridDim.x;
    const int id = blockIdx.x;
    const int per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int ks = L / tiles, tl = L - ks * tiles;
    const int mt = tl / n_tiles, nt = tl - mt * n_tiles;
    constexpr int BM = 128 * TBW;
    const int m0 = mt * BM, n0 = nt * GEMM_BN;

    // weight-loader role: rows n0..n0+127, or (SwiGLU) 64 val rows from
    // nt*64 and the 64 gate rows F + nt*64..  Offsets from the first row fit
    // 32 bits (the launcher requires N * row_bytes < 2^32).
    // two adjacent lanes per weight row (h = which 16 of a chunk's 32 bytes)
    const int r = tid >> 1, h = tid & 1;
    const int F = N >> 1;
    const int rowbase = epi == EPI_SWIGLU ? nt * 64 : n0;
    int orow = n0 + r;
    if (epi == EPI_SWIGLU) orow = r < 64 ? nt * 64 + r : F + nt * 64 + r - 64;
    orow = orow < N ? orow : N - 1;
    const __amdgpu_buffer_rsrc_t wr =
        buf_rsrc(W + (size_t)rowbase * row_bytes, (uint32_t)((size_t)(N - rowbase) * row_bytes));
    const uint32_t woff = (uint32_t)(orow - rowbase) * (uint32_t)row_bytes;
    const uint32_t woffq = woff + (QT == FH3K_Q5_K ? 48u : (QT == FH3K_Q6_K ? 0u : 16u)) + 16u * (uint32_t)h;
    const uint8_t *wbase = W + (size_t)rowbase * row_bytes;
    const int wf = (r >> 5) * 4;   // first LDS fragment of this row's 32-row block
    const int wl = r & 31;

    // activation fragments of this wavefront: token blocks T0 .. T0+TBW-1
    const int kf_n = K / 16;
    const int tbs = kf_n * 1024;
    const __amdgpu_buffer_rsrc_t xr =
        buf_rsrc(X16 + ((size_t)(m0 / 32 + TBW * wave) * kf_n) * 64, (uint32_t)TBW * (uint32_t)tbs);
    const uint32_t xoff = (uint32_t)lane * 16u;

    // super-blocks [sb0, sb1) of K: all of them, or this workgroup's window
    const int nsb = K / 256;
    const int sb0 = ks * C;
    const int sb1 = sb0 + C < nsb ? sb0 + C : nsb;
    f32x16 acc[TBW][4];
#pragma unroll
    for (int a = 0; a < TBW; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    GemmRaw<QT> re, ro;              // raw weights of even / odd steps
    half8 xe[TBW][4], xo[TBW][4];  // activations of even / odd steps
    gemm_load_raw<QT, 0>(wr, wbase, woff, woffq, sb0, re, re);
    gemm_load_xs<TBW, QT>(xr, xoff, tbs, 4 * sb0, xe);
    gemm_load_raw<QT, 1>(wr, wbase, woff, woffq, sb0, ro, re);
    gemm_dequant<QT, 0>(lds[0], re, wf, wl, h);
    __syncthreads();
    // one super-block (4 K steps) per iteration; the loads and the dequant of
    // the step after the last are clamped onto the last super-block (valid
    // addresses, results unused), so no step has a branch and the scheduler
    // can interleave each step's loads and dequant with its MFMAs
    for (int sb = sb0; sb < sb1; sb++) {
        const int s = 4 * sb;
        const int nb = sb + 1 < sb1 ? sb + 1 : sb;
        // step s (chunk 0): MFMA from lds[0]; dequant chunk 1 into lds[1]
        gemm_load_xs<TBW, QT>(xr, xoff, tbs, s + 1, xo);
        gemm_load_raw<QT, 2>(wr, wbase, woff, woffq, sb, re, ro);
        gemm_dequant<QT, 1>(lds[1], ro, wf, wl, h);
        __builtin_amdgcn_s_setprio(2);
        gemm_mfma(lds[0], lane, xe, acc);
        gemm_pipe<TBW>();
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // step s+1 (chunk 1): MFMA from lds[1]; dequant chunk 2 into lds[0]
        gemm_load_xs<TBW, QT>(xr, xoff, tbs, s + 2, xe);
        gemm_load_raw<QT, 3>(wr, wbase, woff, woffq, sb, ro, re);
        gemm_dequant<QT, 2>(lds[0], re, wf, wl, h);
        __builtin_amdgcn_s_setprio(2);
        gemm_mfma(lds[1], lane, xo, acc);
        gemm_pipe<TBW>();
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // step s+2 (chunk 2): MFMA from lds[0]; dequant chunk 3 into lds[1]
        gemm_load_xs<TBW, QT>(xr, xoff, tbs, s + 3, xo);
        gemm_load_raw<QT, 0>(wr, wbase, woff, woffq, nb, re, ro);
        gemm_dequant<QT, 3>(lds[1], ro, wf, wl, h);
        __builtin_amdgcn_s_setprio(2);
        gemm_mfma(lds[0], lane, xe, acc);
        gemm_pipe<TBW>();
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // step s+3 (chunk 3): MFMA from lds[1]; dequant the next chunk 0 into lds[0]
        gemm_load_xs<TBW, QT>(xr, xoff, tbs, 4 * nb, xe);
        gemm_load_raw<QT, 1>(wr, wbase, woff, woffq, nb, ro, re);
        gemm_dequant<QT, 0>(lds[0], re, wf, wl, h);
        __builtin_amdgcn_s_setprio(2);
        gemm_mfma(lds[1], lane, xo, acc);
        gemm_pipe<TBW>();
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
    }

    // epilogue: 32x32 output D, lane l holds column l%32 (weight row) and rows
    // 8*(v/4) + 4*(l/32) + v%4 (tokens).
    // Fast path: a 32x32 block whose rows and 32 columns are all inside the
    // output (row stride a multiple of 4 floats) goes through this wavefront's
    // 4 KiB of LDS (free after the loop's last barrier) and leaves as 16-byte
    // row pieces: 4 vector stores per lane instead of 16 scalar ones (the
    // scalar stores cost ~7 % of the kernel on the DiT shapes).  Values and
    // rounding are the same either way.
    float *stg = reinterpret_cast<float *>(&lds[0][0][0]) + wave * 1024;
    // dst points at the block's top-left element, ld is the row stride;
    // mode 0 store, 1 gate residual (dst += g * y, g at the same offsets in aux)
    auto block_store = [&](const float (&val)[16], float *dst, const float *g, size_t ld, int mode) {
#pragma unroll
        for (int v = 0; v < 16; v++) stg[(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * 32 + (lane & 31)] = val[v];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = (lane >> 3) + 8 * i, c = 4 * (lane & 7);
            const f32x4 y = *reinterpret_cast<const f32x4 *>(stg + r * 32 + c);
            f32x4 *d = reinterpret_cast<f32x4 *>(dst + (size_t)r * ld + c);
            if (mode == 1) {
                const f32x4 gg = *reinterpret_cast<const f32x4 *>(g + (size_t)r * ld + c);
                const f32x4 h = *d;
                *d = f32x4{__builtin_fmaf(gg.x, y.x, h.x), __builtin_fmaf(gg.y, y.y, h.y), __builtin_fmaf(gg.z, y.z, h.z),
                           __builtin_fmaf(gg.w, y.w, h.w)};
            } else {
                *d = y;
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    const int wt0 = m0 + 32 * TBW * wave;  // this wavefront's first token
    const bool rows_in = wt0 + 32 * TBW <= M;
    // 16-byte stores and gate reads need 16-byte aligned Y and aux (the
    // entry points accept any float pointer for them; part is the library's)
    const bool out16 = ((reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(aux)) & 15) == 0;
    if (part) {
        // split K: this window's raw sums, part[ks][t][row] over all N rows
        const bool vec = rows_in && (N & 3) == 0 &&
                         (epi == EPI_SWIGLU ? nt * 64 + 64 <= F : n0 + 128 <= N);
        if (vec) {
#pragma unroll
            for (int tb = 0; tb < TBW; tb++) {
                const int tb0 = wt0 + 32 * tb;
#pragma unroll
                for (int ob = 0; ob < 4; ob++) {
                    const int c0 = epi == EPI_SWIGLU ? (ob < 2 ? nt * 64 + 32 * ob : F + nt * 64 + 32 * (ob - 2))
                                                     : n0 + 32 * ob;
                    float vals[16];
#pragma unroll
                    for (int v = 0; v < 16; v++) vals[v] = acc[tb][ob][v];
                    block_store(vals, part + ((size_t)ks * M + tb0) * N + c0, nullptr, (size_t)N, 0);
                }
            }
            return;
        }
#pragma unroll
        for (int tb = 0; tb < TBW; tb++) {
            const int tbase = wt0 + 32 * tb + 4 * (lane >> 5);
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                int o = n0 + 32 * ob + (lane & 31);
                if (epi == EPI_SWIGLU) o = ob < 2 ? nt * 64 + 32 * ob + (lane & 31) : F + nt * 64 + 32 * (ob - 2) + (lane & 31);
                if (o >= N) continue;
                float *pp = part + (size_t)ks * M * N + o;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int t = tbase + 8 * (v >> 2) + (v & 3);
                    if (t < M) pp[(size_t)t * N] = acc[tb][ob][v];
                }
            }
        }
        return;
    }
    if (epi == EPI_SWIGLU) {
        // tiles ob = 0, 1 hold val rows nt*64 + 32*ob + l%32, tiles 2, 3 the
        // matching gate rows
        if (rows_in && out16 && (F & 3) == 0 && nt * 64 + 64 <= F) {
#pragma unroll
            for (int tb = 0; tb < TBW; tb++) {
                const int tb0 = wt0 + 32 * tb;
#pragma unroll
                for (int ob = 0; ob < 2; ob++) {
                    const int o = nt * 64 + 32 * ob + (lane & 31);
                    const float bv = bias ? bias[o] : 0.f, bg = bias ? bias[F + o] : 0.f;
                    float vals[16];
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int t = tb0 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                        vals[v] = (acc[tb][ob][v] * xs_inv[t] + bv) * silu_f32(acc[tb][ob + 2][v] * xs_inv[t] + bg);
                    }
                    block_store(vals, Y + (size_t)tb0 * F + nt * 64 + 32 * ob, nullptr, (size_t)F, 0);
                }
            }
            return;
        }
#pragma unroll
        for (int tb = 0; tb < TBW; tb++) {
            const int tbase = wt0 + 32 * tb + 4 * (lane >> 5);
#pragma unroll
            for (int ob = 0; ob < 2; ob++) {
                const int o = nt * 64 + 32 * ob + (lane & 31);
                const float bv = bias ? bias[o] : 0.f, bg = bias ? bias[F + o] : 0.f;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int t = tbase + 8 * (v >> 2) + (v & 3);
                    if (t < M)
                        Y[(size_t)t * F + o] = (acc[tb][ob][v] * xs_inv[t] + bv) *
                                               silu_f32(acc[tb][ob + 2][v] * xs_inv[t] + bg);
                }
            }
        }
        return;
    }
    if (rows_in && out16 && (N & 3) == 0 && n0 + 128 <= N) {
#pragma unroll
        for (int tb = 0; tb < TBW; tb++) {
            const int tb0 = wt0 + 32 * tb;
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                const int o = n0 + 32 * ob + (lane & 31);
                const float bo = bias ? bias[o] : 0.f;
                float vals[16];
#pragma unroll
                for (int v = 0; v < 16; v++)
                    vals[v] = acc[tb][ob][v] * xs_inv[tb0 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)] + bo;
                const size_t off = (size_t)tb0 * N + n0 + 32 * ob;
                block_store(vals, Y + off, epi == EPI_GATE_RES ? aux + off : nullptr, (size_t)N,
                            epi == EPI_GATE_RES ? 1 : 0);
            }
        }
        return;
    }
#pragma unroll
    for (int tb = 0; tb < TBW; tb++) {
        const int tbase = wt0 + 32 * tb + 4 * (lane >> 5);
#pragma unroll
        for (int ob = 0; ob < 4; ob++) {
            const int o = n0 + 32 * ob + (lane & 31);
            if (o >= N) continue;
            const float bo = bias ? bias[o] : 0.f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int t = tbase + 8 * (v >> 2) + (v & 3);
                if (t < M) epi_store(Y, aux, epi, (size_t)t * N + o, acc[tb][ob][v] * xs_inv[t] + bo);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Weights of the other types (the reference's fh3_matmul takes every type its
// fh3_dequant decodes, src/core/fh3_ops.c:325-333).  They are decoded once per
// call to fp16 rows W16[N][K] -- the reference's fp32 value rounded once to
// fp16, as k_gemm rounds Q4_K -- and multiplied by k_skinny16 / k_gemm16, which
// read those rows directly.  F16 weights are used as they are.
// ---------------------------------------------------------------------------
// Output rows hold nblk_out >= nblk blocks; blocks nblk.. of a row (the
// padding up to a whole number of 256-column steps) are written as zeros.
template <int T>
__global__ __launch_bounds__(256) void k_weights_f16_blocks(const uint8_t *__restrict__ src, int64_t row_bytes,
                                                            int64_t nblk, int64_t nblk_out, int64_t rows,
                                                            _Float16 *__restrict__ dst) {
    constexpr int BL = Fmt<T>::BL, BB = Fmt<T>::BB, P = Fmt<T>::P;
    const int64_t per_row = nblk_out * P;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * per_row) return;
    const int64_t row = gid / per_row;
    const int64_t rem = gid - row * per_row;
    const int64_t b = rem / P;
    const int G = (int)(rem - b * P);
    float o[16];
    if (b < nblk) {
        deq_piece<T>(src + row * row_bytes + b * BB, G, o);
    } else {
#pragma unroll
        for (int e = 0; e < 16; e++) o[e] = 0.f;
    }
    half8 *out = reinterpret_cast<half8 *>(dst + row * nblk_out * BL + b * BL + 16 * G);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = (_Float16)o[8 * j + e];
        out[j] = h;
    }
}

// F32 / F16 / BF16 rows of any length K (rows row_bytes apart, element
// aligned) -> fp16 rows of Kp >= K columns (Kp % 8 == 0), zeros at k >= K;
// 8 outputs per thread.  F16 values are copied bit for bit, the others rounded
// once to fp16 as k_weights_f16_elem rounds them.
template <int T>
__global__ __launch_bounds__(256) void k_weights_f16_any(const uint8_t *__restrict__ src, int64_t row_bytes, int K,
                                                         int Kp, int64_t rows, _Float16 *__restrict__ dst) {
    const int64_t per_row = Kp / 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * per_row) return;
    const int64_t row = gid / per_row;
    const int k0 = (int)(gid - row * per_row) * 8;
    const uint8_t *s = src + row * row_bytes;
    uint32_t bits[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int k = k0 + e;
        uint32_t b = 0;
        if (k < K) {
            if constexpr (T == FH3K_F16) {
                b = reinterpret_cast<const uint16_t *>(s)[k];
            } else if constexpr (T == FH3K_BF16) {
                const float f = __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t *>(s)[k] << 16);
                b = __builtin_bit_cast(uint16_t, (_Float16)f);
            } else {
                b = __builtin_bit_cast(uint16_t, (_Float16)reinterpret_cast<const float *>(s)[k]);
            }
        }
        bits[e] = b;
    }
    const u32x4 v = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16), bits[4] | (bits[5] << 16),
                     bits[6] | (bits[7] << 16)};
    *reinterpret_cast<u32x4 *>(dst + row * Kp + k0) = v;
}

// F32 / BF16 rows -> fp16, 8 elements per thread (n % 8 == 0).
template <bool BF>
__global__ __launch_bounds__(256) void k_weights_f16_elem(const uint8_t *__restrict__ src, int64_t n8,
                                                          _Float16 *__restrict__ dst) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n8) return;
    half8 h;
    if (BF) {
        const u32x4 v = reinterpret_cast<const u32x4 *>(src)[gid];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[2 * e] = (_Float16)__builtin_bit_cast(float, v[e] << 16);
            h[2 * e + 1] = (_Float16)__builtin_bit_cast(float, v[e] & 0xFFFF0000u);
        }
    } else {
        const f32x4 *s = reinterpret_cast<const f32x4 *>(src) + 2 * gid;
        const f32x4 a = s[0], c = s[1];
        h = half8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                  (_Float16)c.x, (_Float16)c.y, (_Float16)c.z, (_Float16)c.w};
    }
    reinterpret_cast<half8 *>(dst)[gid] = h;
}

// Small M on fp16 rows: the k_skinny work split (NW wavefronts x C windows of
// 256 k over 16 rows, last window moved inside the row, padding windows
// skipped), B = 8 fp16 weights of row l%16 at k offset 8*(l/16) of a 32-k
// window, loaded straight from W16; A = the same k of the X16 fragments.
// Deterministic: wave partials added in order through LDS.
template <int TB, int C>
__global__ __launch_bounds__(512) void k_skinny16(const _Float16 *__restrict__ W16, int N, int K,
                                                  const half8 *__restrict__ X16, const float *__restrict__ xs_inv,
                                                  const float *__restrict__ bias, float *__restrict__ Y, int M) {
    extern __shared__ f32x4 red[];  // [NW][TB][64]
    const int NW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int o0 = blockIdx.x * 16;
    const int orow = o0 + j < N ? o0 + j : N - 1;
    const int nsb = K / 256;
    const int kf_n = K / 16;
    const int own = wave * C;
    const int s0 = own < nsb - C ? own : nsb - C;
    const half8 *wr = reinterpret_cast<const half8 *>(W16 + (size_t)orow * K + (size_t)s0 * 256) + q;
    const half8 *xq[TB];
    f32x4 acc[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) {
        acc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        int t = tb * 16 + j;
        t = t < M ? t : M - 1;
        // window m of super-block i: k = 32m + 8q -> fragment 2m + q/2, half q&1
        xq[tb] = X16 + ((size_t)(t >> 5) * kf_n + (size_t)s0 * 16 + (q >> 1)) * 64 + (t & 31) + 32 * (q & 1);
    }
    // weights one window ahead; activations one window ahead for one token
    // block, loaded at the start of the window otherwise (register budget)
    constexpr int AB = TB == 1 ? 2 : 1;
    half8 b[2][8], a[AB][8][TB];
#pragma unroll
    for (int m = 0; m < 8; m++) {
        b[0][m] = wr[4 * m];
#pragma unroll
        for (int tb = 0; tb < TB; tb++) a[0][m][tb] = xq[tb][(2 * m) * 64];
    }
#pragma unroll
    for (int i = 0; i < C; i++) {
        const int cur = i & 1, ac = AB == 2 ? cur : 0;
        if (i + 1 < C) {
#pragma unroll
            for (int m = 0; m < 8; m++) {
                b[cur ^ 1][m] = wr[(i + 1) * 32 + 4 * m];
                if constexpr (AB == 2) {
#pragma unroll
                    for (int tb = 0; tb < TB; tb++) a[ac ^ 1][m][tb] = xq[tb][((i + 1) * 16 + 2 * m) * 64];
                }
            }
        }
        if (AB == 1 && i > 0) {
#pragma unroll
            for (int m = 0; m < 8; m++)
#pragma unroll
                for (int tb = 0; tb < TB; tb++) a[0][m][tb] = xq[tb][(i * 16 + 2 * m) * 64];
        }
        if (s0 + i >= own) {
#pragma unroll
            for (int m = 0; m < 8; m++)
#pragma unroll
                for (int tb = 0; tb < TB; tb++)
                    acc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ac][m][tb], b[cur][m], acc[tb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++) red[(wave * TB + tb) * 64 + lane] = acc[tb];
    __syncthreads();
    for (int idx = threadIdx.x; idx < TB * 64; idx += blockDim.x) {
        const int tb = idx >> 6, l = idx & 63;
        f32x4 s = red[tb * 64 + l];
        for (int w = 1; w < NW; w++) s += red[(w * TB + tb) * 64 + l];
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

// Large M on fp16 rows: the k_gemm tile (256 tokens x 128 rows, 4 wavefronts
// of 64 tokens, v_mfma_f32_32x32x16_f16) with the B fragments copied from W16
// instead of dequantised: per K step of 64, thread (r, h) moves k 16h..16h+15
// and 32+16h..32+16h+15 of row r into the same LDS fragment slots k_gemm's
// dequantisation writes.  Next step's rows and activations are loaded during
// the current step's MFMAs; one barrier per step.
__global__ __launch_bounds__(256, 2) void k_gemm16(const _Float16 *__restrict__ W16, int N, int K,
                                                   const half8 *__restrict__ X16, const float *__restrict__ xs_inv,
                                                   const float *__restrict__ bias, float *__restrict__ Y, int M,
                                                   int m_tiles, int n_tiles) {
    __shared__ half8 lds[2][16][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int total = m_tiles * n_tiles;
    const int id = blockIdx.x;
    const int per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int mt = L / n_tiles, nt = L - mt * n_tiles;
    const int m0 = mt * GEMM_BM, n0 = nt * GEMM_BN;
    const int r = tid & 127, h = tid >> 7;
    int orow = n0 + r;
    orow = orow < N ? orow : N - 1;
    const half8 *wrow = reinterpret_cast<const half8 *>(W16 + (size_t)orow * K) + 2 * h;
    const int wf = (r >> 5) * 4, wl = r & 31;
    const int kf_n = K / 16;
    const half8 *xa0 = X16 + ((size_t)(m0 / 32 + 2 * wave) * kf_n) * 64 + lane;
    const half8 *xa1 = xa0 + (size_t)kf_n * 64;
    const int S = K / 64;
    f32x16 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = f32x16{};
    half8 wb[4], xc[2][4], xn[2][4];
    // step s of row r: half8 index 8s + 2h + {0, 1} (k 16h..) and 8s + 4 + 2h + {0, 1} (k 32+16h..)
    wb[0] = wrow[0], wb[1] = wrow[1], wb[2] = wrow[4], wb[3] = wrow[5];
    gemm_load_x(xa0, xa1, 0, xc);
    lds[0][wf + h][wl] = wb[0], lds[0][wf + h][wl + 32] = wb[1];
    lds[0][wf + 2 + h][wl] = wb[2], lds[0][wf + 2 + h][wl + 32] = wb[3];
    __syncthreads();
    for (int s = 0; s < S; s++) {
        const int cur = s & 1;
        const bool more = s + 1 < S;
        if (more) {
            const half8 *p = wrow + 8 * (s + 1);
            wb[0] = p[0], wb[1] = p[1], wb[2] = p[4], wb[3] = p[5];
            gemm_load_x(xa0, xa1, s + 1, xn);
        }
        gemm_mfma(lds[cur], lane, xc, acc);
        if (more) {
            lds[cur ^ 1][wf + h][wl] = wb[0], lds[cur ^ 1][wf + h][wl + 32] = wb[1];
            lds[cur ^ 1][wf + 2 + h][wl] = wb[2], lds[cur ^ 1][wf + 2 + h][wl + 32] = wb[3];
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int k = 0; k < 4; k++) xc[a][k] = xn[a][k];
        }
        __syncthreads();
    }
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
template <int T>
static hipError_t launch_dequant_blocks(const void *src, int64_t row_bytes, int64_t n, int64_t rows, float *dst,
                                        hipStream_t st) {
    const int64_t nblk = n / Fmt<T>::BL;
    const int64_t blocks = (rows * nblk * Fmt<T>::P + 255) / 256;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dequant_blocks<T>, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t *)src,
                       row_bytes, nblk, rows, dst);
    return hipGetLastError();
}

extern "C" int fh3k_dequant_block_len(int type) {
    switch (type) {
        case FH3K_F32: case FH3K_F16: case FH3K_BF16: return 1;
        case FH3K_Q8_0: return 32;
        case FH3K_Q2_K: case FH3K_Q3_K: case FH3K_Q4_K: case FH3K_Q5_K: case FH3K_Q6_K: return 256;
        default: return 0;
    }
}

extern "C" hipError_t fh3k_dequant_f32(int type, const void *src, int64_t row_bytes, int64_t n, int64_t rows,
                                       float *dst, hipStream_t st) {
    const int bl = fh3k_dequant_block_len(type);
    if (bl == 0 || n <= 0 || rows <= 0 || n % bl) return hipErrorInvalidValue;
    if (type == FH3K_F32) {
        return hipMemcpy2DAsync(dst, (size_t)n * sizeof(float), src, (size_t)row_bytes, (size_t)n * sizeof(float),
                                (size_t)rows, hipMemcpyDeviceToDevice, st);
    }
    if (type == FH3K_F16 || type == FH3K_BF16) {
        const int64_t blocks = (rows * n + 255) / 256;
        if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
        if (type == FH3K_F16)
            hipLaunchKernelGGL(k_dequant_half<false>, dim3((unsigned)blocks), dim3(256), 0, st,
                               (const uint8_t *)src, row_bytes, n, rows, dst);
        else
            hipLaunchKernelGGL(k_dequant_half<true>, dim3((unsigned)blocks), dim3(256), 0, st,
                               (const uint8_t *)src, row_bytes, n, rows, dst);
        return hipGetLastError();
    }
    switch (type) {
        case FH3K_Q8_0: return launch_dequant_blocks<FH3K_Q8_0>(src, row_bytes, n, rows, dst, st);
        case FH3K_Q2_K: return launch_dequant_blocks<FH3K_Q2_K>(src, row_bytes, n, rows, dst, st);
        case FH3K_Q3_K: return launch_dequant_blocks<FH3K_Q3_K>(src, row_bytes, n, rows, dst, st);
        case FH3K_Q4_K: return launch_dequant_blocks<FH3K_Q4_K>(src, row_bytes, n, rows, dst, st);
        case FH3K_Q5_K: return launch_dequant_blocks<FH3K_Q5_K>(src, row_bytes, n, rows, dst, st);
        default: return launch_dequant_blocks<FH3K_Q6_K>(src, row_bytes, n, rows, dst, st);
    }
}

// From this many rows the 8-row kernel is used (below it its few 1024-thread
// workgroups are slower: 7.2 against 3.7 us at M = 16, equal at M = 8192).
constexpr int XPREP_R8_MIN_ROWS = 8192;

extern "C" hipError_t fh3k_xprep_norm(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv,
                                      const float *norm_w, float eps, const float *shift, const float *scale,
                                      float *xsum, hipStream_t st) {
    if (Mpad % 8 || Mpad < M || (shift != nullptr) != (scale != nullptr) || (shift && !norm_w))
        return hipErrorInvalidValue;
    const RowNorm nm{norm_w, eps, shift, scale};
    if (M >= XPREP_R8_MIN_ROWS && K <= (norm_w ? 8192 : 14336) && !xsum) {
        const dim3 g8((unsigned)(Mpad / 8)), b8(1024);
        if (norm_w) {
            if (K <= 4096)
                hipLaunchKernelGGL((k_xprep_r8<4, true>), g8, b8, 0, st, x, M, K, (half8 *)x16, xs_inv, nm);
            else
                hipLaunchKernelGGL((k_xprep_r8<8, true>), g8, b8, 0, st, x, M, K, (half8 *)x16, xs_inv, nm);
        } else {
            if (K <= 4096)
                hipLaunchKernelGGL((k_xprep_r8<4, false>), g8, b8, 0, st, x, M, K, (half8 *)x16, xs_inv, nm);
            else if (K <= 8192)
                hipLaunchKernelGGL((k_xprep_r8<8, false>), g8, b8, 0, st, x, M, K, (half8 *)x16, xs_inv, nm);
            else  // 4 rows per workgroup: 7 chunks of 8 per thread fit the 128 VGPRs of 1024 threads
                hipLaunchKernelGGL((k_xprep_r8<7, false, 4>), dim3((unsigned)(Mpad / 4)), b8, 0, st, x, M, K,
                                   (half8 *)x16, xs_inv, nm);
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)Mpad), block(256);
    if (K <= 4096)
        hipLaunchKernelGGL(k_xprep<4>, grid, block, 0, st, x, M, K, (half8 *)x16, xs_inv, nm, xsum);
    else if (K <= 8192)
        hipLaunchKernelGGL(k_xprep<8>, grid, block, 0, st, x, M, K, (half8 *)x16, xs_inv, nm, xsum);
    else if (K <= 16384)
        hipLaunchKernelGGL(k_xprep<16>, grid, block, 0, st, x, M, K, (half8 *)x16, xs_inv, nm, xsum);
    else if (K <= 32768)
        hipLaunchKernelGGL(k_xprep<32>, grid, block, 0, st, x, M, K, (half8 *)x16, xs_inv, nm, xsum);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t fh3k_xprep(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv,
                                 float *xsum, hipStream_t st) {
    return fh3k_xprep_norm(x, M, K, Mpad, x16, xs_inv, nullptr, 0.f, nullptr, nullptr, xsum, st);
}

extern "C" hipError_t fh3k_xprep_any(const float *x, int M, int K, int Mpad, void *x16, float *xs_inv,
                                     hipStream_t st) {
    if (M <= 0 || K <= 0 || Mpad < M || Mpad % 32) return hipErrorInvalidValue;
    const int64_t Kp = (int64_t)(K + 255) / 256 * 256;
    if (Kp > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_xprep_any, dim3((unsigned)Mpad), dim3(256), 0, st, x, M, K, (int)Kp, (half8 *)x16, xs_inv);
    return hipGetLastError();
}

extern "C" hipError_t fh3k_rownorm_f32(const float *x, int M, int K, float *y, const float *norm_w, float eps,
                                       const float *shift, const float *scale, hipStream_t st) {
    if (!norm_w || M <= 0 || K % 4 || (shift != nullptr) != (scale != nullptr)) return hipErrorInvalidValue;
    const RowNorm nm{norm_w, eps, shift, scale};
    const dim3 grid((unsigned)M), block(256);
    if (K <= 4096)
        hipLaunchKernelGGL(k_rownorm_f32<4>, grid, block, 0, st, x, K, y, nm);
    else if (K <= 8192)
        hipLaunchKernelGGL(k_rownorm_f32<8>, grid, block, 0, st, x, K, y, nm);
    else if (K <= 16384)
        hipLaunchKernelGGL(k_rownorm_f32<16>, grid, block, 0, st, x, K, y, nm);
    else if (K <= 32768)
        hipLaunchKernelGGL(k_rownorm_f32<32>, grid, block, 0, st, x, K, y, nm);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" int fh3k_max_in(void) { return 32768; }

// Workspace of the no-allocation entry point (fh3_hip_matmul_noalloc_dev):
// each device that loads this library holds its own copy until the process
// ends.  Host code must never pass `scratch` itself to a kernel: its host-side
// name is a stand-in, not a device address; fh3k_scratch_bind gives the
// current device's address of it.
static __device__ __align__(256) uint8_t scratch[FH3_HIP_NOALLOC_SCRATCH_BYTES];

extern "C" hipError_t fh3k_scratch_bind(void **ptr) {
    return hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch));
}

// Super-blocks per wavefront C (compile-time, C <= nsb) and wavefronts per
// workgroup NW (<= 8, runtime) for K/256 = nsb super-blocks: the fewest
// padding super-blocks NW*C - nsb, then, for one token block, C closest to 5
// (the best measured balance of per-wave work and parallelism at K = 5120),
// for more the smallest C (most wavefronts: each super-block's activation
// fragments, 32 VGPRs per token block, are loaded and waited for in turn;
// 64 x 4096 -> 4096: 14.8 us per call at C = 2, 15.7 at C = 4; 64 x 3072:
// 12.3 against 13.5).
static const int kSkinnyC[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 13, 16};

static void skinny_split(int nsb, int tb, int &C, int &NW) {
    int best = -1, bw = 1 << 30, bd = 1 << 30;
    for (int i = 0; i < (int)(sizeof kSkinnyC / sizeof kSkinnyC[0]); i++) {
        const int c = kSkinnyC[i], nw = (nsb + c - 1) / c;
        if (nw > 8 || c > nsb) continue;
        const int waste = nw * c - nsb, dist = tb > 1 ? c : (c > 5 ? c - 5 : 5 - c);
        if (waste < bw || (waste == bw && dist < bd)) best = i, bw = waste, bd = dist;
    }
    C = best >= 0 ? kSkinnyC[best] : 0;
    NW = C ? (nsb + C - 1) / C : 0;
}

// Workgroups of the 16-row kernels: 16 rows each, or 8 output columns (16
// weight rows) under SwiGLU.
static unsigned row_blocks16(int N, int epi) {
    return (unsigned)(epi == EPI_SWIGLU ? (N / 2) / 8 : (N + 15) / 16);
}

// S > 1 (Q5_K / Q6_K only): K windows of L super-blocks, raw sums to part.
template <int QT, int TB, int C>
static hipError_t launch_skinny_c(const void *W, int64_t rb, int N, int K, const void *x16, const float *xs_inv,
                                  const float *bias, float *y, int M, int NW, int epi, const float *aux,
                                  hipStream_t st, int L, int S, float *part) {
    const size_t lds = (size_t)NW * TB * 64 * sizeof(f32x4);
    hipLaunchKernelGGL((k_skinny<QT, TB, C>), dim3(row_blocks16(N, epi), (unsigned)S), dim3(NW * 64), lds, st,
                       (const uint8_t *)W, rb, N, K, (const half8 *)x16, xs_inv, bias, y, M, epi, aux, L,
                       S > 1 ? part : nullptr);
    return hipGetLastError();
}

template <int TB, int QT = FH3K_Q4_K>
static hipError_t launch_skinny(const void *W, int64_t rb, int N, int K, const void *x16,
                                const float *xs_inv, const float *bias, float *y, int M, int epi, const float *aux,
                                hipStream_t st, int L = 0, int S = 1, float *part = nullptr) {
    int C, NW;
    skinny_split(S > 1 ? L : K / 256, TB, C, NW);
#define FH3_SKINNY_C(c)                                                                                            \
    case c: return launch_skinny_c<QT, TB, c>(W, rb, N, K, x16, xs_inv, bias, y, M, NW, epi, aux, st, L, S, part)
    switch (C) {
        FH3_SKINNY_C(1);
        FH3_SKINNY_C(2);
        FH3_SKINNY_C(3);
        FH3_SKINNY_C(4);
        FH3_SKINNY_C(5);
        FH3_SKINNY_C(6);
        FH3_SKINNY_C(7);
        FH3_SKINNY_C(8);
        FH3_SKINNY_C(10);
        FH3_SKINNY_C(13);
        FH3_SKINNY_C(16);
        default: return hipErrorInvalidValue;
    }
#undef FH3_SKINNY_C
}

extern "C" hipError_t fh3k_skinny_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                      const float *xs_inv, const float *bias, float *y, int M, int epi,
                                      const float *aux, hipStream_t st) {
    if (epi == EPI_SWIGLU && (N % 16)) return hipErrorInvalidValue;
    const int tb = (M + 15) / 16;
    switch (tb) {
        case 1: return launch_skinny<1>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, epi, aux, st);
        case 2: return launch_skinny<2>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, epi, aux, st);
        case 3: return launch_skinny<3>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, epi, aux, st);
        case 4: return launch_skinny<4>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, epi, aux, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t fh3k_skinny(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                  const float *xs_inv, const float *bias, float *y, int M, hipStream_t st) {
    return fh3k_skinny_epi(W, row_bytes, N, K, x16, xs_inv, bias, y, M, EPI_NONE, nullptr, st);
}

extern "C" int fh3k_skinny_max_tokens(void) { return 64; }

static int device_cus(void) {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        const bool ok = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
        cus[dev] = ok && n > 0 ? n : 256;
    }
    return cus[dev];
}

namespace {
__global__ __launch_bounds__(256) void k_midm_sum(const float *__restrict__ part, int S, int M, int N,
                                                  const float *__restrict__ xs_inv, const float *__restrict__ bias,
                                                  float *__restrict__ Y, int epi, const float *__restrict__ aux);
}  // namespace

// K windows of the Q5_K / Q6_K small-M product: when the 16-row blocks
// number fewer than four per CU, S windows of L >= 4 super-blocks (S * L >= nsb,
// every window non-empty), so that the grid fills the chip (Q6_K 25600 ->
// 5120 is 320 row blocks, 1.25 rounds of 256 CUs at one workgroup per CU;
// 5120 -> 1024 is 64).
static void skinny_kwin(int N, int K, int &L, int &S) {
    const int nsb = K / 256, rbs = (N + 15) / 16;
    const int want = (4 * device_cus() + rbs - 1) / rbs;
    S = want < nsb / 4 ? want : nsb / 4;
    if (S < 2) {
        S = 1, L = nsb;
        return;
    }
    L = (nsb + S - 1) / S;
    S = (nsb + L - 1) / L;
}

extern "C" size_t fh3k_skinny_q_part_bytes(int N, int K, int M) {
    int L, S;
    if (N < 1 || K < 256 || M < 1) return 0;
    skinny_kwin(N, K, L, S);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// Q5_K / Q6_K rows read in place by k_skinny (n_tok <= 64): no decoded copy.
template <int QT>
static hipError_t launch_skinny_q(const void *W, int64_t rb, int N, int K, const void *x16, const float *xs_inv,
                                  const float *bias, float *y, int M, float *part, hipStream_t st) {
    int L, S;
    skinny_kwin(N, K, L, S);
    if (S > 1 && !part) return hipErrorInvalidValue;
    hipError_t e;
#define FH3_SKINNY_Q(tb)                                                                                          \
    case tb: e = launch_skinny<tb, QT>(W, rb, N, K, x16, xs_inv, bias, y, M, EPI_NONE, nullptr, st, L, S, part); break
    switch ((M + 15) / 16) {
        FH3_SKINNY_Q(1);
        FH3_SKINNY_Q(2);
        FH3_SKINNY_Q(3);
        FH3_SKINNY_Q(4);
        default: return hipErrorInvalidValue;
    }
#undef FH3_SKINNY_Q
    if (e != hipSuccess || S == 1) return e;
    const int64_t outs = (int64_t)M * N;
    hipLaunchKernelGGL(k_midm_sum, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st, part, S, M, N, xs_inv,
                       bias, y, (int)EPI_NONE, (const float *)nullptr);
    return hipGetLastError();
}

extern "C" int fh3k_skinny_q_takes(int type) { return type == FH3K_Q5_K || type == FH3K_Q6_K; }

extern "C" hipError_t fh3k_skinny_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                    const float *xs_inv, const float *bias, float *y, int M, float *part,
                                    hipStream_t st) {
    if (K % 256 || K < 256 || N < 1 || M < 1 || M > 64) return hipErrorInvalidValue;
    if (type == FH3K_Q5_K)
        return launch_skinny_q<FH3K_Q5_K>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, part, st);
    if (type == FH3K_Q6_K)
        return launch_skinny_q<FH3K_Q6_K>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, part, st);
    return hipErrorInvalidValue;
}

// k_gemv8: C = ceil(nsb / 16) super-blocks per wavefront, NW = ceil(nsb / C)
// <= 16 wavefronts (more, smaller windows measured faster at K = 5120: C = 2,
// NW = 10 beats C = 4, NW = 5 and C = 5, NW = 4); grid = min(row blocks, CUs),
// each workgroup walking its row blocks.  At 1024 threads a wavefront has 128
// VGPRs: C <= 5 (one or two tokens) and C <= 3 (four) compile without spills,
// so K <= 20480 and K <= 12288; longer rows take the other kernels.
static const size_t kGemv8MaxLds = 160u << 10;  // one workgroup per CU

static int gemv8_mt(int M) { return M == 1 ? 1 : (M == 2 ? 2 : 4); }

static size_t gemv8_lds(int K, int M, int &C, int &NW) {
    const int nsb = K / 256, mt = gemv8_mt(M);
    C = (nsb + 15) / 16;
    NW = C ? (nsb + C - 1) / C : 0;
    if (C < 1 || C > (mt == 4 ? 3 : 5)) return 0;
    return (size_t)NW * C * mt * (2 * G8_REC + G8_XS) + 2 * (size_t)NW * 64 * sizeof(float);
}

extern "C" int fh3k_gemv8_max_tokens(void) { return G8_MAX_TOKENS; }

extern "C" int fh3k_gemv8_fits(int K, int M) {
    int C, NW;
    if (M < 1 || M > G8_MAX_TOKENS || K < 256 || K % 256) return 0;
    const size_t lds = gemv8_lds(K, M, C, NW);
    return lds > 0 && lds <= kGemv8MaxLds;
}

template <int MT, int C, int EPI>
static hipError_t launch_gemv8_c(const void *W, int64_t rb, int N, int K, const float *x, const float *bias,
                                 float *y, int M, int NW, const float *aux, hipStream_t st) {
    int C_, NW_;
    const size_t lds = gemv8_lds(K, M, C_, NW_);
    const int nblk = (int)row_blocks16(N, EPI);
    const int cus = device_cus();
    const int grid = nblk < cus ? nblk : cus;
    hipLaunchKernelGGL((k_gemv8<MT, C, 1024, EPI>), dim3(grid), dim3(NW * 64), lds, st, (const uint8_t *)W, rb, N,
                       K, x, bias, y, M, aux, nblk);
    return hipGetLastError();
}

template <int MT, int EPI>
static hipError_t launch_gemv8_e(const void *W, int64_t rb, int N, int K, const float *x, const float *bias,
                                 float *y, int M, const float *aux, hipStream_t st) {
    int C, NW;
    gemv8_lds(K, M, C, NW);
    switch (C) {
        case 1: return launch_gemv8_c<MT, 1, EPI>(W, rb, N, K, x, bias, y, M, NW, aux, st);
        case 2: return launch_gemv8_c<MT, 2, EPI>(W, rb, N, K, x, bias, y, M, NW, aux, st);
        case 3: return launch_gemv8_c<MT, 3, EPI>(W, rb, N, K, x, bias, y, M, NW, aux, st);
        default: break;
    }
    if constexpr (MT <= 2) {
        switch (C) {
            case 4: return launch_gemv8_c<MT, 4, EPI>(W, rb, N, K, x, bias, y, M, NW, aux, st);
            case 5: return launch_gemv8_c<MT, 5, EPI>(W, rb, N, K, x, bias, y, M, NW, aux, st);
            default: break;
        }
    }
    return hipErrorInvalidValue;
}

template <int MT>
static hipError_t launch_gemv8(const void *W, int64_t rb, int N, int K, const float *x, const float *bias, float *y,
                               int M, int epi, const float *aux, hipStream_t st) {
    switch (epi) {
        case EPI_NONE: return launch_gemv8_e<MT, EPI_NONE>(W, rb, N, K, x, bias, y, M, aux, st);
        case EPI_GATE_RES: return launch_gemv8_e<MT, EPI_GATE_RES>(W, rb, N, K, x, bias, y, M, aux, st);
        case EPI_SWIGLU: return launch_gemv8_e<MT, EPI_SWIGLU>(W, rb, N, K, x, bias, y, M, aux, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t fh3k_gemv8_epi(const void *W, int64_t row_bytes, int N, int K, const float *x,
                                     const float *bias, float *y, int M, int epi, const float *aux, hipStream_t st) {
    if (!fh3k_gemv8_fits(K, M) || N < 1 || (epi == EPI_SWIGLU && (N % 16))) return hipErrorInvalidValue;
    switch (gemv8_mt(M)) {
        case 1: return launch_gemv8<1>(W, row_bytes, N, K, x, bias, y, M, epi, aux, st);
        case 2: return launch_gemv8<2>(W, row_bytes, N, K, x, bias, y, M, epi, aux, st);
        default: return launch_gemv8<4>(W, row_bytes, N, K, x, bias, y, M, epi, aux, st);
    }
}

extern "C" hipError_t fh3k_gemv8(const void *W, int64_t row_bytes, int N, int K, const float *x, const float *bias,
                                 float *y, int M, hipStream_t st) {
    return fh3k_gemv8_epi(W, row_bytes, N, K, x, bias, y, M, EPI_NONE, nullptr, st);
}

// k_sweep: up to 16 tokens (one token block) with C = 2 super-blocks per
// wavefront, 17..32 tokens (two token blocks) with C = 1 (on rows of at most
// 16 super-blocks: see sweep_groups); either way the
// activation fragments of a wavefront's window take 64 VGPRs and at most 10
// wavefronts run at <= 168 VGPRs (about 160 used; C = 3 would spill), so a
// K slice holds at most 10 C super-blocks.  Longer rows (to K = 32768) are
// split into S equal slices whose raw sums go to part[S][M][N] and are added
// in slice order by k_midm_sum (slices of at most 20 measured best for one
// token block: at K = 8192 two slices of 16 beat one of 32 by 3-10 %, at
// K = 25600 five of 20 beat four of 25 and seven of 15; K = 5120 stays whole).
static int sweep_tb(int M) { return (M + 15) / 16; }

// 17..64 tokens on rows of at most 16 super-blocks: groups of 32 tokens (two
// token blocks) swept by their own workgroups, two super-blocks per
// wavefront (128 VGPRs of activations, at most 8 wavefronts), no K split.
// Each CU then reads the fp16 activations of one group only (64 x 4096:
// 256 KB instead of 512 KB).
static bool sweep_groups(int nsb, int M) { return M > 16 && nsb <= 16; }

// qt: the weight type.  Q6_K with one token block: rows of at most 16
// super-blocks whole, eight wavefronts of two (its larger weight ring leaves
// no room for ten), longer rows in slices of at most 10, one super-block per
// wavefront (K = 25600: 47.9 against 54.6 us per call in slices of 16, two
// each; K = 3072 whole: 9.2 against 11.9 in two slices).
static bool sweep_q6_one(int nsb, int qt) { return qt == FH3K_Q6_K && nsb > 16; }

static void sweep_split(int nsb, int M, int &S, int &SL, int qt = FH3K_Q4_K) {
    if (sweep_groups(nsb, M)) {
        S = 1, SL = nsb;
        return;
    }
    const int tb = sweep_tb(M);
    const int cap = tb == 1 ? (qt == FH3K_Q6_K ? (sweep_q6_one(nsb, qt) ? 10 : 16) : 20) : (tb == 2 ? 10 : 8);
    S = (nsb + cap - 1) / cap;
    SL = (nsb + S - 1) / S;
}

extern "C" int fh3k_sweep_max_tokens(void) { return 64; }

extern "C" int fh3k_sweep_fits(int K, int M) {
    return M >= 1 && M <= 64 && K >= 512 && K <= 32768 && K % 256 == 0;
}

extern "C" size_t fh3k_sweep_part_bytes(int N, int K, int M) {
    int S, SL;
    if (!fh3k_sweep_fits(K, M) || N < 1) return 0;
    sweep_split(K / 256, M, S, SL);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <int C, int TB, int LB, int EPI, int QT = FH3K_Q4_K>
static hipError_t launch_sweep_c(const void *W, int64_t rb, int N, int K, const void *x16, const float *xs_inv,
                                 const float *xsum, const float *bias, float *y, int M, const float *aux, float *part,
                                 hipStream_t st) {
    int S, SL;
    sweep_split(K / 256, M, S, SL, QT);
    const int NW = (SL + C - 1) / C;
    const int nblk = (int)row_blocks16(N, EPI);
    const int TG = (M + 16 * TB - 1) / (16 * TB);  // token groups (k_sweep)
    const int per = device_cus() / (S * TG);      // workgroups per slice and group
    const int grid = (nblk < per ? nblk : per) * S * TG;
    const size_t lds = 2 * (size_t)NW * TB * 64 * sizeof(f32x4);
    if (NW * 64 > (LB < 640 ? LB : 640) || SL < C || nblk < 1 || grid < S || (S > 1 && !part))
        return hipErrorInvalidValue;
    float *pp = S > 1 ? part : nullptr;
    hipLaunchKernelGGL((k_sweep<C, TB, LB, EPI, QT>), dim3(grid), dim3(NW * 64), lds, st, (const uint8_t *)W, rb, N,
                       K, (const half8 *)x16, xs_inv, xsum, bias, y, M, aux, nblk, S, pp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int64_t outs = (int64_t)M * (EPI == EPI_SWIGLU ? N / 2 : N);
    hipLaunchKernelGGL(k_midm_sum, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st, part, S, M, N, xs_inv,
                       bias, y, EPI, aux);
    return hipGetLastError();
}

template <int EPI, int QT = FH3K_Q4_K>
static hipError_t launch_sweep_e(const void *W, int64_t rb, int N, int K, const void *x16, const float *xs_inv,
                                 const float *xsum, const float *bias, float *y, int M, const float *aux, float *part,
                                 hipStream_t st) {
    constexpr int LB1 = QT == FH3K_Q6_K ? 512 : 768;  // one token block: see sweep_split
    if (sweep_groups(K / 256, M))
        return launch_sweep_c<2, 2, 512, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
    switch (sweep_tb(M)) {
        case 1:
            if (sweep_q6_one(K / 256, QT))
                return launch_sweep_c<1, 1, 768, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
            return launch_sweep_c<2, 1, LB1, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        case 2: return launch_sweep_c<1, 2, 768, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        // three or four token blocks: 96 / 128 VGPRs of activations, so at most
        // 8 wavefronts (two per SIMD, 256 VGPRs each)
        case 3: return launch_sweep_c<1, 3, 512, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        default: return launch_sweep_c<1, 4, 512, EPI, QT>(W, rb, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
    }
}

// Q6_K weights read in place by the sweep (no epilogue, no group sums).
extern "C" int fh3k_sweep_q_takes(int type) { return type == FH3K_Q6_K; }

extern "C" size_t fh3k_sweep_q_part_bytes(int type, int N, int K, int M) {
    int S, SL;
    if (!fh3k_sweep_q_takes(type) || !fh3k_sweep_fits(K, M) || N < 1) return 0;
    sweep_split(K / 256, M, S, SL, type);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

extern "C" hipError_t fh3k_sweep_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                   const float *xs_inv, const float *bias, float *y, int M, float *part,
                                   hipStream_t st) {
    if (!fh3k_sweep_q_takes(type) || !fh3k_sweep_fits(K, M) || N < 1) return hipErrorInvalidValue;
    return launch_sweep_e<EPI_NONE, FH3K_Q6_K>(W, row_bytes, N, K, x16, xs_inv, nullptr, bias, y, M, nullptr, part,
                                                st);
}

extern "C" hipError_t fh3k_sweep_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                     const float *xs_inv, const float *xsum, const float *bias, float *y, int M,
                                     int epi, const float *aux, float *part, hipStream_t st) {
    if (!fh3k_sweep_fits(K, M) || N < 1 || !xsum || (epi == EPI_SWIGLU && (N % 16))) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_NONE:
            return launch_sweep_e<EPI_NONE>(W, row_bytes, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        case EPI_GATE_RES:
            return launch_sweep_e<EPI_GATE_RES>(W, row_bytes, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        case EPI_SWIGLU:
            return launch_sweep_e<EPI_SWIGLU>(W, row_bytes, N, K, x16, xs_inv, xsum, bias, y, M, aux, part, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" int fh3k_gemm_row_pad(void) { return GEMM_BM; }

// ---------------------------------------------------------------------------
// Middle M (17..64 tokens): split K, then an ordered sum.
//
// With few tokens and few weight rows (M = 64, N = 4096 is 256 tiles of
// 32 x 32) the work only fills the chip when K is split as well, and a
// 16-row wavefront that reads every token's activations for the whole of K
// (k_skinny) moves M*K*2 bytes through L2 per 16 rows.  k_midm gives a
// workgroup 128 weight rows (4 wavefronts x 32) and a window of C super-blocks:
//   - the window's activation fragments (TB2 token blocks of 32) are staged
//     once per super-block into LDS and read by all four wavefronts;
//   - each wavefront dequantises its own 32 rows straight into B operands
//     (v_fma_mix, as k_gemm rounds Q4_K), so the weights need no LDS;
//   - v_mfma_f32_32x32x16_f16, one 32x32 accumulator per token block.
// Partial sums go to part[ks][t][o]; k_midm_sum adds the S windows in
// window order (deterministic), scales, adds the bias and applies the
// epilogue.
// ---------------------------------------------------------------------------
namespace {

constexpr int MIDM_ROWS = 128;

template <int TB2>
__global__ __launch_bounds__(256, 2) void k_midm(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int K,
                                                 const half8 *__restrict__ X16, int M, int C, int n_rg,
                                                 float *__restrict__ part) {
    __shared__ half8 sx[2][TB2][16][64];  // staged fragments of one super-block, double-buffered
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;

    // consecutive ids go to different XCDs: give each XCD a contiguous run of
    // (window, row group) pairs so that one window's activations stay in one L2
    const int total = gridDim.x, id = blockIdx.x, per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int ks = L / n_rg, rg = L - ks * n_rg;
    const int nsb = K / 256, kf_n = K / 16;
    const int sb0 = ks * C;
    const int nw = nsb - sb0 < C ? nsb - sb0 : C;  // >= 1 by the launch

    int orow = rg * MIDM_ROWS + 32 * wave + (lane & 31);
    const bool orow_ok = orow < N;
    orow = orow_ok ? orow : N - 1;
    const uint8_t *wrow = W + (size_t)orow * row_bytes;

    // raw bytes of one super-block for this lane: the header and, per chunk c,
    // bytes 8h..8h+7 and 16+8h..16+8h+7 (k steps 4c..4c+3 take them)
    struct Raw {
        u32x4 hv;
        uint32_t q[4][2][2];
    };
    auto load_raw = [&](int sb, Raw &r) {
        const uint8_t *b = wrow + (size_t)sb * 144;
        r.hv = ld16(b);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const uint2 u = *reinterpret_cast<const uint2 *>(b + 16 + 32 * c + 16 * hf + 8 * h);
                r.q[c][hf][0] = u.x;
                r.q[c][hf][1] = u.y;
            }
    };
    // staging: thread tid moves fragment pieces f = tid + 256 i of the
    // TB2 x 16 x 64 half8 of one super-block
    constexpr int SPT = TB2 * 16 * 64 / 256;
    half8 stg[SPT];
    auto stage_load = [&](int sb) {
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int f = tid + 256 * i;
            const int tb = f / 1024, fr = (f / 64) % 16, l = f % 64;
            stg[i] = X16[((size_t)tb * kf_n + (size_t)sb * 16 + fr) * 64 + l];
        }
    };
    auto stage_store = [&](int b) {
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int f = tid + 256 * i;
            (&sx[b][0][0][0])[f] = stg[i];
        }
    };

    f32x16 acc[TB2];
#pragma unroll
    for (int t = 0; t < TB2; t++) acc[t] = f32x16{};

    Raw ra, rb;
    load_raw(sb0, ra);
    stage_load(sb0);
    stage_store(0);
    __syncthreads();
    for (int i = 0; i < nw; i++) {
        const int b = i & 1;
        const bool more = i + 1 < nw;
        if (more) {
            load_raw(sb0 + i + 1, rb);
            stage_load(sb0 + i + 1);
        }
        float Dg[8], Cg[8];
#pragma unroll
        for (int g = 0; g < 8; g++) q4k_group_fast(ra.hv, g, Dg[g], Cg[g]);
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int c = st >> 2, nib = (st >> 1) & 1, hf = st & 1, g = 2 * c + nib;
            const half8 bq = q4k_deq8_f16(ra.q[c][hf][0], ra.q[c][hf][1], nib != 0, Dg[g], Cg[g]);
#pragma unroll
            for (int t = 0; t < TB2; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sx[b][t][st][lane], bq, acc[t], 0, 0, 0);
        }
        if (more) stage_store(b ^ 1);
        ra = rb;
        __syncthreads();
    }

    // D: lane holds weight row orow, tokens 32 t + 8 (v/4) + 4 h + v%4
    if (orow_ok) {
        float *pp = part + (size_t)ks * M * N + orow;
#pragma unroll
        for (int t = 0; t < TB2; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int tok = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                if (tok < M) pp[(size_t)tok * N] = acc[t][v];
            }
    }
}

// y[t][o] = (sum over windows in order) * xs_inv[t] + bias[o], then the
// epilogue; one thread per output (SwiGLU: per val/gate pair).
__global__ __launch_bounds__(256) void k_midm_sum(const float *__restrict__ part, int S, int M, int N,
                                                  const float *__restrict__ xs_inv, const float *__restrict__ bias,
                                                  float *__restrict__ Y, int epi, const float *__restrict__ aux) {
    const int F = N >> 1;
    const int width = epi == EPI_SWIGLU ? F : N;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * width) return;
    const int t = (int)(i / width), o = (int)(i - (int64_t)t * width);
    const size_t mn = (size_t)M * N;
    const float *p = part + (size_t)t * N + o;
    // the windows' partials are loaded eight at a time before they are added
    // (in window order), so their latencies overlap
    auto ordered_sum = [&](const float *q) {
        float s = 0.f;
        for (int k0 = 0; k0 < S; k0 += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = k0 + k < S ? q[(size_t)(k0 + k) * mn] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (k0 + k < S) s = k0 + k == 0 ? v[0] : s + v[k];
        }
        return s;
    };
    const float s = ordered_sum(p);
    if (epi == EPI_SWIGLU) {
        const float sg = ordered_sum(p + F);
        const float bv = bias ? bias[o] : 0.f, bg = bias ? bias[F + o] : 0.f;
        Y[(size_t)t * F + o] = (s * xs_inv[t] + bv) * silu_f32(sg * xs_inv[t] + bg);
        return;
    }
    epi_store(Y, aux, epi, (size_t)t * N + o, s * xs_inv[t] + (bias ? bias[o] : 0.f));
}

}  // namespace

// Window length C and split count S for k_midm: about two workgroups per CU
// (512) and at least two super-blocks per window where K allows it.
static void midm_split(int N, int K, int &C, int &S) {
    const int nsb = K / 256, n_rg = (N + MIDM_ROWS - 1) / MIDM_ROWS;
    int s = (512 + n_rg - 1) / n_rg;
    const int smax = nsb >= 2 ? nsb / 2 : 1;
    s = s < 1 ? 1 : (s > smax ? smax : s);
    C = (nsb + s - 1) / s;
    S = (nsb + C - 1) / C;
}

extern "C" int fh3k_midm_max_tokens(void) { return 64; }

extern "C" size_t fh3k_midm_part_bytes(int N, int K, int M) {
    int C, S;
    if (N <= 0 || K < 256 || M <= 0) return 0;
    midm_split(N, K, C, S);
    return (size_t)S * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" hipError_t fh3k_midm_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                    const float *xs_inv, const float *bias, float *y, int M, int epi,
                                    const float *aux, float *part, hipStream_t st) {
    if (M < 1 || M > 64 || K % 256 || (epi == EPI_SWIGLU && (N % 2))) return hipErrorInvalidValue;
    int C, S;
    midm_split(N, K, C, S);
    const int n_rg = (N + MIDM_ROWS - 1) / MIDM_ROWS;
    const dim3 grid((unsigned)(n_rg * S)), block(256);
    if (M <= 32)
        hipLaunchKernelGGL(k_midm<1>, grid, block, 0, st, (const uint8_t *)W, row_bytes, N, K, (const half8 *)x16, M,
                           C, n_rg, part);
    else
        hipLaunchKernelGGL(k_midm<2>, grid, block, 0, st, (const uint8_t *)W, row_bytes, N, K, (const half8 *)x16, M,
                           C, n_rg, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int width = epi == EPI_SWIGLU ? N / 2 : N;
    const int64_t outs = (int64_t)M * width;
    hipLaunchKernelGGL(k_midm_sum, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st, part, S, M, N, xs_inv,
                       bias, y, epi, aux);
    return hipGetLastError();
}

// Split K for k_gemm when its tiles alone would not fill the chip (a few
// hundred tokens or fewer): S windows of C super-blocks (at least two each).
// S minimises a simple time model in units of one super-block step of a
// workgroup (~5 us): rounds of 512 resident workgroups x (C + 1), plus the
// partial sums (written and read: S*M*N*8 bytes at ~5 TB/s) and the extra
// launch.
// 32-token blocks per k_gemm wavefront: one (128-token tiles) up to 128
// tokens, and up to 256 while the 128-token tiles number at most 128; two
// (256-token tiles) otherwise.  (Measured, K = 5120, calls incl. preparation
// and ordered sum: at N = 5120, 65-128 tokens 26.2-28.4 us against 32.2-34.3
// with 256-token tiles, 192 / 256 tokens 34.8 / 36.2 against 37.6 / 40.4; at
// N = 17408, 65-128 tokens 46-54 against 63-68, while at 192 / 256 tokens the
// 256-token tiles are faster, 76 / 82 against 88 / 92 us.)  257-384 tokens
// take 128-token tiles at every N: three of them pad to 384 rows where two
// 256-token tiles pad to 512 (300 tokens, K = 5120: N = 1024 / 5120 / 17408
// 25.3 / 44.4 / 103 us against 29.9 / 51.9 / 142; K = 8192-25600: 2-12 %
// faster).  From 385 tokens both pad alike and the 256-token tiles are faster.
static int gemm_tbw(int M, int N, int epi) {
    if (M <= 128) return 1;
    if (M > 256) return M <= 384 ? 1 : 2;
    const int n_tiles = epi == EPI_SWIGLU ? (N / 2) / 64 : (N + GEMM_BN - 1) / GEMM_BN;
    return M <= 256 && 2 * n_tiles <= 128 ? 1 : 2;
}

extern "C" int fh3k_gemm_rows(int M) {
    const int BM = M <= 128 || (M > 256 && M <= 384) ? 128 : 256;
    return (M + BM - 1) / BM * BM;
}

static void gemm_split(int M, int N, int K, int epi, int &C, int &S) {
    const int nsb = K / 256;
    const int BM = 128 * gemm_tbw(M, N, epi);
    const int m_tiles = (M + BM - 1) / BM;
    const int n_tiles = epi == EPI_SWIGLU ? (N / 2) / 64 : (N + GEMM_BN - 1) / GEMM_BN;
    const int64_t tiles = (int64_t)m_tiles * n_tiles;
    const int smax = nsb >= 4 ? nsb / 2 : 1;
    auto rounds = [](int64_t wgs) { return (double)((wgs + 511) / 512); };
    double best = rounds(tiles) * (nsb + 1);
    C = nsb;
    S = 1;
    for (int s = 2; s <= smax && tiles * s <= 4096; s++) {
        const int c = (nsb + s - 1) / s;
        if ((nsb + c - 1) / c != s) continue;  // same windows as a smaller s
        const double cost = rounds(tiles * s) * (c + 1) + (double)s * M * N * 8.0 / 2.5e7 + 0.4;
        if (cost < best) best = cost, C = c, S = s;
    }
}

extern "C" size_t fh3k_gemm_part_bytes(int N, int K, int M, int epi) {
    int C, S;
    if (N <= 0 || K < 256 || M <= 0) return 0;
    gemm_split(M, N, K, epi, C, S);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <int QT>
static hipError_t launch_gemm(const void *W, int64_t row_bytes, int N, int K, const void *x16, const float *xs_inv,
                              const float *bias, float *y, int M, int epi, const float *aux, float *part,
                              hipStream_t st) {
    if (epi == EPI_SWIGLU && (N % 128)) return hipErrorInvalidValue;
    if ((uint64_t)N * (uint64_t)row_bytes >= (1ull << 32)) return hipErrorInvalidValue;  // 32-bit row offsets
    int C, S;
    gemm_split(M, N, K, epi, C, S);
    if (S > 1 && !part) return hipErrorInvalidValue;
    const int tbw = gemm_tbw(M, N, epi), BM = 128 * tbw;
    const int m_tiles = (M + BM - 1) / BM;
    const int n_tiles = epi == EPI_SWIGLU ? (N / 2) / 64 : (N + GEMM_BN - 1) / GEMM_BN;
    if (tbw == 1)
        hipLaunchKernelGGL((k_gemm<1, QT>), dim3((unsigned)(m_tiles * n_tiles * S)), dim3(256), 0, st,
                           (const uint8_t *)W, row_bytes, N, K, (const half8 *)x16, xs_inv, bias, y, M,
                           m_tiles, n_tiles, epi, aux, C, S > 1 ? part : nullptr);
    else
        hipLaunchKernelGGL((k_gemm<2, QT>), dim3((unsigned)(m_tiles * n_tiles * S)), dim3(256), 0, st,
                           (const uint8_t *)W, row_bytes, N, K, (const half8 *)x16, xs_inv, bias, y, M,
                           m_tiles, n_tiles, epi, aux, C, S > 1 ? part : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int width = epi == EPI_SWIGLU ? N / 2 : N;
    const int64_t outs = (int64_t)M * width;
    hipLaunchKernelGGL(k_midm_sum, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st, part, S, M, N, xs_inv,
                       bias, y, epi, aux);
    return hipGetLastError();
}

extern "C" hipError_t fh3k_gemm_epi(const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                    const float *xs_inv, const float *bias, float *y, int M, int epi,
                                    const float *aux, float *part, hipStream_t st) {
    return launch_gemm<FH3K_Q4_K>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, epi, aux, part, st);
}

extern "C" int fh3k_gemm_q_takes(int type) { return type == FH3K_Q5_K || type == FH3K_Q6_K; }

extern "C" hipError_t fh3k_gemm_q(int type, const void *W, int64_t row_bytes, int N, int K, const void *x16,
                                  const float *xs_inv, const float *bias, float *y, int M, float *part,
                                  hipStream_t st) {
    if (K % 256 || K < 256 || N < 1 || M < 1) return hipErrorInvalidValue;
    if (type == FH3K_Q5_K)
        return launch_gemm<FH3K_Q5_K>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, EPI_NONE, nullptr, part, st);
    if (type == FH3K_Q6_K)
        return launch_gemm<FH3K_Q6_K>(W, row_bytes, N, K, x16, xs_inv, bias, y, M, EPI_NONE, nullptr, part, st);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Other weight types: decode to fp16 rows, then k_skinny16 / k_gemm16
// ---------------------------------------------------------------------------
template <int T>
static hipError_t launch_weights_f16_blocks(const void *src, int64_t row_bytes, int64_t n, int64_t n_out,
                                            int64_t rows, void *dst, hipStream_t st) {
    const int64_t nblk = n / Fmt<T>::BL, nblk_out = n_out / Fmt<T>::BL;
    const int64_t blocks = (rows * nblk_out * Fmt<T>::P + 255) / 256;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_weights_f16_blocks<T>, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t *)src,
                       row_bytes, nblk, nblk_out, rows, (_Float16 *)dst);
    return hipGetLastError();
}

template <int T>
static hipError_t launch_weights_f16_any(const void *src, int64_t row_bytes, int K, int Kp, int64_t rows,
                                         void *dst, hipStream_t st) {
    const int64_t blocks = (rows * (Kp / 8) + 255) / 256;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_weights_f16_any<T>, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t *)src,
                       row_bytes, K, Kp, rows, (_Float16 *)dst);
    return hipGetLastError();
}

extern "C" hipError_t fh3k_weights_f16(int type, const void *src, int64_t row_bytes, int K, int Kp, int N,
                                       void *dst, hipStream_t st) {
    const int bl = fh3k_dequant_block_len(type);
    if (bl == 0 || K <= 0 || N <= 0 || K % bl || Kp < K || Kp % 256) return hipErrorInvalidValue;
    if (type == FH3K_F16 && Kp == K)
        return hipMemcpyAsync(dst, src, (size_t)N * K * 2, hipMemcpyDeviceToDevice, st);
    if ((type == FH3K_F32 || type == FH3K_BF16) && Kp == K) {
        const int64_t n8 = (int64_t)N * K / 8, blocks = (n8 + 255) / 256;
        if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
        if (type == FH3K_BF16)
            hipLaunchKernelGGL(k_weights_f16_elem<true>, dim3((unsigned)blocks), dim3(256), 0, st,
                               (const uint8_t *)src, n8, (_Float16 *)dst);
        else
            hipLaunchKernelGGL(k_weights_f16_elem<false>, dim3((unsigned)blocks), dim3(256), 0, st,
                               (const uint8_t *)src, n8, (_Float16 *)dst);
        return hipGetLastError();
    }
    switch (type) {
        case FH3K_F32: return launch_weights_f16_any<FH3K_F32>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_F16: return launch_weights_f16_any<FH3K_F16>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_BF16: return launch_weights_f16_any<FH3K_BF16>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_Q8_0: return launch_weights_f16_blocks<FH3K_Q8_0>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_Q2_K: return launch_weights_f16_blocks<FH3K_Q2_K>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_Q3_K: return launch_weights_f16_blocks<FH3K_Q3_K>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_Q4_K: return launch_weights_f16_blocks<FH3K_Q4_K>(src, row_bytes, K, Kp, N, dst, st);
        case FH3K_Q5_K: return launch_weights_f16_blocks<FH3K_Q5_K>(src, row_bytes, K, Kp, N, dst, st);
        default: return launch_weights_f16_blocks<FH3K_Q6_K>(src, row_bytes, K, Kp, N, dst, st);
    }
}

template <int TB, int C>
static hipError_t launch_skinny16_c(const void *W16, int N, int K, const void *x16, const float *xs_inv,
                                    const float *bias, float *y, int M, int NW, hipStream_t st) {
    const size_t lds = (size_t)NW * TB * 64 * sizeof(f32x4);
    hipLaunchKernelGGL((k_skinny16<TB, C>), dim3((unsigned)((N + 15) / 16)), dim3(NW * 64), lds, st,
                       (const _Float16 *)W16, N, K, (const half8 *)x16, xs_inv, bias, y, M);
    return hipGetLastError();
}

template <int TB>
static hipError_t launch_skinny16(const void *W16, int N, int K, const void *x16, const float *xs_inv,
                                  const float *bias, float *y, int M, hipStream_t st) {
    int C, NW;
    skinny_split(K / 256, 1, C, NW);  // the one-token-block rule (not measured otherwise here)
    switch (C) {
        case 1: return launch_skinny16_c<TB, 1>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 2: return launch_skinny16_c<TB, 2>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 3: return launch_skinny16_c<TB, 3>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 4: return launch_skinny16_c<TB, 4>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 5: return launch_skinny16_c<TB, 5>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 6: return launch_skinny16_c<TB, 6>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 7: return launch_skinny16_c<TB, 7>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 8: return launch_skinny16_c<TB, 8>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 10: return launch_skinny16_c<TB, 10>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 13: return launch_skinny16_c<TB, 13>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        case 16: return launch_skinny16_c<TB, 16>(W16, N, K, x16, xs_inv, bias, y, M, NW, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t fh3k_skinny16(const void *W16, int N, int K, const void *x16, const float *xs_inv,
                                    const float *bias, float *y, int M, hipStream_t st) {
    switch ((M + 15) / 16) {
        case 1: return launch_skinny16<1>(W16, N, K, x16, xs_inv, bias, y, M, st);
        case 2: return launch_skinny16<2>(W16, N, K, x16, xs_inv, bias, y, M, st);
        case 3: return launch_skinny16<3>(W16, N, K, x16, xs_inv, bias, y, M, st);
        case 4: return launch_skinny16<4>(W16, N, K, x16, xs_inv, bias, y, M, st);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t fh3k_gemm16(const void *W16, int N, int K, const void *x16, const float *xs_inv,
                                  const float *bias, float *y, int M, hipStream_t st) {
    const int m_tiles = (M + GEMM_BM - 1) / GEMM_BM;
    const int n_tiles = (N + GEMM_BN - 1) / GEMM_BN;
    hipLaunchKernelGGL(k_gemm16, dim3((unsigned)(m_tiles * n_tiles)), dim3(256), 0, st, (const _Float16 *)W16, N, K,
                       (const half8 *)x16, xs_inv, bias, y, M, m_tiles, n_tiles);
    return hipGetLastError();
}
