// fh3_attn.hip -- the DiT block's attention branch on gfx950: q/k rmsnorm,
// rope3 and dense online-softmax attention (src/core/fh3_ops.c:410-456,
// 458-505, 587-695; the sequence of src/model/fh3_dit.c:390-411).
//
// Two launches per call:
//   k_attn_prep  fp32 q, k, v rows (any token stride, so q/k/v can be read in
//                place from the qkv projection's output) -> fp16 operands in
//                the layouts the matrix cores read: Qp[h][slot][d] and
//                Kp[h][slot][d] row-major, Vt[h][d][slot] transposed.  Optional
//                per-head rmsnorm of q and k (weights [hd]) and rope3 on their
//                first rot_dim channels are applied on the way; q is scaled by
//                log2(e)/sqrt(hd) so that the softmax runs on exp2.
//   k_attn_fwd   flash-style attention: a workgroup owns 128 queries of one
//                head (4 wavefronts x 32), streams 64-key tiles of K and V^T
//                through double-buffered LDS, S^T = K.Q^T and O^T = V^T.P^T on
//                v_mfma_f32_32x32x16_f16 with fp32 accumulation, and keeps the
//                running max / sum in fp32 registers.
//
// Slots beyond n are zero in the prepared operands and masked as keys, so
// any n >= 1 works; the prepared buffers hold n_pad = round_up(n, 128) slots.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fh3_kernels.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int ATT_KT = 64;   // keys per tile
constexpr int ATT_QW = 32;   // queries per wavefront
constexpr int ATT_NW = 4;    // wavefronts per workgroup
constexpr int ATT_QB = ATT_QW * ATT_NW;
constexpr int ATT_PREP_T = 64;  // slots per prep workgroup
// The softmax offset m of a query is only raised when a tile's maximum
// exceeds it by more than ATT_TAU (log2 units), so p = exp2(s - m) <= 2^8 and
// the rescale of the accumulators is skipped on almost every tile.  Any offset
// gives the same o = sum(p v) / sum(p); fp16 holds p up to 65504.
constexpr float ATT_TAU = 8.0f;

// Order of the keys inside each 16-key block of Vt.  The P^T operand of the
// PV product is taken straight from the S^T accumulator, where lane half hf
// holds keys {4hf..4hf+3, 8+4hf..8+4hf+3} of each 16-key block; storing V^T
// in that order lets one 16-byte LDS read feed the matching A operand.
__device__ __forceinline__ int vt_key(int p) {
    const int b = p & 15;
    return (p & ~15) + ((b & 3) | ((b & 4) << 1) | ((b & 8) >> 1));
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prep(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int64_t ld, int n,
                                                   const int *__restrict__ gather,
                                                   const float *__restrict__ qn_w, const float *__restrict__ kn_w,
                                                   float eps, const float *__restrict__ cosb,
                                                   const float *__restrict__ sinb, int rot, float qscale,
                                                   int n_pad, _Float16 *__restrict__ Qp, _Float16 *__restrict__ Kp,
                                                   _Float16 *__restrict__ Vt) {
    constexpr int DPT = HD / 4;
    __shared__ float sx[ATT_PREP_T][HD + 4];
    const int t = threadIdx.x, r = t >> 2, c = t & 3;
    const int slot = blockIdx.x * ATT_PREP_T + r, h = blockIdx.y;
    const int tok = gather ? gather[slot] : (slot < n ? slot : -1);
    const int d0 = c * DPT;

    for (int which = 0; which < 2; which++) {
        const float *src = which ? k : q;
        const float *nw = which ? kn_w : qn_w;
        float x[DPT];
        if (tok >= 0) {
            const f32x4 *p = (const f32x4 *)(src + (size_t)tok * ld + (size_t)h * HD + d0);
#pragma unroll
            for (int i = 0; i < DPT / 4; i++) {
                const f32x4 u = p[i];
                x[4 * i] = u[0], x[4 * i + 1] = u[1], x[4 * i + 2] = u[2], x[4 * i + 3] = u[3];
            }
        } else {
#pragma unroll
            for (int i = 0; i < DPT; i++) x[i] = 0.f;
        }
        if (nw) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < DPT; i++) ss = fmaf(x[i], x[i], ss);
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2);
            const float inv = tok >= 0 ? 1.0f / sqrtf(ss / (float)HD + eps) : 0.f;
#pragma unroll
            for (int i = 0; i < DPT; i++) x[i] = x[i] * inv * nw[d0 + i];
        }
        if (cosb) {
            __syncthreads();
#pragma unroll
            for (int i = 0; i < DPT; i++) sx[r][d0 + i] = x[i];
            __syncthreads();
            const int half = rot >> 1;
            if (tok >= 0 && (rot & 7) == 0) {
                // 4-element chunks never straddle half or rot: one region
                // test, and 16-byte reads of the tables and the partner chunk
                const float *cr = cosb + (size_t)tok * rot, *sr = sinb + (size_t)tok * rot;
#pragma unroll
                for (int i = 0; i < DPT / 4; i++) {
                    const int d = d0 + 4 * i;
                    if (d < rot) {
                        const bool lo = d < half;
                        const f32x4 cv = *(const f32x4 *)(cr + d), sv = *(const f32x4 *)(sr + d);
                        const f32x4 pv = *(const f32x4 *)&sx[r][lo ? d + half : d - half];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float a = x[4 * i + e] * cv[e], b = pv[e] * sv[e];
                            x[4 * i + e] = lo ? a - b : a + b;
                        }
                    }
                }
            } else if (tok >= 0) {
                const float *cr = cosb + (size_t)tok * rot, *sr = sinb + (size_t)tok * rot;
#pragma unroll
                for (int i = 0; i < DPT; i++) {
                    const int d = d0 + i;
                    if (d < half) {
                        const float a = x[i] * cr[d], b = sx[r][d + half] * sr[d];
                        x[i] = a - b;
                    } else if (d < rot) {
                        const float a = x[i] * cr[d], b = sx[r][d - half] * sr[d];
                        x[i] = a + b;
                    }
                }
            }
        }
        if (!which) {
#pragma unroll
            for (int i = 0; i < DPT; i++) x[i] *= qscale;
        }
        half8 *dst = (half8 *)((which ? Kp : Qp) + ((size_t)h * n_pad + slot) * HD + d0);
#pragma unroll
        for (int i = 0; i < DPT / 8; i++) {
            half8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = (_Float16)x[8 * i + e];
            dst[i] = o;
        }
    }

    // v: through LDS, written transposed in the vt_key order
    __syncthreads();
    if (tok >= 0) {
        const f32x4 *p = (const f32x4 *)(v + (size_t)tok * ld + (size_t)h * HD + d0);
#pragma unroll
        for (int i = 0; i < DPT / 4; i++) {
            const f32x4 u = p[i];
#pragma unroll
            for (int e = 0; e < 4; e++) sx[r][d0 + 4 * i + e] = u[e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < DPT; i++) sx[r][d0 + i] = 0.f;
    }
    __syncthreads();
    constexpr int PER = ATT_PREP_T * HD / 256;  // slots written per thread (32 or 16)
    constexpr int GROUPS = ATT_PREP_T / PER;
    const int d = t / GROUPS, p0 = (t % GROUPS) * PER;
    half8 *dst = (half8 *)(Vt + ((size_t)h * HD + d) * n_pad + (size_t)blockIdx.x * ATT_PREP_T + p0);
#pragma unroll
    for (int i = 0; i < PER / 8; i++) {
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (_Float16)sx[vt_key(p0 + 8 * i + e)][d];
        dst[i] = o;
    }
}

__device__ __forceinline__ float wave_swap_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }

template <int HD>
__global__ __launch_bounds__(256, 2) void k_attn_fwd(const _Float16 *__restrict__ Qp,
                                                     const _Float16 *__restrict__ Kp,
                                                     const _Float16 *__restrict__ Vt, int n, int n_pad,
                                                     int heads, float *__restrict__ O, int64_t o_ld) {
    constexpr int KS = HD / 16;            // 16-wide steps of the S product
    constexpr int DB = HD / 32;            // 32-row blocks of O^T
    constexpr int KROW = HD + 8;           // LDS row of K (halfs), padded against bank conflicts
    constexpr int VROW = ATT_KT + 8;       // LDS row of V^T (halfs)
    constexpr int NT = 64 * ATT_NW;
    constexpr int KCH = ATT_KT * HD / 8 / NT;  // 16-byte chunks per thread per tile, K and V each
    __shared__ _Float16 sk[2][ATT_KT][KROW];
    __shared__ _Float16 sv[2][HD][VROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hf = lane >> 5;

    // XCD-aware order: consecutive workgroup ids land on different XCDs, so
    // give each XCD a contiguous run of (head, query block) pairs
    const int nqb = n_pad / ATT_QB;
    const int total = heads * nqb;
    const int id = blockIdx.x;
    const int per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int h = L / nqb, qb = L - h * nqb;
    const int q0 = qb * ATT_QB + wave * ATT_QW;

    const _Float16 *kh = Kp + (size_t)h * n_pad * HD;
    const _Float16 *vh = Vt + (size_t)h * HD * n_pad;

    // Q^T fragments (B operand): lane holds query q0 + l32, d = 16 kk + 8 hf ..
    half8 qf[KS];
    {
        const half8 *qp = (const half8 *)(Qp + ((size_t)h * n_pad + q0 + l32) * HD + 8 * hf);
#pragma unroll
        for (int kk = 0; kk < KS; kk++) qf[kk] = qp[2 * kk];
    }

    half8 rk[KCH], rv[KCH];
    auto load_tile = [&](int j) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * NT;
            const int kr = c / (HD / 8), kc = c % (HD / 8);
            rk[i] = *(const half8 *)(kh + (size_t)(j * ATT_KT + kr) * HD + kc * 8);
            const int vr = c / (ATT_KT / 8), vc = c % (ATT_KT / 8);
            rv[i] = *(const half8 *)(vh + (size_t)vr * n_pad + j * ATT_KT + vc * 8);
        }
    };
    auto store_tile = [&](int b) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + i * NT;
            const int kr = c / (HD / 8), kc = c % (HD / 8);
            *(half8 *)&sk[b][kr][kc * 8] = rk[i];
            const int vr = c / (ATT_KT / 8), vc = c % (ATT_KT / 8);
            *(half8 *)&sv[b][vr][vc * 8] = rv[i];
        }
    };

    f32x16 o[DB];
#pragma unroll
    for (int i = 0; i < DB; i++) o[i] = f32x16{};
    float m = -INFINITY, lsum = 0.f;

    const int nkt = (n + ATT_KT - 1) / ATT_KT;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int j = 0; j < nkt; j++) {
        const int b = j & 1;
        if (j + 1 < nkt) load_tile(j + 1);

        // S^T[key][query] for the 64 keys: two 32-key accumulators
        f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const half8 a = *(const half8 *)&sk[b][32 * st + l32][16 * kk + 8 * hf];
                s[st] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], s[st], 0, 0, 0);
            }
        }
        // lane holds keys 32 st + 8 (v/4) + 4 hf + v%4 of query q0 + l32
        const int kv = n - j * ATT_KT;  // valid keys in this tile (>= 1)
        if (kv < ATT_KT) {
#pragma unroll
            for (int st = 0; st < 2; st++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    if (32 * st + 8 * (v >> 2) + 4 * hf + (v & 3) >= kv) s[st][v] = -INFINITY;
        }
        float mt = s[0][0];
#pragma unroll
        for (int v = 1; v < 16; v++) mt = fmaxf(mt, s[0][v]);
#pragma unroll
        for (int v = 0; v < 16; v++) mt = fmaxf(mt, s[1][v]);
        mt = wave_swap_max(mt);
        const bool grow = mt > m + ATT_TAU;
        if (__ballot(grow)) {  // wave-uniform: some query's offset must rise
            const float mn = grow ? mt : m;
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            lsum *= alpha;
#pragma unroll
            for (int i = 0; i < DB; i++) o[i] *= alpha;
        }
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int v = 0; v < 16; v++) s[st][v] = __builtin_amdgcn_exp2f(s[st][v] - m);

        // P^T fragments: 16-key step t = values 4g..4g+7 of accumulator t/2,
        // g = 2 (t % 2); they pair with V^T stored in the vt_key order.  The
        // row sum is taken over the same fp16 values the product uses.
        half8 pf[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
#pragma unroll
            for (int e = 0; e < 8; e++) pf[tt][e] = (_Float16)s[tt >> 1][8 * (tt & 1) + e];
        }
        float ps[2] = {0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                ps[e & 1] = __builtin_amdgcn_fdot2(half2v{pf[tt][2 * e], pf[tt][2 * e + 1]}, half2v{1, 1},
                                                   ps[e & 1], false);
        lsum += ps[0] + ps[1];
#pragma unroll
        for (int db = 0; db < DB; db++) {
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const half8 a = *(const half8 *)&sv[b][32 * db + l32][16 * tt + 8 * hf];
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[tt], o[db], 0, 0, 0);
            }
        }
        if (j + 1 < nkt) store_tile(b ^ 1);
        __syncthreads();
    }

    const float l = lsum + __shfl_xor(lsum, 32);
    const float inv = 1.0f / l;
    const int qq = q0 + l32;
    if (qq < n) {
        float *orow = O + (size_t)qq * o_ld + (size_t)h * HD;
#pragma unroll
        for (int db = 0; db < DB; db++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; e++) w[e] = o[db][4 * g + e] * inv;
                *(f32x4 *)(orow + 32 * db + 8 * g + 4 * hf) = w;
            }
    }
}

template <int HD>
hipError_t attn_launch(const float *q, const float *k, const float *v, int64_t ld, int n, int heads,
                       const float *qn_w, const float *kn_w, float eps, const float *cosb, const float *sinb,
                       int rot, void *ws, float *o, int64_t o_ld, hipStream_t st) {
    const int n_pad = (int)fh3k_attn_pad(n);
    _Float16 *Qp = (_Float16 *)ws;
    _Float16 *Kp = Qp + (size_t)heads * n_pad * HD;
    _Float16 *Vt = Kp + (size_t)heads * n_pad * HD;
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    hipLaunchKernelGGL(k_attn_prep<HD>, dim3(n_pad / ATT_PREP_T, heads), dim3(256), 0, st, q, k, v, ld, n,
                       (const int *)nullptr, qn_w, kn_w, eps, cosb, sinb, rot, qscale, n_pad, Qp, Kp, Vt);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int blocks = heads * (n_pad / ATT_QB);
    hipLaunchKernelGGL(k_attn_fwd<HD>, dim3(blocks), dim3(64 * ATT_NW), 0, st, Qp, Kp, Vt, n, n_pad, heads, o,
                       o_ld);
    return hipGetLastError();
}

}  // namespace

extern "C" int64_t fh3k_attn_pad(int n) { return ((int64_t)n + ATT_QB - 1) / ATT_QB * ATT_QB; }

extern "C" size_t fh3k_attn_ws_bytes(int n, int heads, int hd) {
    return (size_t)3 * heads * fh3k_attn_pad(n) * hd * sizeof(_Float16);
}

extern "C" int fh3k_attn_head_dim_ok(int hd) { return hd == 64 || hd == 128; }

extern "C" hipError_t fh3k_attention(const float *q, const float *k, const float *v, int64_t ld, int n, int heads,
                                     int hd, const float *qn_w, const float *kn_w, float eps, const float *cosb,
                                     const float *sinb, int rot, void *ws, float *o, int64_t o_ld, hipStream_t st) {
    if (hd == 128) return attn_launch<128>(q, k, v, ld, n, heads, qn_w, kn_w, eps, cosb, sinb, rot, ws, o, o_ld, st);
    if (hd == 64) return attn_launch<64>(q, k, v, ld, n, heads, qn_w, kn_w, eps, cosb, sinb, rot, ws, o, o_ld, st);
    return hipErrorInvalidValue;
}
