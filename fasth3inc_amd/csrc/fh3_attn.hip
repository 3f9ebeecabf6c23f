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
//   k_attn_fwd   flash-style attention: a workgroup owns 32 queries per
//                wavefront of one head (8 wavefronts for hd 128, 4 for hd 64
//                and for the sparse form), streams 64-key tiles of K and V^T
//                through double-buffered LDS, S^T = K.Q^T and O^T = V^T.P^T on
//                v_mfma_f32_32x32x16_f16 with fp32 accumulation, and keeps the
//                running max / sum in fp32 registers.
//
// Slots beyond n are zero in the prepared operands and masked as keys, so
// any n >= 1 works; the prepared buffers hold n_pad = round_up(n, 32 x wavefronts) slots.
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
constexpr int ATT_NW = 4;    // wavefronts per workgroup of the sparse kernel (two query tiles)
constexpr int ATT_QB = ATT_QW * ATT_NW;
// Dense kernel: with hd = 128, 8 wavefronts (256 queries, 2 per SIMD) share
// each K/V tile in LDS, halving the tile loads and LDS writes per query (+5 %);
// with hd = 64 the 4-wavefront form keeps 3 wavefronts per SIMD and is faster.
constexpr int dense_nw(int hd) { return hd == 128 ? 8 : 4; }
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

// Tile pooling (video sparse attention): with a gather map each prep
// workgroup holds exactly one 64-slot tile, so it also writes the tile's
// mean-pooled q, k (and v when vpool is set), pool[h][tile][d] = sum over the
// tile's tokens in order of x * inv[tile], from the final fp32 rows (after
// norm and rope, before the softmax scale) -- the reference's accumulation
// order and roundings (src/core/fh3_vsa.c:224-250).
struct Pool {
    const float *inv;
    const int *cnt;
    float *q, *k, *v;
    int T;
};

// sum over the first cnt rows of sx, in row order, times w (thread d < HD)
template <int HD>
__device__ __forceinline__ void pool_rows(const float (*sx)[HD + 4], int cnt, float w, float *dst) {
    const int d = threadIdx.x;
    if (d < HD) {
        float a = 0.f;
        for (int r = 0; r < cnt; r++) a = a + sx[r][d] * w;
        dst[d] = a;
    }
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prep(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int64_t ld, int64_t ldv, int n,
                                                   const int *__restrict__ gather,
                                                   const float *__restrict__ qn_w, const float *__restrict__ kn_w,
                                                   float eps, const float *__restrict__ cosb,
                                                   const float *__restrict__ sinb, int rot, float qscale,
                                                   int n_pad, _Float16 *__restrict__ Qp, _Float16 *__restrict__ Kp,
                                                   _Float16 *__restrict__ Vt, Pool pl) {
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
            // rot through an empty asm: otherwise the per-element region
            // tests below are hoisted out of the q/k loop and their 64-bit
            // lane masks, two per element, overflow the scalar registers
            int rv = rot;
            asm volatile("" : "+s"(rv));
            const int half = rv >> 1;
            if (tok >= 0 && (rv & 7) == 0) {
                // 4-element chunks never straddle half or rot: one region
                // test, and 16-byte reads of the tables and the partner chunk
                const float *cr = cosb + (size_t)tok * rv, *sr = sinb + (size_t)tok * rv;
#pragma unroll
                for (int i = 0; i < DPT / 4; i++) {
                    const int d = d0 + 4 * i;
                    if (d < rv) {
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
                const float *cr = cosb + (size_t)tok * rv, *sr = sinb + (size_t)tok * rv;
#pragma unroll
                for (int i = 0; i < DPT; i++) {
                    const int d = d0 + i;
                    if (d < half) {
                        const float a = x[i] * cr[d], b = sx[r][d + half] * sr[d];
                        x[i] = a - b;
                    } else if (d < rv) {
                        const float a = x[i] * cr[d], b = sx[r][d - half] * sr[d];
                        x[i] = a + b;
                    }
                }
            }
        }
        const int tile = blockIdx.x;
        if (pl.q && tile < pl.T) {  // uniform over the workgroup
            __syncthreads();
#pragma unroll
            for (int i = 0; i < DPT; i++) sx[r][d0 + i] = x[i];
            __syncthreads();
            pool_rows<HD>(sx, pl.cnt[tile], pl.inv[tile], (which ? pl.k : pl.q) + ((size_t)h * pl.T + tile) * HD);
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
        const f32x4 *p = (const f32x4 *)(v + (size_t)tok * ldv + (size_t)h * HD + d0);
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
    if (pl.v && blockIdx.x < pl.T)
        pool_rows<HD>(sx, pl.cnt[blockIdx.x], pl.inv[blockIdx.x], pl.v + ((size_t)h * pl.T + blockIdx.x) * HD);
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

// Block-sparse mode (video sparse attention).  Slots are tile-ordered: tile i
// owns slots 64 i .. 64 i + cnt[i] - 1 and gather[slot] names the token there
// (-1 for the empty rest of the tile).  The workgroup of query block qb holds
// query tiles 2 qb (wavefronts 0, 1) and 2 qb + 1 (wavefronts 2, 3); it walks
// the union of their selected key tiles, lists[(h * nqb + qb) * T + e] =
// key tile | (bit 14: tile 2 qb selects it) | (bit 15: tile 2 qb + 1 does),
// e < list_len[h * nqb + qb], and each pair of wavefronts skips the tiles its
// query tile did not select.  The output row of a slot goes to its token,
// plus coarse[h][tile][d] * gate[token][h][d] when a gate is given.
struct Sparse {
    const uint16_t *lists;
    const int *list_len;
    const int *cnt;
    const int *gather;
    const float *coarse;
    const float *gate;
    int T;
};

// (the second launch bound is the minimum number of wavefronts per SIMD: two)
template <int HD, bool SPARSE, int NW>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_fwd(const _Float16 *__restrict__ Qp,
                                                     const _Float16 *__restrict__ Kp,
                                                     const _Float16 *__restrict__ Vt, int n, int n_pad,
                                                     int heads, float *__restrict__ O, int64_t o_ld, Sparse sp) {
    constexpr int KS = HD / 16;            // 16-wide steps of the S product
    constexpr int DB = HD / 32;            // 32-row blocks of O^T
    constexpr int KROW = HD + 8;           // LDS row of K (halfs), padded against bank conflicts
    constexpr int VROW = ATT_KT + 8;       // LDS row of V^T (halfs)
    constexpr int NT = 64 * NW;
    constexpr int QB = ATT_QW * NW;
    constexpr int KCH = ATT_KT * HD / 8 / NT;  // 16-byte chunks per thread per tile, K and V each
    __shared__ _Float16 sk[2][ATT_KT][KROW];
    __shared__ _Float16 sv[2][HD][VROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hf = lane >> 5;

    // XCD-aware order: consecutive workgroup ids land on different XCDs, so
    // give each XCD a contiguous run of (head, query block) pairs
    const int nqb = n_pad / QB;
    const int total = heads * nqb;
    const int id = blockIdx.x;
    const int per = total >> 3;
    const int L = (id < per * 8) ? (id & 7) * per + (id >> 3) : id;
    const int h = L / nqb, qb = L - h * nqb;
    const int q0 = qb * QB + wave * ATT_QW;

    const _Float16 *kh = Kp + (size_t)h * n_pad * HD;
    const _Float16 *vh = Vt + (size_t)h * HD * n_pad;

    // Q^T fragments (B operand): lane holds query q0 + l32, d = 16 kk + 8 hf ..
    half8 qf[KS];
    {
        const half8 *qp = (const half8 *)(Qp + ((size_t)h * n_pad + q0 + l32) * HD + 8 * hf);
#pragma unroll
        for (int kk = 0; kk < KS; kk++) qf[kk] = qp[2 * kk];
    }

    // key tiles to visit: 0 .. nkt-1 (dense) or the block's list (sparse)
    const uint16_t *lst = nullptr;
    int nkt = (n + ATT_KT - 1) / ATT_KT;
    if (SPARSE) {
        lst = sp.lists + (size_t)L * sp.T;
        nkt = sp.list_len[L];
    }
    auto tile_of = [&](int e) { return SPARSE ? (int)(lst[e] & 0x3FFF) : e; };

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

    if (nkt > 0) {
        load_tile(tile_of(0));
        store_tile(0);
    }
    __syncthreads();
    for (int e = 0; e < nkt; e++) {
        const int b = e & 1;
        const int j = tile_of(e);
        if (e + 1 < nkt) load_tile(tile_of(e + 1));
        // valid keys in this tile (>= 1); in sparse mode, whether this pair of
        // wavefronts' query tile selected it (wave-uniform)
        const int kv = SPARSE ? sp.cnt[j] : n - j * ATT_KT;
        const bool active = SPARSE ? ((lst[e] >> (14 + (wave >> 1))) & 1) != 0 : true;
        if (active) {
            // dense: raised wave priority through the tile's matrix and softmax
            // work (the other wavefront on the SIMD is then mostly loading or
            // waiting; +1-2 %; the sparse walk loses with it)
            if constexpr (!SPARSE) __builtin_amdgcn_s_setprio(2);
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

            // P^T fragments: 16-key step t = values 4g..4g+7 of accumulator
            // t/2, g = 2 (t % 2); they pair with V^T stored in the vt_key
            // order.  The row sum is taken over the same fp16 values the
            // product uses.
            half8 pf[4];
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
#pragma unroll
                for (int q = 0; q < 8; q++) pf[tt][q] = (_Float16)s[tt >> 1][8 * (tt & 1) + q];
            }
            float ps[2] = {0.f, 0.f};
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    ps[q & 1] = __builtin_amdgcn_fdot2(half2v{pf[tt][2 * q], pf[tt][2 * q + 1]}, half2v{1, 1},
                                                       ps[q & 1], false);
            lsum += ps[0] + ps[1];
#pragma unroll
            for (int db = 0; db < DB; db++) {
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const half8 a = *(const half8 *)&sv[b][32 * db + l32][16 * tt + 8 * hf];
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[tt], o[db], 0, 0, 0);
                }
            }
        }
        if constexpr (!SPARSE) __builtin_amdgcn_s_setprio(0);
        if (e + 1 < nkt) store_tile(b ^ 1);
        __syncthreads();
    }

    const float l = lsum + __shfl_xor(lsum, 32);
    const float inv = 1.0f / l;
    const int slot = q0 + l32;
    int row = slot < n ? slot : -1;
    int tile = 0;
    if (SPARSE) {
        tile = slot / ATT_KT;
        row = (tile < sp.T && slot - tile * ATT_KT < sp.cnt[tile]) ? sp.gather[slot] : -1;
    }
    if (row >= 0) {
        float *orow = O + (size_t)row * o_ld + (size_t)h * HD;
        const float *crow = SPARSE && sp.coarse ? sp.coarse + ((size_t)h * sp.T + tile) * HD : nullptr;
        const float *grow_ = crow ? sp.gate + (size_t)row * o_ld + (size_t)h * HD : nullptr;
#pragma unroll
        for (int db = 0; db < DB; db++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = 32 * db + 8 * g + 4 * hf;
                f32x4 w;
#pragma unroll
                for (int q = 0; q < 4; q++) w[q] = o[db][4 * g + q] * inv;
                if (crow) {
                    const f32x4 cv = *(const f32x4 *)(crow + d), gv = *(const f32x4 *)(grow_ + d);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float t = cv[q] * gv[q];
                        w[q] = w[q] + t;
                    }
                }
                *(f32x4 *)(orow + d) = w;
            }
    }
}


// ---------------------------------------------------------------------------
// Video sparse attention (src/core/fh3_vsa.c:186-507).  The tile statistics
// are computed in the reference's exact order and roundings (one thread per
// output, products and sums rounded separately), so the tile scores -- and
// with them the top-k tile choice -- are bit-identical to the CPU's; the fine
// attention then runs on k_attn_fwd over each query tile's selected tiles.
// ---------------------------------------------------------------------------

// scores[h][i][j] = (sum_d qp[h][i][d] * kp[h][j][d], in order) * scale
template <int HD>
__global__ __launch_bounds__(256) void k_vsa_scores(const float *__restrict__ qp, const float *__restrict__ kp,
                                                    int T, float scale, float *__restrict__ sc) {
    __shared__ float qrow[HD];
    const int i = blockIdx.x, h = blockIdx.y;
    if (threadIdx.x < HD) qrow[threadIdx.x] = qp[((size_t)h * T + i) * HD + threadIdx.x];
    __syncthreads();
    for (int j = threadIdx.x; j < T; j += blockDim.x) {
        const float *kr = kp + ((size_t)h * T + j) * HD;
        float dot = 0.f;
        for (int d = 0; d < HD; d++) dot = dot + qrow[d] * kr[d];
        sc[((size_t)h * T + i) * T + j] = dot * scale;
    }
}

// The selection of query tile i as flags sel[j] (LDS): every tile for prefix
// query tiles or when all are kept; otherwise the prefix tiles and the kv
// video tiles of largest score, ties to the lower tile index (the order of
// the reference's qsort comparator, src/core/fh3_vsa.c:178-184).  The kv-th
// largest score is found by a 4-pass radix select on order-preserving keys.
__device__ void vsa_select_row(const float *__restrict__ srow, int T, int P, int kv, bool all, int i,
                               uint32_t *keys, uint8_t *sel, int *hist, int *scal) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if (i < P || all) {
        for (int j = tid; j < T; j += nt) sel[j] = 1;
        __syncthreads();
        return;
    }
    const int NV = T - P;
    for (int j = tid; j < T; j += nt) {
        sel[j] = j < P;
        if (j >= P) {
            float f = srow[j];
            f = f == 0.f ? 0.f : f;  // -0 ties with +0, as in the comparator
            const uint32_t u = __float_as_uint(f);
            keys[j - P] = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        }
    }
    uint32_t prefix = 0, mask = 0;
    int want = kv;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int b = tid; b < 256; b += nt) hist[b] = 0;
        __syncthreads();
        for (int j = tid; j < NV; j += nt)
            if ((keys[j] & mask) == prefix) atomicAdd(&hist[(keys[j] >> shift) & 255], 1);
        __syncthreads();
        if (tid == 0) {
            int above = 0, b = 255;
            for (; b > 0; b--) {
                if (above + hist[b] >= want) break;
                above += hist[b];
            }
            scal[0] = b;
            scal[1] = want - above;
        }
        __syncthreads();
        prefix |= (uint32_t)scal[0] << shift;
        mask |= 0xFFu << shift;
        want = scal[1];
        __syncthreads();
    }
    // keys above the threshold are in; of those equal to it, the first `want`
    // by tile index (a block-wide running count over j in order)
    if (tid == 0) scal[2] = 0;
    __syncthreads();
    for (int j0 = 0; j0 < NV; j0 += nt) {
        const int j = j0 + tid;
        const bool eq = j < NV && keys[j] == prefix;
        const uint64_t bal = __ballot(eq);
        const int wave = tid >> 6, lane = tid & 63;
        if (lane == 0) hist[wave] = __popcll(bal);
        __syncthreads();
        int before = scal[2];
        for (int w = 0; w < wave; w++) before += hist[w];
        before += __popcll(bal & ((lane ? (~0ull >> (64 - lane)) : 0ull)));
        if (j < NV) sel[P + j] = keys[j] > prefix || (eq && before < want);
        __syncthreads();
        if (tid == 0) {
            int tot = 0;
            for (int w = 0; w < (nt >> 6); w++) tot += hist[w];
            scal[2] += tot;
        }
        __syncthreads();
    }
}

// Union tile lists of query-tile pairs (2 qb, 2 qb + 1) for k_attn_fwd.
__global__ __launch_bounds__(256) void k_vsa_lists(const float *__restrict__ sc, int T, int P, int kv, int all,
                                                   int nqb, uint16_t *__restrict__ lists,
                                                   int *__restrict__ list_len) {
    extern __shared__ uint8_t smem[];
    uint32_t *keys = (uint32_t *)smem;                    // [T]
    uint8_t *sel0 = smem + (size_t)4 * T, *sel1 = sel0 + T;
    __shared__ int hist[256];
    __shared__ int scal[4];
    const int qb = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
    const int i0 = 2 * qb, i1 = 2 * qb + 1;
    vsa_select_row(sc + ((size_t)h * T + i0) * T, T, P, kv, all != 0, i0, keys, sel0, hist, scal);
    if (i1 < T) {
        vsa_select_row(sc + ((size_t)h * T + i1) * T, T, P, kv, all != 0, i1, keys, sel1, hist, scal);
    } else {
        for (int j = tid; j < T; j += nt) sel1[j] = 0;
        __syncthreads();
    }
    // stream compaction in tile order
    uint16_t *out = lists + ((size_t)h * nqb + qb) * T;
    if (tid == 0) scal[3] = 0;
    __syncthreads();
    for (int j0 = 0; j0 < T; j0 += nt) {
        const int j = j0 + tid;
        const int bits = j < T ? (sel0[j] ? 1 : 0) | (sel1[j] ? 2 : 0) : 0;
        const uint64_t bal = __ballot(bits != 0);
        const int wave = tid >> 6, lane = tid & 63;
        if (lane == 0) hist[wave] = __popcll(bal);
        __syncthreads();
        int at = scal[3];
        for (int w = 0; w < wave; w++) at += hist[w];
        at += __popcll(bal & ((lane ? (~0ull >> (64 - lane)) : 0ull)));
        if (bits) out[at] = (uint16_t)(j | (bits << 14));
        __syncthreads();
        if (tid == 0) {
            int tot = 0;
            for (int w = 0; w < (nt >> 6); w++) tot += hist[w];
            scal[3] += tot;
        }
        __syncthreads();
    }
    if (tid == 0) list_len[h * nqb + qb] = scal[3];
}

// Gated coarse branch: per (query tile i, head h) a softmax over all tile
// scores mixes the pooled v: coarse[h][i][d] = sum_j expf(s_j - max) / sum * vp[h][j][d].
template <int HD>
__global__ __launch_bounds__(HD) void k_vsa_coarse(const float *__restrict__ sc, const float *__restrict__ vp,
                                                   int T, float *__restrict__ coarse) {
    extern __shared__ float wsh[];  // [T] softmax weights
    __shared__ float red[HD / 64];
    __shared__ float bc[2];
    const int i = blockIdx.x, h = blockIdx.y, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    const float *srow = sc + ((size_t)h * T + i) * T;
    float mx = -1e30f;
    for (int j = d; j < T; j += HD) mx = fmaxf(mx, srow[j]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    if (d == 0) {
        float m = red[0];
        for (int w = 1; w < HD / 64; w++) m = fmaxf(m, red[w]);
        bc[0] = m;
    }
    __syncthreads();
    mx = bc[0];
    float sum = 0.f;
    for (int j = d; j < T; j += HD) {
        wsh[j] = expf(srow[j] - mx);
        sum += wsh[j];
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    __syncthreads();
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    if (d == 0) {
        float t = 0.f;
        for (int w = 0; w < HD / 64; w++) t += red[w];
        bc[1] = 1.0f / t;
    }
    __syncthreads();
    const float inv = bc[1];
    for (int j = d; j < T; j += HD) wsh[j] = wsh[j] * inv;
    __syncthreads();
    float acc = 0.f;
    const float *vcol = vp + (size_t)h * T * HD + d;
    for (int j = 0; j < T; j++) acc += wsh[j] * vcol[(size_t)j * HD];
    coarse[((size_t)h * T + i) * HD + d] = acc;
}

int64_t attn_pad_dense(int n, int hd) {
    const int64_t qb = ATT_QW * dense_nw(hd);
    return ((int64_t)n + qb - 1) / qb * qb;
}

template <int HD>
hipError_t attn_launch(const float *q, const float *k, const float *v, int64_t ld, int n, int heads,
                       const float *qn_w, const float *kn_w, float eps, const float *cosb, const float *sinb,
                       int rot, void *ws, float *o, int64_t o_ld, hipStream_t st) {
    const int n_pad = (int)attn_pad_dense(n, HD);
    _Float16 *Qp = (_Float16 *)ws;
    _Float16 *Kp = Qp + (size_t)heads * n_pad * HD;
    _Float16 *Vt = Kp + (size_t)heads * n_pad * HD;
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    hipLaunchKernelGGL(k_attn_prep<HD>, dim3(n_pad / ATT_PREP_T, heads), dim3(256), 0, st, q, k, v, ld, ld, n,
                       (const int *)nullptr, qn_w, kn_w, eps, cosb, sinb, rot, qscale, n_pad, Qp, Kp, Vt, Pool{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int NW = dense_nw(HD);
    const int blocks = heads * (n_pad / (ATT_QW * NW));
    hipLaunchKernelGGL((k_attn_fwd<HD, false, NW>), dim3(blocks), dim3(64 * NW), 0, st, Qp, Kp, Vt, n, n_pad, heads, o,
                       o_ld, Sparse{});
    return hipGetLastError();
}

}  // namespace

extern "C" int64_t fh3k_attn_pad(int n) { return ((int64_t)n + ATT_QB - 1) / ATT_QB * ATT_QB; }

extern "C" size_t fh3k_attn_ws_bytes(int n, int heads, int hd) {
    return (size_t)3 * heads * attn_pad_dense(n, hd) * hd * sizeof(_Float16);
}

extern "C" int fh3k_attn_head_dim_ok(int hd) { return hd == 64 || hd == 128; }

extern "C" hipError_t fh3k_attention(const float *q, const float *k, const float *v, int64_t ld, int n, int heads,
                                     int hd, const float *qn_w, const float *kn_w, float eps, const float *cosb,
                                     const float *sinb, int rot, void *ws, float *o, int64_t o_ld, hipStream_t st) {
    if (hd == 128) return attn_launch<128>(q, k, v, ld, n, heads, qn_w, kn_w, eps, cosb, sinb, rot, ws, o, o_ld, st);
    if (hd == 64) return attn_launch<64>(q, k, v, ld, n, heads, qn_w, kn_w, eps, cosb, sinb, rot, ws, o, o_ld, st);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Video sparse attention launchers
// ---------------------------------------------------------------------------
namespace {

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct VsaWs {
    _Float16 *Qp, *Kp, *Vt;
    float *qp, *kp, *vp, *sc, *coarse;
    uint16_t *lists;
    int *list_len;
    size_t bytes;
};

VsaWs vsa_ws(void *base, int T, int heads, int hd) {
    const int64_t n_pad = fh3k_attn_pad(ATT_KT * T);
    const int64_t nqb = n_pad / ATT_QB;
    char *p = (char *)base;
    VsaWs w;
    size_t at = 0;
    auto take = [&](size_t b) {
        char *r = p ? p + at : nullptr;
        at += align256(b);
        return r;
    };
    const size_t op = (size_t)heads * n_pad * hd * sizeof(_Float16);
    w.Qp = (_Float16 *)take(op);
    w.Kp = (_Float16 *)take(op);
    w.Vt = (_Float16 *)take(op);
    const size_t pool = (size_t)heads * T * hd * sizeof(float);
    w.qp = (float *)take(pool);
    w.kp = (float *)take(pool);
    w.vp = (float *)take(pool);
    w.coarse = (float *)take(pool);
    w.sc = (float *)take((size_t)heads * T * T * sizeof(float));
    w.lists = (uint16_t *)take((size_t)heads * nqb * T * sizeof(uint16_t));
    w.list_len = (int *)take((size_t)heads * nqb * sizeof(int));
    w.bytes = at;
    return w;
}

template <int HD>
hipError_t vsa_launch(const float *q, const float *k, const float *v, int64_t ld, int64_t ldv, const float *qn_w,
                      const float *kn_w, float eps, const float *cosb, const float *sinb, int rot, const float *gate,
                      float *o, int64_t o_ld, int heads, const float *inv, const int *gather, const int *cnt, int T,
                      int P, int kv, int all, float scale, void *ws, hipStream_t st) {
    const int n_pad = (int)fh3k_attn_pad(ATT_KT * T);
    const int nqb = n_pad / ATT_QB;
    VsaWs w = vsa_ws(ws, T, heads, HD);
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    Pool pl{inv, cnt, w.qp, w.kp, gate ? w.vp : nullptr, T};
    hipLaunchKernelGGL(k_attn_prep<HD>, dim3(n_pad / ATT_PREP_T, heads), dim3(256), 0, st, q, k, v, ld, ldv,
                       ATT_KT * T, gather, qn_w, kn_w, eps, cosb, sinb, rot, qscale, n_pad, w.Qp, w.Kp, w.Vt, pl);
    hipLaunchKernelGGL((k_vsa_scores<HD>), dim3(T, heads), dim3(256), 0, st, w.qp, w.kp, T, scale, w.sc);
    hipLaunchKernelGGL(k_vsa_lists, dim3(nqb, heads), dim3(256), (size_t)align256(6 * (size_t)T), st, w.sc, T, P, kv,
                       all, nqb, w.lists, w.list_len);
    if (gate)
        hipLaunchKernelGGL((k_vsa_coarse<HD>), dim3(T, heads), dim3(HD), (size_t)T * sizeof(float), st, w.sc, w.vp, T,
                           w.coarse);
    Sparse sp{w.lists, w.list_len, cnt, gather, gate ? w.coarse : nullptr, gate, T};
    hipLaunchKernelGGL((k_attn_fwd<HD, true, ATT_NW>), dim3(heads * nqb), dim3(64 * ATT_NW), 0, st, w.Qp, w.Kp, w.Vt,
                       ATT_KT * T, n_pad, heads, o, o_ld, sp);
    return hipGetLastError();
}

}  // namespace

extern "C" int fh3k_vsa_max_tiles(void) { return 4096; }

extern "C" size_t fh3k_vsa_ws_bytes(int T, int heads, int hd) { return vsa_ws(nullptr, T, heads, hd).bytes; }

extern "C" hipError_t fh3k_vsa_attention(const float *q, const float *k, const float *v, int64_t ld, int64_t ldv,
                                         const float *qn_w, const float *kn_w, float eps, const float *cosb,
                                         const float *sinb, int rot, const float *gate, float *o, int64_t o_ld,
                                         int heads, int hd, const float *inv, const int *gather, const int *cnt,
                                         int T, int P, int kv, int all, float scale, void *ws, hipStream_t st) {
    if (T <= 0 || T > fh3k_vsa_max_tiles()) return hipErrorInvalidValue;
    if (hd == 128)
        return vsa_launch<128>(q, k, v, ld, ldv, qn_w, kn_w, eps, cosb, sinb, rot, gate, o, o_ld, heads, inv, gather,
                               cnt, T, P, kv, all, scale, ws, st);
    if (hd == 64)
        return vsa_launch<64>(q, k, v, ld, ldv, qn_w, kn_w, eps, cosb, sinb, rot, gate, o, o_ld, heads, inv, gather,
                              cnt, T, P, kv, all, scale, ws, st);
    return hipErrorInvalidValue;
}
