// fh3_calib.hip -- calibration of the rooflines the product kernels are
// measured against: what the matrix cores and HBM sustain on this GPU.
//
// mfma: every SIMD of the chip issues back-to-back MFMAs of one kind (the
// kinds the kernels use: fp16 32x32x16 in k_gemm and the attention, fp16
// 16x16x32 in k_skinny / k_sweep, int8 16x16x64 in k_gemv8; bf16 32x32x16 for
// the bf16 figure), on register operands, in independent accumulator chains
// (each chain's next MFMA issues 128 or more clocks after its last), with no
// memory traffic but one store per wavefront at the end.  One workgroup per
// CU (its LDS request leaves room for no second one), 4 or 8 wavefronts.
// Prints the rate of each kind against the published dense peak (fp16 / bf16
// 2.5 PFLOP/s, int8 5.0 POP/s, both at a 2.4 GHz clock) and the clock the
// rate implies at a fully busy matrix pipe: measured / peak * 2.4 GHz.
//
// hbm: one launch reads a contiguous run of S bytes with 16-byte loads and
// keeps nothing (a load-only stream, two load forms, three grid sizes; the
// best of them is reported), S = the Q4_K weights of the GEMV shapes
// (5120 x 5120: 14,745,600 B; 17408 x 5120: 50,135,040 B), 256 MiB and 1 GiB;
// successive launches read successive runs of a 2 GiB buffer, so no launch
// finds its bytes in the 256 MB Infinity Cache.  Prints the mean time per
// launch and the rate against the published 8 TB/s: the shortest time one
// launch needs to stream a weight matrix of that size.
//
//   fasth3inc_amd/lib/fh3_calib [mfma|hbm|gemv|all] [iterations]
//   (gemv: the hbm mode at the two GEMV weight sizes only; iterations: MFMA
//   loop trips per launch, default 20000)
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

enum { K_F16_32 = 0, K_F16_16 = 1, K_BF16_32 = 2, K_I8_16 = 3, NKIND = 4 };

#define CK(x)                                                                                  \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

// Sum of the accumulators, so that none of the chains is dead code.
template <typename V, int N, int C>
__device__ __forceinline__ float acc_sum(const V (&acc)[C]) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int i = 0; i < N; i++) s += (float)acc[c][i];
    return s;
}

template <int KIND>
__global__ __launch_bounds__(512) void k_mfma_loop(int iters, float *__restrict__ out) {
    const int lane = (int)threadIdx.x & 63;
    float s;
    if constexpr (KIND == K_F16_32 || KIND == K_F16_16) {
        half8 a, b;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a[i] = (_Float16)((float)(lane + i) * 0x1p-10f);
            b[i] = (_Float16)((float)(lane - i) * 0x1p-10f);
        }
        if constexpr (KIND == K_F16_32) {
            f32x16 acc[4] = {};
            for (int it = 0; it < iters; it++)
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
            s = acc_sum<f32x16, 16>(acc);
        } else {
            f32x4 acc[8] = {};
            for (int it = 0; it < iters; it++)
#pragma unroll
                for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
            s = acc_sum<f32x4, 4>(acc);
        }
    } else if constexpr (KIND == K_BF16_32) {
        bf16x8 a, b;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a[i] = (__bf16)((float)(lane + i) * 0x1p-10f);
            b[i] = (__bf16)((float)(lane - i) * 0x1p-10f);
        }
        f32x16 acc[4] = {};
        for (int it = 0; it < iters; it++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
        s = acc_sum<f32x16, 16>(acc);
    } else {
        const i32x4 a = {lane, lane + 1, lane + 2, lane + 3}, b = {3 - lane, 2 - lane, 1 - lane, -lane};
        i32x4 acc[8] = {};
        for (int it = 0; it < iters; it++)
#pragma unroll
            for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
        s = acc_sum<i32x4, 4>(acc);
    }
    // one value per wavefront: out holds gridDim.x * 8 floats
    if (lane == 0) out[blockIdx.x * 8 + (threadIdx.x >> 6)] = s;
}

// Load-only stream over n16 16-byte pieces, grid-stride.  U = 8: eight
// loads per trip, each predicated on its index, all issued before the trip's
// one wait; U = 1: one load per trip (the wavefronts pace the requests).  The
// XOR of everything read is stored only if it equals a value the zero-filled
// buffer cannot give (so the loads are not dead code).
template <int U>
__global__ __launch_bounds__(512) void k_hbm_stream(const u32x4 *__restrict__ p, size_t n16, u32x4 *__restrict__ out) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const u32x4 z = {0u, 0u, 0u, 0u};
    u32x4 acc = z;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = i + u * stride < n16 ? p[i + u * stride] : z;
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u];
    }
    if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u) out[0] = acc;
}

struct Kind {
    const char *name;
    double ops_per_inst;   // 2 * m * n * k
    int chains;            // MFMAs per loop iteration
    double peak;           // published dense peak, ops/s
    void (*kern)(int, float *);
};

static void run_mfma(const hipDeviceProp_t &prop, int iters) {
    const int cus = prop.multiProcessorCount;
    // more than half the CU's LDS: one workgroup per CU
    const size_t lds = prop.sharedMemPerMultiprocessor / 2 + 1024;
    const Kind kinds[NKIND] = {
        {"fp16 v_mfma_f32_32x32x16_f16", 2.0 * 32 * 32 * 16, 4, 2.5e15, k_mfma_loop<K_F16_32>},
        {"fp16 v_mfma_f32_16x16x32_f16", 2.0 * 16 * 16 * 32, 8, 2.5e15, k_mfma_loop<K_F16_16>},
        {"bf16 v_mfma_f32_32x32x16_bf16", 2.0 * 32 * 32 * 16, 4, 2.5e15, k_mfma_loop<K_BF16_32>},
        {"int8 v_mfma_i32_16x16x64_i8", 2.0 * 16 * 16 * 64, 8, 5.0e15, k_mfma_loop<K_I8_16>},
    };
    float *out;
    CK(hipMalloc(&out, (size_t)cus * 8 * sizeof(float)));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    printf("%s: %d CUs, %zu B of LDS per workgroup, %d iterations per launch\n", prop.gcnArchName, cus, lds, iters);
    for (int k = 0; k < NKIND; k++) {
        CK(hipFuncSetAttribute((const void *)kinds[k].kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        for (int threads : {256, 512}) {
            auto launch = [&]() {
                hipLaunchKernelGGL(kinds[k].kern, dim3((unsigned)cus), dim3((unsigned)threads), lds, 0, iters, out);
            };
            launch();  // warm-up (clock ramp)
            CK(hipGetLastError());
            CK(hipDeviceSynchronize());
            const int reps = 10;
            CK(hipEventRecord(a, 0));
            for (int r = 0; r < reps; r++) launch();
            CK(hipEventRecord(b, 0));
            CK(hipEventSynchronize(b));
            CK(hipGetLastError());
            float ms = 0.f;
            CK(hipEventElapsedTime(&ms, a, b));
            const double sec = (double)ms * 1e-3 / reps;
            const double ops = kinds[k].ops_per_inst * kinds[k].chains * (double)iters * (threads / 64) * cus;
            const double rate = ops / sec;
            printf("%-30s %4d threads: %8.3f ms per launch, %7.1f T%s/s, %.3f of the %.1f P peak, implied clock "
                   "%.2f GHz\n",
                   kinds[k].name, threads, sec * 1e3, rate * 1e-12, k == K_I8_16 ? "OP" : "FLOP",
                   rate / kinds[k].peak, kinds[k].peak * 1e-15, rate / kinds[k].peak * 2.4);
        }
    }
    CK(hipFree(out));
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
}

static void run_hbm(const hipDeviceProp_t &prop, bool gemv_only) {
    const int cus = prop.multiProcessorCount;
    const size_t region = (size_t)2 << 30;
    uint8_t *buf;
    u32x4 *out;
    CK(hipMalloc(&buf, region));
    CK(hipMemset(buf, 0, region));
    CK(hipMalloc(&out, sizeof(u32x4)));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    const size_t all_sizes[] = {14745600, 50135040, (size_t)256 << 20, (size_t)1 << 30};
    const int nsizes = gemv_only ? 2 : 4;
    printf("%s: %d CUs, load-only stream, runs rotated over %zu MiB\n", prop.gcnArchName, cus, region >> 20);
    for (int si = 0; si < nsizes; si++) {
        const size_t bytes = all_sizes[si];
        // successive runs at successive 4 KiB-aligned offsets, every run inside the region
        const size_t step = (bytes + 4095) & ~(size_t)4095;
        const size_t nrun = region / step;
        double best = 1e30;
        for (int u : {8, 1})
            for (int wpc : {1, 2, 4}) {
                const unsigned grid = (unsigned)(cus * wpc);
                size_t run = 0;
                auto launch = [&]() {
                    const u32x4 *p = (const u32x4 *)(buf + (run % nrun) * step);
                    run++;
                    if (u == 8)
                        hipLaunchKernelGGL(k_hbm_stream<8>, dim3(grid), dim3(512), 0, 0, p, bytes / 16, out);
                    else
                        hipLaunchKernelGGL(k_hbm_stream<1>, dim3(grid), dim3(512), 0, 0, p, bytes / 16, out);
                };
                launch();
                CK(hipGetLastError());
                CK(hipDeviceSynchronize());
                const int reps = bytes >= ((size_t)256 << 20) ? 8 : 40;
                CK(hipEventRecord(a, 0));
                for (int r = 0; r < reps; r++) launch();
                CK(hipEventRecord(b, 0));
                CK(hipEventSynchronize(b));
                CK(hipGetLastError());
                float ms = 0.f;
                CK(hipEventElapsedTime(&ms, a, b));
                const double sec = (double)ms * 1e-3 / reps;
                best = sec < best ? sec : best;
                printf("%11zu B, %d load%s per trip, %4u workgroups of 512: %9.2f us per launch, %7.1f GB/s, %.3f of "
                       "8 TB/s\n",
                       bytes, u, u > 1 ? "s" : " ", grid, sec * 1e6, bytes / sec * 1e-9, bytes / sec / 8e12);
            }
        printf("%11zu B best: %9.2f us per launch, %.3f of 8 TB/s\n", bytes, best * 1e6, bytes / best / 8e12);
    }
    CK(hipFree(buf));
    CK(hipFree(out));
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
}

int main(int argc, char **argv) {
    const char *mode = argc > 1 ? argv[1] : "all";
    const int iters = argc > 2 ? atoi(argv[2]) : 20000;
    const bool g = !strcmp(mode, "gemv");
    const bool m = !strcmp(mode, "mfma") || !strcmp(mode, "all"), h = !strcmp(mode, "hbm") || !strcmp(mode, "all");
    if ((!m && !h && !g) || iters < 1 || iters > 10000000) {
        fprintf(stderr, "usage: fh3_calib [mfma|hbm|gemv|all] [iterations 1..10000000]\n");
        return 2;
    }
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    if (m) run_mfma(prop, iters);
    if (h || g) run_hbm(prop, g);
    return 0;
}
