// fh3_mfma_peak.hip -- matrix-core calibration for the rooflines of the
// product kernels.
//
// Every SIMD of the chip issues back-to-back MFMAs of one kind (the kinds the
// kernels use: fp16 32x32x16 in k_gemm and the attention, fp16 16x16x32 in
// k_skinny / k_sweep, int8 16x16x64 in k_gemv8; bf16 32x32x16 for the bf16
// figure), on register operands, in independent accumulator chains (each
// chain's next MFMA issues 128 or more clocks after its last), with no memory
// traffic but one store per wavefront at the end.  One workgroup per CU (its
// LDS request leaves room for no second one), 4 or 8 wavefronts.  Prints the
// rate of each kind against the published dense peak (fp16 / bf16 2.5 PFLOP/s,
// int8 5.0 POP/s, both at a 2.4 GHz clock) and the clock the rate implies at
// a fully busy matrix pipe: measured / peak * 2.4 GHz.
//
//   fasth3inc_amd/lib/fh3_mfma_peak [iterations]   (default 20000 per launch)
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

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

struct Kind {
    const char *name;
    double ops_per_inst;   // 2 * m * n * k
    int chains;            // MFMAs per loop iteration
    double peak;           // published dense peak, ops/s
    void (*kern)(int, float *);
};

int main(int argc, char **argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 20000;
    if (iters < 1 || iters > 10000000) {
        fprintf(stderr, "iterations must be in 1..10000000\n");
        return 2;
    }
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
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
    return 0;
}
