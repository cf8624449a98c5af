// mfma-rate — the dense f16 matrix-core rate this GPU sustains, for the roofline's peak.
//   mfma-rate [iterations=20000]
// Every wave issues back-to-back v_mfma_f32_32x32x16_f16 on four independent accumulators
// (no loads, no other work), four waves per workgroup (one per SIMD).  Two grids are timed
// with HIP events: one workgroup (a single CU, the rate at the clock a lightly loaded chip
// holds) and 2 x CUs workgroups (every SIMD busy, the clock under full matrix-core load).
// Prints one JSON line: TFLOP/s of each and their ratio.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) k_mfma_rate(float * out, int iters) {
    const float s = 1.0f / 1024.0f;
    half8 a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)(s * (float)((threadIdx.x + i) & 7));
        b[i] = (_Float16)(s * (float)((threadIdx.x * 3 + i) & 7));
    }
    float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    float t = 0.0f;
    for (int r = 0; r < 16; r++) t += c0[r] + c1[r] + c2[r] + c3[r];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = t;
}

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "mfma-rate: %s: %s\n", #x, hipGetErrorString(e_));         \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

static int timed(int wgs, int iters, float * out, double * tflops) {
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    hipLaunchKernelGGL(k_mfma_rate, dim3(wgs), dim3(256), 0, 0, out, iters / 10);   // warm-up
    CK(hipGetLastError());
    CK(hipEventRecord(a, 0));
    hipLaunchKernelGGL(k_mfma_rate, dim3(wgs), dim3(256), 0, 0, out, iters);
    CK(hipGetLastError());
    CK(hipEventRecord(b, 0));
    CK(hipEventSynchronize(b));
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, a, b));
    const double flop = 2.0 * 32 * 32 * 16 * 4.0 * iters * 4.0 * wgs;   // 4 MFMAs x 4 waves per iteration
    *tflops = flop / (ms * 1e-3) / 1e12;
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
    return 0;
}

int main(int argc, char ** argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 20000;
    if (iters < 10 || iters > 10000000) {
        fprintf(stderr, "Usage: %s [iterations in 10..10000000]\n", argv[0]);
        return 1;
    }
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int full = 2 * cus;
    float * out = nullptr;
    CK(hipMalloc(&out, (size_t)full * 256 * sizeof(float)));
    double one = 0.0, all = 0.0;
    if (timed(1, iters, out, &one) || timed(full, iters, out, &all)) return 1;
    CK(hipFree(out));
    printf("{\"cus\": %d, \"iterations\": %d, \"one_cu_tflops\": %.2f, \"one_cu_scaled_to_chip_tflops\": %.1f, "
           "\"all_cus_tflops\": %.1f, \"all_over_one_scaled\": %.4f}\n",
           cus, iters, one, one * cus, all, all / (one * cus));
    return 0;
}
