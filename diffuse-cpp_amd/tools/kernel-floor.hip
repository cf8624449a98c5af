// kernel-floor — what one kernel boundary costs on this GPU.
//   kernel-floor [launches=1000]
// Back-to-back launches of a kernel that writes `bytes` (grid-stride, at most 2048
// workgroups of 256), on one stream: once launched one by one, once captured into a HIP
// graph and replayed.  HIP events around the batch give the time per kernel.  The sizes run
// from 256 bytes (the floor: launch, wave start-up and the end-of-kernel release) to 16 MB
// (write bandwidth).  Prints one JSON line per size.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "kernel-floor: %s: %s\n", #x, hipGetErrorString(e_));      \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

__global__ void k_fill(float * p, long n, float v) {
    const long s = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += s) p[i] = v;
}

int main(int argc, char ** argv) {
    const int launches = argc > 1 ? atoi(argv[1]) : 1000;
    if (launches < 10 || launches > 100000) {
        fprintf(stderr, "Usage: %s [launches in 10..100000]\n", argv[0]);
        return 2;
    }
    const long max_n = 1L << 22;   // floats per slot: 16 MB
    const long sizes[] = {64, 1L << 18, 1L << 20, max_n};
    float * buf = nullptr;
    CK(hipMalloc(&buf, 2 * max_n * sizeof(float)));   // two slots: consecutive kernels alternate
    hipStream_t st;
    CK(hipStreamCreate(&st));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    for (const long n : sizes) {
        const int grid = (int)std::min<long>((n + 255) / 256, 2048);
        auto enqueue = [&](int count) {
            for (int i = 0; i < count; i++)
                hipLaunchKernelGGL(k_fill, dim3(grid), dim3(256), 0, st, buf + (i & 1) * max_n, n, (float)i);
        };
        enqueue(20);   // warm-up
        CK(hipGetLastError());
        CK(hipStreamSynchronize(st));
        CK(hipEventRecord(a, st));
        enqueue(launches);
        CK(hipEventRecord(b, st));
        CK(hipEventSynchronize(b));
        float ms_direct = 0.0f;
        CK(hipEventElapsedTime(&ms_direct, a, b));

        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        enqueue(launches);
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, st));   // first replay uploads the graph
        CK(hipStreamSynchronize(st));
        CK(hipEventRecord(a, st));
        CK(hipGraphLaunch(ge, st));
        CK(hipEventRecord(b, st));
        CK(hipEventSynchronize(b));
        float ms_graph = 0.0f;
        CK(hipEventElapsedTime(&ms_graph, a, b));
        printf("{\"bytes\": %ld, \"workgroups\": %d, \"launches\": %d, \"us_per_kernel_direct\": %.3f, "
               "\"us_per_kernel_graph\": %.3f}\n",
               n * (long)sizeof(float), grid, launches, 1000.0 * ms_direct / launches, 1000.0 * ms_graph / launches);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    CK(hipFree(buf));
    return 0;
}
