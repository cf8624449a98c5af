// dfx_api.cpp — error reporting, device plumbing and the host-side weight repack
// of the C ABI (dfx.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "dfx.h"

static thread_local char g_err[1024] = "";

extern "C" void dfx_set_error(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char * dfx_last_error(void) { return g_err; }

#define HIP_TRY(call, what)                                                        \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) {                                                    \
            dfx_set_error("%s: %s", what, hipGetErrorString(e_));                  \
            return e_ == hipErrorOutOfMemory ? DFX_ERR_OOM : DFX_ERR_HIP;          \
        }                                                                          \
    } while (0)

extern "C" int dfx_device_count(int * n) {
    HIP_TRY(hipGetDeviceCount(n), "hipGetDeviceCount");
    return DFX_OK;
}
extern "C" int dfx_malloc(void ** ptr, size_t bytes) {
    HIP_TRY(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
    return DFX_OK;
}
extern "C" int dfx_free(void * ptr) {
    if (ptr) HIP_TRY(hipFree(ptr), "hipFree");
    return DFX_OK;
}
extern "C" int dfx_memcpy_h2d(void * dst, const void * src, size_t bytes, void * stream) {
    if (!bytes) return DFX_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpy H2D");
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return DFX_OK;
}
extern "C" int dfx_memcpy_d2h(void * dst, const void * src, size_t bytes, void * stream) {
    if (!bytes) return DFX_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpy D2H");
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return DFX_OK;
}
extern "C" int dfx_memcpy_d2d(void * dst, const void * src, size_t bytes, void * stream) {
    if (!bytes) return DFX_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpy D2D");
    return DFX_OK;
}
extern "C" int dfx_memset(void * dst, int value, size_t bytes, void * stream) {
    if (!bytes) return DFX_OK;
    HIP_TRY(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream), "hipMemsetAsync");
    return DFX_OK;
}
extern "C" int dfx_stream_create(void ** stream) {
    hipStream_t s;
    HIP_TRY(hipStreamCreate(&s), "hipStreamCreate");
    *stream = s;
    return DFX_OK;
}
extern "C" int dfx_stream_destroy(void * stream) {
    if (stream) HIP_TRY(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    return DFX_OK;
}
extern "C" int dfx_stream_sync(void * stream) {
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return DFX_OK;
}

struct dfx_timer_t { hipEvent_t a, b; };

extern "C" int dfx_timer_start(void ** timer, void * stream) {
    dfx_timer_t * t = new dfx_timer_t;
    if (hipEventCreate(&t->a) != hipSuccess || hipEventCreate(&t->b) != hipSuccess) {
        delete t;
        dfx_set_error("hipEventCreate failed");
        return DFX_ERR_HIP;
    }
    HIP_TRY(hipEventRecord(t->a, (hipStream_t)stream), "hipEventRecord");
    *timer = t;
    return DFX_OK;
}
extern "C" int dfx_timer_stop(void * timer, void * stream, float * ms) {
    dfx_timer_t * t = (dfx_timer_t *)timer;
    hipError_t e = hipEventRecord(t->b, (hipStream_t)stream);
    if (e == hipSuccess) e = hipEventSynchronize(t->b);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, t->a, t->b);
    (void)hipEventDestroy(t->a);
    (void)hipEventDestroy(t->b);
    delete t;
    if (e != hipSuccess) {
        dfx_set_error("timer: %s", hipGetErrorString(e));
        return DFX_ERR_HIP;
    }
    return DFX_OK;
}

// ---------------------------------------------------------------------------
// Device weight layout
// ---------------------------------------------------------------------------
extern "C" int dfx_device_type(int gguf_type) {
    switch (gguf_type) {
        case DFX_TYPE_Q4_K: case DFX_TYPE_Q6_K: case DFX_TYPE_Q8_0: case DFX_TYPE_F16: case DFX_TYPE_F32:
            return gguf_type;
    }
    return -1;
}

extern "C" int64_t dfx_device_row_bytes(int type, int64_t n_cols) {
    if (n_cols <= 0 || (n_cols % 256)) return -1;
    const int64_t nsb = n_cols / 256;
    switch (dfx_device_type(type)) {
        case DFX_TYPE_Q4_K: return nsb * 144;
        case DFX_TYPE_Q6_K: return nsb * 224;
        case DFX_TYPE_Q8_0: return nsb * 272;
        case DFX_TYPE_F16:  return n_cols * 2;
        case DFX_TYPE_F32:  return n_cols * 4;
    }
    return -1;
}

extern "C" int dfx_repack_rows(int gguf_type, const void * src, int64_t n_rows, int64_t n_cols, void * dst) {
    const int64_t drb = dfx_device_row_bytes(gguf_type, n_cols);
    if (drb < 0 || n_rows < 0) {
        dfx_set_error("dfx_repack_rows: type %d with %lld columns has no device layout", gguf_type, (long long)n_cols);
        return DFX_ERR_UNSUPPORTED;
    }
    const int64_t nsb = n_cols / 256;
    const uint8_t * s = (const uint8_t *)src;
    uint8_t * d = (uint8_t *)dst;
    switch (gguf_type) {
        case DFX_TYPE_Q4_K:
        case DFX_TYPE_F16:
        case DFX_TYPE_F32:
            memcpy(d, s, (size_t)(drb * n_rows));
            return DFX_OK;
        case DFX_TYPE_Q6_K:
            for (int64_t b = 0; b < n_rows * nsb; b++) {
                memcpy(d + b * 224, s + b * 210, 210);
                memset(d + b * 224 + 210, 0, 14);
            }
            return DFX_OK;
        case DFX_TYPE_Q8_0:
            // eight 34-byte {d, qs[32]} blocks -> {d[8], qs[8][32]}
            for (int64_t b = 0; b < n_rows * nsb; b++) {
                const uint8_t * sb = s + b * 272;
                uint8_t * db = d + b * 272;
                for (int j = 0; j < 8; j++) {
                    memcpy(db + 2 * j, sb + 34 * j, 2);
                    memcpy(db + 16 + 32 * j, sb + 34 * j + 2, 32);
                }
            }
            return DFX_OK;
    }
    dfx_set_error("dfx_repack_rows: unsupported type %d", gguf_type);
    return DFX_ERR_UNSUPPORTED;
}
