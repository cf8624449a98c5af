// k_attn.hip — NEOX RoPE + KV-cache store, and bidirectional attention.
//
// The inter-step cache lives in HBM as kc/vc[pos][n_head_kv][head_dim] f32 per
// layer.  The reference keeps it expanded to n_head (src/diffuse-cache.h:23-26)
// and concatenates [cached ‖ active] keys (src/diffuse-graph.cpp:524-525); here the
// active rows are scattered into the cache first and every query attends over the
// cache in position order.  Softmax without a mask is invariant to key order, and
// the GQA repeat (src/diffuse-graph.cpp:84-95) is the index h / n_rep.
#include "dfx_device.h"

#include <algorithm>

// One thread per (row, head of Q|K|V, rotation pair).
__global__ void k_rope_store(const float * __restrict__ qkv, const int32_t * __restrict__ pos, int64_t M, int H,
                             int Hkv, int hd, const float * __restrict__ tab, float * __restrict__ q_out,
                             float * __restrict__ kc, float * __restrict__ vc) {
#pragma clang fp contract(off)
    const int half = hd / 2, heads = H + 2 * Hkv;
    const int64_t total = M * heads * half;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % half);
        const int64_t t = idx / half;
        const int hh = (int)(t % heads);
        const int64_t m = t / heads;
        const float * src = qkv + m * heads * hd + (int64_t)hh * hd;
        const int p = pos[m];
        const float x0 = src[i], x1 = src[i + half];
        if (hh < H + Hkv) {
            // ggml_rope_ext NEOX: rotate (i, i + n_dims/2) by theta_i(p)
            const float c = tab[((int64_t)p * half + i) * 2 + 0];
            const float s = tab[((int64_t)p * half + i) * 2 + 1];
            const float y0 = x0 * c - x1 * s;
            const float y1 = x0 * s + x1 * c;
            float * dst = (hh < H) ? q_out + (m * H + hh) * hd
                                   : kc + ((int64_t)p * Hkv + (hh - H)) * hd;
            dst[i] = y0;
            dst[i + half] = y1;
        } else {
            float * dst = vc + ((int64_t)p * Hkv + (hh - H - Hkv)) * hd;
            dst[i] = x0;
            dst[i + half] = x1;
        }
    }
}

// Attention for TQ query rows of one head per workgroup (256 threads).  The whole
// score row of every query (n_keys floats) is kept in LDS so the softmax follows
// the reference op for op (src/diffuse-graph.cpp:107-114 with GGML soft_max):
//   s = dot(k, q) * (1/sqrtf(hd));  max;  e = exp(s - max);  sum in double;
//   p = e * (float)(1/sum);  out = sum_n v_n * p_n.
// Dot products and the P.V sums add float products in double and round once, so
// the result does not depend on the summation order (the CPU path adds in its own
// SIMD order); exp is correctly rounded.
template <int HD, int TQ>
__global__ void __launch_bounds__(256) k_attention(const float * __restrict__ q, const float * __restrict__ kc,
                                                   const float * __restrict__ vc, int M, int n_keys, int H,
                                                   int Hkv, float * __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ float smem[];
    float * Qs = smem;                 // [TQ][HD]
    float * S = smem + TQ * HD;        // [TQ][n_keys]
    const int h = blockIdx.y, kvh = h / (H / Hkv);
    const int q0 = blockIdx.x * TQ;
    const int nq = min(TQ, M - q0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float scale = 1.0f / sqrtf((float)HD);

    for (int i = tid; i < TQ * HD; i += 256) {
        const int r = i / HD, j = i - r * HD;
        Qs[i] = (r < nq) ? q[((int64_t)(q0 + r) * H + h) * HD + j] : 0.0f;
    }
    __syncthreads();

    // scores: thread per key, HD in slices of 16
    for (int n = tid; n < n_keys; n += 256) {
        const float * kr = kc + ((int64_t)n * Hkv + kvh) * HD;
        double acc[TQ];
#pragma unroll
        for (int r = 0; r < TQ; r++) acc[r] = 0.0;
        for (int d0 = 0; d0 < HD; d0 += 16) {
            float kv[16];
#pragma unroll
            for (int j = 0; j < 16; j += 4) {
                const float4 t = *(const float4 *)(kr + d0 + j);
                kv[j] = t.x; kv[j + 1] = t.y; kv[j + 2] = t.z; kv[j + 3] = t.w;
            }
#pragma unroll
            for (int r = 0; r < TQ; r++) {
                double a = acc[r];
#pragma unroll
                for (int j = 0; j < 16; j++) a += (double)(kv[j] * Qs[r * HD + d0 + j]);
                acc[r] = a;
            }
        }
#pragma unroll
        for (int r = 0; r < TQ; r++) S[r * n_keys + n] = (float)acc[r] * scale;
    }
    __syncthreads();

    // softmax: wave per row
    for (int r = wv; r < nq; r += 4) {
        float * sr = S + r * n_keys;
        float mx = -INFINITY;
        for (int n = lane; n < n_keys; n += 64) mx = fmaxf(mx, sr[n]);
        mx = wave_max(mx);
        double sum = 0.0;
        for (int n = lane; n < n_keys; n += 64) {
            const float e = (float)exp((double)(sr[n] - mx));
            sr[n] = e;
            sum += (double)e;
        }
        sum = wave_sum_d(sum);
        const float inv = (float)(1.0 / sum);
        for (int n = lane; n < n_keys; n += 64) sr[n] = sr[n] * inv;
    }
    __syncthreads();

    // out = P V: thread per (output column j, group of query rows)
    constexpr int G = 256 / HD;
    constexpr int RP = (TQ + G - 1) / G;      // query rows per thread
    const int j = tid % HD, g = tid / HD;
    const int r0 = g * RP;
    if (r0 >= TQ) return;
    double acc[RP];
#pragma unroll
    for (int r = 0; r < RP; r++) acc[r] = 0.0;
    for (int n = 0; n < n_keys; n++) {
        const float v = vc[((int64_t)n * Hkv + kvh) * HD + j];
#pragma unroll
        for (int r = 0; r < RP; r++) acc[r] += (double)(v * S[(r0 + r) * n_keys + n]);
    }
#pragma unroll
    for (int r = 0; r < RP; r++)
        if (r0 + r < nq) out[(int64_t)(q0 + r0 + r) * H * HD + (int64_t)h * HD + j] = (float)acc[r];
}

extern "C" int dfx_rope_store(const float * qkv, const int32_t * pos, int64_t M, int H, int Hkv, int hd,
                              const float * tab, float * q_out, float * kc, float * vc, void * stream) {
    if (M < 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || (hd & 1)) {
        dfx_set_error("dfx_rope_store: bad shape M=%lld H=%d Hkv=%d hd=%d", (long long)M, H, Hkv, hd);
        return DFX_ERR_ARG;
    }
    if (M == 0) return DFX_OK;
    const int64_t total = M * (H + 2 * Hkv) * (hd / 2);
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_rope_store, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, qkv, pos, M, H, Hkv,
                       hd, tab, q_out, kc, vc);
    DFX_CHECK_LAUNCH("dfx_rope_store");
    return DFX_OK;
}

#define ATTN_LDS_MAX (64 * 1024)

extern "C" int dfx_attention(const float * q, const float * kc, const float * vc, int64_t M, int64_t n_keys,
                             int H, int Hkv, int hd, float * out, void * stream) {
    if (M < 0 || n_keys <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128)) {
        dfx_set_error("dfx_attention: unsupported shape M=%lld keys=%lld H=%d Hkv=%d hd=%d", (long long)M,
                      (long long)n_keys, H, Hkv, hd);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    int TQ = 32;
    while (TQ > 1 && (size_t)TQ * (hd + n_keys) * sizeof(float) > ATTN_LDS_MAX) TQ >>= 1;
    const size_t lds = (size_t)TQ * (hd + n_keys) * sizeof(float);
    if (lds > ATTN_LDS_MAX) {
        dfx_set_error("dfx_attention: %lld keys exceed the LDS score row", (long long)n_keys);
        return DFX_ERR_UNSUPPORTED;
    }
    dim3 grid((unsigned)((M + TQ - 1) / TQ), (unsigned)H);
    hipStream_t st = (hipStream_t)stream;
#define ATTN_CASE(HD_, TQ_)                                                                              \
    if (hd == HD_ && TQ == TQ_)                                                                          \
        hipLaunchKernelGGL((k_attention<HD_, TQ_>), grid, dim3(256), lds, st, q, kc, vc, (int)M, (int)n_keys, \
                           H, Hkv, out);
    ATTN_CASE(128, 32) ATTN_CASE(128, 16) ATTN_CASE(128, 8) ATTN_CASE(128, 4) ATTN_CASE(128, 2) ATTN_CASE(128, 1)
    ATTN_CASE(64, 32) ATTN_CASE(64, 16) ATTN_CASE(64, 8) ATTN_CASE(64, 4) ATTN_CASE(64, 2) ATTN_CASE(64, 1)
#undef ATTN_CASE
    DFX_CHECK_LAUNCH("dfx_attention");
    return DFX_OK;
}
