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

// Both attention kernels follow the reference op for op (src/diffuse-graph.cpp:107-114
// with GGML soft_max):
//   s = dot(k, q) * (1/sqrtf(hd));  max;  e = exp(s - max);  sum in double;
//   p = e * (float)(1/sum);  out = sum_n v_n * p_n.
// f32 x f32 products are exact in f64; the dot products and the P.V sums are
// accumulated in f64 and rounded to float once, so the float result does not
// depend on the summation order.  exp is correctly rounded.

typedef double double4v __attribute__((ext_vector_type(4)));

// v_mfma_f64_16x16x4f64: D[16][16] += A[16][4] B[4][16].
// Lane l supplies A[l%16][l/16] and B[l/16][l%16]; it holds D[l/16 + 4i][l%16], i < 4.
__device__ __forceinline__ double4v mfma_f64(double a, double b, double4v c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Matrix-core attention: one head, RT tiles of 16 query rows per workgroup (4 waves).
// Phase 1: S = Q K^T on the f64 MFMA, each wave taking key tiles of 16 (two at a time);
// a reduction step of 16 head dims is split so that lane group g = l/16 supplies dims
// 16s+4g+c to MFMA c (c < 4): one float4 load per lane per operand and step.
// Phase 2: softmax, one wave per row, scores resident in LDS.
// Phase 3: O = P V on the f64 MFMA; each wave owns head-dim column tiles, keys are
// the reduction (keys 16s+4g+c to MFMA c, the same split).
template <int HD, int RT>
__global__ void __launch_bounds__(256) k_attn_mfma(const float * __restrict__ q, const float * __restrict__ kc,
                                                   const float * __restrict__ vc, int M, int n_keys, int H, int Hkv,
                                                   int sstride, float * __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ float S[];       // [RT*16][sstride] scores, then probabilities
    constexpr int SS = HD / 16;        // reduction steps of 16 head dims
    constexpr int CT = HD / 16 / 4;    // phase-3 column tiles per wave (HD=128: 2, HD=64: 1)
    const int h = blockIdx.y, kvh = h / (H / Hkv);
    const int q0 = blockIdx.x * RT * 16;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int64_t kvstride = (int64_t)Hkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int ntiles = (n_keys + 15) >> 4;
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

    // ---- phase 1
    float4 qf[RT][SS];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int row = q0 + 16 * rt + li;
        const float * qr = q + ((int64_t)row * H + h) * HD + 4 * lg;
#pragma unroll
        for (int s = 0; s < SS; s++) qf[rt][s] = (row < M) ? *(const float4 *)(qr + 16 * s) : zero4;
    }
    for (int t0 = wv; t0 < ntiles; t0 += 8) {
        const int t1 = t0 + 4;
        const bool has1 = t1 < ntiles;
        const int n0 = 16 * t0 + li, n1 = 16 * t1 + li;
        const float * k0 = kc + (int64_t)n0 * kvstride + (int64_t)kvh * HD + 4 * lg;
        const float * k1 = kc + (int64_t)n1 * kvstride + (int64_t)kvh * HD + 4 * lg;
        float4 kf0[SS], kf1[SS];
#pragma unroll
        for (int s = 0; s < SS; s++) {
            kf0[s] = (n0 < n_keys) ? *(const float4 *)(k0 + 16 * s) : zero4;
            kf1[s] = (has1 && n1 < n_keys) ? *(const float4 *)(k1 + 16 * s) : zero4;
        }
        double4v a0[RT], a1[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) { a0[rt] = 0.0; a1[rt] = 0.0; }
#pragma unroll
        for (int s = 0; s < SS; s++) {
            const float kb0[4] = {kf0[s].x, kf0[s].y, kf0[s].z, kf0[s].w};
            const float kb1[4] = {kf1[s].x, kf1[s].y, kf1[s].z, kf1[s].w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const double b0 = (double)kb0[c], b1 = (double)kb1[c];
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const float qa[4] = {qf[rt][s].x, qf[rt][s].y, qf[rt][s].z, qf[rt][s].w};
                    const double a = (double)qa[c];
                    a0[rt] = mfma_f64(a, b0, a0[rt]);
                    a1[rt] = mfma_f64(a, b1, a1[rt]);
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 16 * rt + lg + 4 * i;
                S[r * sstride + 16 * t0 + li] = (float)a0[rt][i] * scale;
                if (has1) S[r * sstride + 16 * t1 + li] = (float)a1[rt][i] * scale;
            }
        }
    }
    __syncthreads();

    // ---- phase 2
    for (int r = wv; r < RT * 16; r += 4) {
        float * sr = S + r * sstride;
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
        for (int n = n_keys + lane; n < 16 * ntiles; n += 64) sr[n] = 0.0f;
    }
    __syncthreads();

    // ---- phase 3
    double4v o[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) o[rt][ct] = 0.0;
    const float * vb = vc + (int64_t)kvh * HD + 16 * wv + li;     // column tile wv (+4 per ct)
    for (int s = 0; s < ntiles; s++) {
        float4 pf[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) pf[rt] = *(const float4 *)(S + (16 * rt + li) * sstride + 16 * s + 4 * lg);
        float vf[CT][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int n = 16 * s + 4 * lg + c;
#pragma unroll
            for (int ct = 0; ct < CT; ct++) vf[ct][c] = (n < n_keys) ? vb[(int64_t)n * kvstride + 64 * ct] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const float pa[4] = {pf[rt].x, pf[rt].y, pf[rt].z, pf[rt].w};
                const double a = (double)pa[c];
#pragma unroll
                for (int ct = 0; ct < CT; ct++) o[rt][ct] = mfma_f64(a, (double)vf[ct][c], o[rt][ct]);
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = q0 + 16 * rt + lg + 4 * i;
            if (row >= M) continue;
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                out[(int64_t)row * H * HD + (int64_t)h * HD + 16 * wv + 64 * ct + li] = (float)o[rt][ct][i];
        }
}

// VALU form for key counts whose score rows do not fit the matrix-core kernel's LDS:
// TQ query rows of one head per workgroup (256 threads), full score rows in LDS.
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
                for (int j = 0; j < 16; j++) a += (double)kv[j] * (double)Qs[r * HD + d0 + j];
                acc[r] = a;
            }
        }
#pragma unroll
        for (int r = 0; r < TQ; r++) S[r * n_keys + n] = (float)acc[r] * scale;
    }
    __syncthreads();

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

    constexpr int G = 256 / HD;
    constexpr int RP = (TQ + G - 1) / G;      // query rows per thread
    const int j = tid % HD, g = tid / HD;
    const int r0 = g * RP;
    if (r0 >= TQ) return;
    double acc[RP];
#pragma unroll
    for (int r = 0; r < RP; r++) acc[r] = 0.0;
    for (int n = 0; n < n_keys; n++) {
        const double v = (double)vc[((int64_t)n * Hkv + kvh) * HD + j];
#pragma unroll
        for (int r = 0; r < RP; r++) acc[r] += v * (double)S[(r0 + r) * n_keys + n];
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

// LDS a workgroup may use on the current device (160 KB on gfx950), read once per device.
static size_t attn_lds_limit() {
    static size_t cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        cached[dev] = (size_t)v;
    }
    return cached[dev];
}

// Score-row stride of the matrix-core kernel: whole 16-key tiles, plus 4 floats so
// rows of a 16-row fragment start in different LDS banks.
static inline int attn_sstride(int64_t n_keys) { return (int)(((n_keys + 15) / 16) * 16 + 4); }

extern "C" int dfx_attention(const float * q, const float * kc, const float * vc, int64_t M, int64_t n_keys,
                             int H, int Hkv, int hd, float * out, void * stream) {
    if (M < 0 || n_keys <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128)) {
        dfx_set_error("dfx_attention: unsupported shape M=%lld keys=%lld H=%d Hkv=%d hd=%d", (long long)M,
                      (long long)n_keys, H, Hkv, hd);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    hipStream_t st = (hipStream_t)stream;
    const int sstride = attn_sstride(n_keys);
    // One 16-row query tile per workgroup: the two-tile form needs every VGPR of the
    // SIMD (one wave per SIMD), the one-tile form runs two.
    const size_t lds_max = attn_lds_limit();
    const int RT = 1;
    if ((size_t)RT * 16 * sstride * sizeof(float) <= lds_max) {
        const size_t lds = (size_t)RT * 16 * sstride * sizeof(float);
        dim3 grid((unsigned)((M + 16 * RT - 1) / (16 * RT)), (unsigned)H);
#define ATTN_MFMA_CASE(HD_, RT_)                                                                         \
    if (hd == HD_ && RT == RT_)                                                                          \
        hipLaunchKernelGGL((k_attn_mfma<HD_, RT_>), grid, dim3(256), lds, st, q, kc, vc, (int)M, (int)n_keys, H, \
                           Hkv, sstride, out);
        ATTN_MFMA_CASE(128, 1) ATTN_MFMA_CASE(64, 1)
#undef ATTN_MFMA_CASE
        DFX_CHECK_LAUNCH("dfx_attention");
        return DFX_OK;
    }
    int TQ = 32;
    while (TQ > 1 && (size_t)TQ * (hd + n_keys) * sizeof(float) > ATTN_LDS_MAX) TQ >>= 1;
    const size_t lds = (size_t)TQ * (hd + n_keys) * sizeof(float);
    if (lds > ATTN_LDS_MAX) {
        dfx_set_error("dfx_attention: %lld keys exceed the LDS score row", (long long)n_keys);
        return DFX_ERR_UNSUPPORTED;
    }
    dim3 grid((unsigned)((M + TQ - 1) / TQ), (unsigned)H);
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
