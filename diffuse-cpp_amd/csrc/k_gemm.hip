// k_gemm.hip — GEMMs on gfx950 MFMA (v_mfma_f32_32x32x16_f16).
//
//   Y[m][n] = sum_k X[m][k] * W[n][k]   (+ bias[n]) (+ residual[m][n])
//
// Replaces ggml_mul_mat(W, X) of the reference graph (src/diffuse-graph.cpp:61-63,
// 122, 136-140, 154 and the cached twins 451-453, 556, 570-574, 587).
//
// Quantised weights (Q4_K, Q6_K, Q8_0) run the "exact" kernel k_mmq, which
// reproduces GGML's CPU dot products (ggml_vec_dot_q4_K_q8_K / q6_K_q8_K /
// q8_0_q8_0): integer products summed exactly per block, then scaled and
// accumulated in float in increasing K order with the same operations:
//   Q4_K  sum_sc += (d_w*d_a) * isum;  sum_m += (dmin_w*d_a) * msum;  y = sum_sc - sum_m
//   Q6_K  sum    += (d_w*d_a) * isum
//   Q8_0  sum    += isum * (d_w*d_a)         (per 32-element block)
// The MFMA operands are integer-valued f16: activations q_a (int8), weights
// sc*q (Q4_K, <= 945), 8*sc*c and sc*e with q = 8c+e (Q6_K, a power-of-two
// multiple of an integer below 1024) or q (Q8_0).  Every product is exact in
// f32 and every partial sum is an integer below 2^24 for real data, so the MFMA
// result is GGML's integer sum.  GGML's activation quantisation turns any
// rounding difference into whole quantisation steps that grow over the layers;
// exactness here is what keeps the logits on the CPU path's trajectory.
//
// F16 weights run k_gemm_f16: f16 x f16 products (exact) accumulated by MFMA in
// f32 (GGML accumulates them in f32/f64 SIMD lanes in its own order).
//
// Tiling: workgroup = 4 waves splitting 128 weight rows (32 each); TM tiles of
// 32 activation rows per wave.  K step = 128 (half a super-block).  Raw weight
// bytes and the f16 activation tile are staged in LDS; every wave converts its
// own 32 weight rows into B fragments in registers; the next step's global loads
// are issued before the current step's MFMAs.
#include "dfx_device.h"

#include <algorithm>

#define BK 128

// Raw bytes per weight row per K step (half super-block), as 16-byte chunks.
template <int WT> struct WT_;
template <> struct WT_<DFX_TYPE_Q4_K> { static constexpr int CH = 5,  SB = SB_Q4_K; };
template <> struct WT_<DFX_TYPE_Q6_K> { static constexpr int CH = 8,  SB = SB_Q6_K; };
template <> struct WT_<DFX_TYPE_Q8_0> { static constexpr int CH = 9,  SB = SB_Q8_0; };
template <> struct WT_<DFX_TYPE_F16>  { static constexpr int CH = 16, SB = SB_F16; };

// Byte offset inside a super-block of chunk c of half h.
template <int WT> __device__ __forceinline__ int chunk_off(int c, int h);
template <> __device__ __forceinline__ int chunk_off<DFX_TYPE_Q4_K>(int c, int h) {
    return c == 0 ? 0 : 16 + 64 * h + 16 * (c - 1);                // header | qs half
}
template <> __device__ __forceinline__ int chunk_off<DFX_TYPE_Q6_K>(int c, int h) {
    return c < 4 ? 64 * h + 16 * c                                  // ql half
         : c < 6 ? 128 + 32 * h + 16 * (c - 4)                      // qh half
         : c == 6 ? 192 : 208;                                      // scales | d
}
template <> __device__ __forceinline__ int chunk_off<DFX_TYPE_Q8_0>(int c, int h) {
    return c == 0 ? 0 : 16 + 128 * h + 16 * (c - 1);               // d[8] | qs half
}
template <> __device__ __forceinline__ int chunk_off<DFX_TYPE_F16>(int c, int h) {
    return 256 * h + 16 * c;
}

// LDS bytes per weight row: padded against bank conflicts; F16 rows are read with
// 16-byte loads and keep 16-byte alignment.
template <int WT> __host__ __device__ constexpr int wstride() {
    return WT_<WT>::CH * 16 + (WT == DFX_TYPE_F16 ? 16 : 8);
}

#define ASTR (BK + 8)   // LDS halves per activation row

// Staging of one K step: raw weight chunks and the activation tile.
template <int WT, int BM, int BN>
struct stage {
    static constexpr int CH = WT_<WT>::CH, SB = WT_<WT>::SB;
    static constexpr int W_CHUNKS = BN * CH, A_CHUNKS = BM * (BK / 8);
    static constexpr int W_PER_T = (W_CHUNKS + 255) / 256, A_PER_T = (A_CHUNKS + 255) / 256;
    uint4 w[W_PER_T], a[A_PER_T];

    __device__ __forceinline__ void load(const uint8_t * W, int N, int64_t row_bytes, const half_t * Aq, int M, int K,
                                         int n0, int m0, int kt, int tid) {
        const int sb = kt >> 1, h = kt & 1;
#pragma unroll
        for (int i = 0; i < W_PER_T; i++) {
            const int c = tid + i * 256;
            if (c < W_CHUNKS) {
                const int r = c / CH, cc = c - r * CH;
                const int n = min(n0 + r, N - 1);
                w[i] = *(const uint4 *)(W + (int64_t)n * row_bytes + (int64_t)sb * SB + chunk_off<WT>(cc, h));
            }
        }
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int c = tid + i * 256;
            if (c < A_CHUNKS) {
                const int r = c >> 4, cc = c & 15;
                const int m = m0 + r;
                a[i] = m < M ? *(const uint4 *)(Aq + (int64_t)m * K + kt * BK + cc * 8) : make_uint4(0, 0, 0, 0);
            }
        }
    }
    __device__ __forceinline__ void store(uint8_t * Ws, half_t * As, int tid) const {
        constexpr int WSTR = wstride<WT>();
#pragma unroll
        for (int i = 0; i < W_PER_T; i++) {
            const int c = tid + i * 256;
            if (c < W_CHUNKS) {
                const int r = c / CH, cc = c - r * CH;
                uint2 * dst = (uint2 *)(Ws + r * WSTR + cc * 16);
                dst[0] = make_uint2(w[i].x, w[i].y);
                dst[1] = make_uint2(w[i].z, w[i].w);
            }
        }
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int c = tid + i * 256;
            if (c < A_CHUNKS) {
                const int r = c >> 4, cc = c & 15;
                *(uint4 *)(As + r * ASTR + cc * 8) = a[i];
            }
        }
    }
};

__device__ __forceinline__ half8 to_half8(const int v[8]) {
    half8 r;
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = (half_t)v[j];   // |v| <= 2048, or a power-of-two multiple: exact
    return r;
}

// Row of register r of a 32x32 MFMA tile held by `lane` (its column is lane % 32).
__device__ __forceinline__ int tile_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

__device__ __forceinline__ void epilogue_store(float v, int m, int n, const float * bias, const float * res, float * Y,
                                               int64_t ldy, const int32_t * ymap) {
    const int64_t o = (int64_t)(ymap ? ymap[m] : m) * ldy + n;
    if (bias) v = v + bias[n];
    if (res) v = v + res[o];
    Y[o] = v;
}

// ---------------------------------------------------------------------------
// Exact kernel for quantised weights
// ---------------------------------------------------------------------------
template <int WT, int TM>
__global__ void __launch_bounds__(256, 2)
k_mmq(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
      const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap) {
#pragma clang fp contract(off)
    constexpr int BM = TM * 32, BN = 128, WSTR = wstride<WT>();
    constexpr bool KQ = WT != DFX_TYPE_Q8_0;     // Q8_K activations: d per 256, bsums per 16
    constexpr int BSTR = 24;                     // LDS halves per row of 16 block sums
    __shared__ __attribute__((aligned(16))) uint8_t Ws[BN * WSTR];
    __shared__ __attribute__((aligned(16))) half_t As[BM * ASTR];
    __shared__ __attribute__((aligned(16))) float Ad[BM * 4];          // KQ: [BM]; Q8_0: [BM][4]
    __shared__ __attribute__((aligned(16))) half_t Abs[KQ ? BM * BSTR : 8];

    const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int n_kt = K / BK;
    const int64_t row_bytes = (int64_t)(K >> 8) * WT_<WT>::SB;
    const act_layout Lay = act_layout_of(KQ ? CONV_Q8_K : CONV_Q8_0, M, K);
    const half_t * Aq = (const half_t *)(act + Lay.q);
    const float * Adg = (const float *)(act + Lay.d);
    const half_t * Absg = (const half_t *)(act + Lay.bs);

    stage<WT, BM, BN> st;
    float dreg = 0.0f;                                  // KQ: d_a of row tid (tid < BM)
    float4 dreg4 = make_float4(0, 0, 0, 0);             // Q8_0: d_a of the 4 blocks of the K step
    uint4 bsreg = make_uint4(0, 0, 0, 0);               // KQ: 8 of the 16 block sums of row tid/2

    auto load_meta = [&](int kt) {
        const int sb = kt >> 1;
        if (KQ) {
            if ((kt & 1) == 0) {
                if (tid < BM) dreg = (m0 + tid < M) ? Adg[(int64_t)(m0 + tid) * (K / 256) + sb] : 0.0f;
                if (tid < 2 * BM) {
                    const int r = tid >> 1, c = tid & 1;
                    bsreg = (m0 + r < M) ? *(const uint4 *)(Absg + (int64_t)(m0 + r) * (K / 16) + sb * 16 + c * 8)
                                         : make_uint4(0, 0, 0, 0);
                }
            }
        } else if (tid < BM) {
            dreg4 = (m0 + tid < M) ? *(const float4 *)(Adg + (int64_t)(m0 + tid) * (K / 32) + kt * 4)
                                   : make_float4(0, 0, 0, 0);
        }
    };
    auto store_meta = [&](int kt) {
        if (KQ) {
            if ((kt & 1) == 0) {
                if (tid < BM) Ad[tid] = dreg;
                if (tid < 2 * BM) *(uint4 *)(Abs + (tid >> 1) * BSTR + (tid & 1) * 8) = bsreg;
            }
        } else if (tid < BM) {
            *(float4 *)(Ad + tid * 4) = dreg4;
        }
    };

    float16v P[TM], S1[TM], S2[TM];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) P[i][r] = S1[i][r] = S2[i][r] = 0.0f;

    const uint8_t * wp = Ws + (wn * 32 + (lane & 31)) * WSTR;   // this lane's weight row
    const int hl = lane >> 5;

    st.load(W, N, row_bytes, Aq, M, K, n0, m0, 0, tid);
    load_meta(0);
    for (int kt = 0; kt < n_kt; kt++) {
        __syncthreads();
        st.store(Ws, As, tid);
        store_meta(kt);
        __syncthreads();
        if (kt + 1 < n_kt) {
            st.load(W, N, row_bytes, Aq, M, K, n0, m0, kt + 1, tid);
            load_meta(kt + 1);
        }
        const int h = kt & 1;
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            const int e = kk * 16 + 8 * hl;      // first of this lane's 8 K elements in the step
            int u[8], u2[8];
            if (WT == DFX_TYPE_Q4_K) {
                int sc, mn;
                q4k_scale_min(4 * h + (e >> 5), wp + 4, sc, mn);
                const uint2 q = *(const uint2 *)(wp + 16 + 32 * (e >> 6) + (e & 31));
                const int sh = 4 * ((e >> 5) & 1);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    u[j] = sc * (int)((q.x >> (8 * j + sh)) & 15);
                    u[4 + j] = sc * (int)((q.y >> (8 * j + sh)) & 15);
                }
            } else if (WT == DFX_TYPE_Q6_K) {
                const int quarter = e >> 5, l = e & 31;
                const uint2 lo = *(const uint2 *)(wp + l + 32 * (quarter & 1));
                const uint2 hb = *(const uint2 *)(wp + 64 + l);
                const int sc = (int8_t)wp[96 + 8 * h + 2 * quarter + (l >> 4)];
                const int sl = 4 * (quarter >> 1), sh = 2 * quarter;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t lw = j < 4 ? lo.x : lo.y, hw = j < 4 ? hb.x : hb.y;
                    const int jj = j & 3;
                    const int q6 = (int)(((lw >> (8 * jj + sl)) & 15) | (((hw >> (8 * jj + sh)) & 3) << 4));
                    // q6 - 32 = 8*c + e with c in [-4, 3], e in [0, 7]
                    u[j] = 8 * (sc * ((q6 >> 3) - 4));
                    u2[j] = sc * (q6 & 7);
                }
            } else {   // Q8_0
                const uint2 q = *(const uint2 *)(wp + 16 + e);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    u[j] = (int8_t)(q.x >> (8 * j));
                    u[4 + j] = (int8_t)(q.y >> (8 * j));
                }
            }
            const half8 b = to_half8(u);
            half8 b2;
            if (WT == DFX_TYPE_Q6_K) b2 = to_half8(u2);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const half8 a = *(const half8 *)(As + (i * 32 + (lane & 31)) * ASTR + e);
                P[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, P[i], 0, 0, 0);
                if (WT == DFX_TYPE_Q6_K) P[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b2, P[i], 0, 0, 0);
            }
            if (WT == DFX_TYPE_Q8_0 && (kk & 1)) {
                // a 32-element block is complete: sum += isum * (d_w * d_a)
                const int bl = kk >> 1;
                const float dw = h2f(*(const uint16_t *)(wp + 2 * (4 * h + bl)));
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float da = Ad[(i * 32 + tile_row(r, lane)) * 4 + bl];
                        S1[i][r] = S1[i][r] + P[i][r] * (dw * da);
                        P[i][r] = 0.0f;
                    }
            }
        }
        if (KQ && h == 1) {
            // super-block complete
            if (WT == DFX_TYPE_Q4_K) {
                // msum = sum_j m_j * (bsum_{2j} + bsum_{2j+1}) as a 16-deep product:
                // B[k][n] = m_{k/2}, k = 8*(lane/32) + t
                int mv[8];
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    int sc, mn;
                    q4k_scale_min(4 * hl + t / 2, wp + 4, sc, mn);
                    mv[t] = mv[t + 1] = mn;
                }
                const half8 bm = to_half8(mv);
                const float dw = h2f(*(const uint16_t *)(wp + 0)), dmw = h2f(*(const uint16_t *)(wp + 2));
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const half8 a = *(const half8 *)(Abs + (i * 32 + (lane & 31)) * BSTR + 8 * hl);
                    float16v Q;
#pragma unroll
                    for (int r = 0; r < 16; r++) Q[r] = 0.0f;
                    Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bm, Q, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float da = Ad[i * 32 + tile_row(r, lane)];
                        S1[i][r] = S1[i][r] + (dw * da) * P[i][r];
                        S2[i][r] = S2[i][r] + (dmw * da) * Q[r];
                        P[i][r] = 0.0f;
                    }
                }
            } else {
                const float dw = h2f(*(const uint16_t *)(wp + 112));
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float da = Ad[i * 32 + tile_row(r, lane)];
                        S1[i][r] = S1[i][r] + (dw * da) * P[i][r];
                        P[i][r] = 0.0f;
                    }
            }
        }
    }

    const int n = n0 + wn * 32 + (lane & 31);
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + i * 32 + tile_row(r, lane);
            if (m >= M) continue;
            const float v = WT == DFX_TYPE_Q4_K ? S1[i][r] - S2[i][r] : S1[i][r];
            epilogue_store(v, m, n, bias, res, Y, ldy, ymap);
        }
}

// ---------------------------------------------------------------------------
// F16 weights
// ---------------------------------------------------------------------------
template <int TM>
__global__ void __launch_bounds__(256, 2)
k_gemm_f16(const uint8_t * __restrict__ W, int N, int K, const half_t * __restrict__ A, int M,
           const float * __restrict__ bias, const float * res, float * Y, int64_t ldy,
           const int32_t * __restrict__ ymap, float * __restrict__ ws, int kt_per_split) {
    constexpr int BM = TM * 32, BN = 128, WSTR = wstride<DFX_TYPE_F16>();
    __shared__ __attribute__((aligned(16))) uint8_t Ws[BN * WSTR];
    __shared__ __attribute__((aligned(16))) half_t As[BM * ASTR];
    const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int n_kt = K / BK;
    const int kt0 = blockIdx.z * kt_per_split;
    const int kt1 = min(kt0 + kt_per_split, n_kt);
    const int64_t row_bytes = (int64_t)K * 2;
    stage<DFX_TYPE_F16, BM, BN> st;
    float16v acc[TM];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
    const uint8_t * wp = Ws + (wn * 32 + (lane & 31)) * WSTR;
    if (kt0 < kt1) st.load(W, N, row_bytes, A, M, K, n0, m0, kt0, tid);
    for (int kt = kt0; kt < kt1; kt++) {
        __syncthreads();
        st.store(Ws, As, tid);
        __syncthreads();
        if (kt + 1 < kt1) st.load(W, N, row_bytes, A, M, K, n0, m0, kt + 1, tid);
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            const int e = kk * 16 + 8 * (lane >> 5);
            const half8 b = *(const half8 *)(wp + 2 * e);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const half8 a = *(const half8 *)(As + (i * 32 + (lane & 31)) * ASTR + e);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
            }
        }
    }
    const bool split = gridDim.z > 1;
    const int n = n0 + wn * 32 + (lane & 31);
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + i * 32 + tile_row(r, lane);
            if (m >= M) continue;
            if (split) ws[((int64_t)blockIdx.z * M + m) * N + n] = acc[i][r];
            else epilogue_store(acc[i][r], m, n, bias, res, Y, ldy, ymap);
        }
}

// Fixed-order reduction of split-K partials plus epilogue.
__global__ void k_gemm_reduce(const float * __restrict__ ws, int S, int64_t MN, int N, const float * bias,
                              const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < MN;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = idx / N, n = idx - m * N;
        float v = ws[idx];
        for (int s = 1; s < S; s++) v += ws[(int64_t)s * MN + idx];
        epilogue_store(v, (int)m, (int)n, bias, res, Y, ldy, ymap);
    }
}

#define MAX_SPLIT 8

extern "C" size_t dfx_gemm_ws_bytes(int64_t M, int64_t N) { return (size_t)MAX_SPLIT * M * N * sizeof(float); }

template <int TM>
static int launch_f16(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, void * ws, size_t ws_bytes, hipStream_t st) {
    constexpr int BM = TM * 32, BN = 128;
    const int gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM;
    const int n_kt = K / BK;
    int S = 1;
    if (ws) {
        // split K while the grid is smaller than the CU count, the workspace holds the
        // partials and every split keeps at least 4 K steps
        const int tiles = gx * gy;
        while (S < MAX_SPLIT && tiles * S < 256 && n_kt / (S * 2) >= 4 &&
               (size_t)(S * 2) * M * N * sizeof(float) <= ws_bytes)
            S *= 2;
    }
    const int per = (n_kt + S - 1) / S;
    S = (n_kt + per - 1) / per;
    hipLaunchKernelGGL((k_gemm_f16<TM>), dim3(gx, gy, S), dim3(256), 0, st, (const uint8_t *)w, N, K,
                       (const half_t *)act, M, bias, res, y, ldy, ymap, (float *)ws, per);
    DFX_CHECK_LAUNCH("dfx_gemm f16");
    if (S > 1) {
        const int64_t MN = (int64_t)M * N;
        const int64_t blocks = std::min<int64_t>((MN + 255) / 256, 8192);
        hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)blocks), dim3(256), 0, st, (const float *)ws, S, MN, N,
                           bias, res, y, ldy, ymap);
        DFX_CHECK_LAUNCH("dfx_gemm reduce");
    }
    return DFX_OK;
}

template <int WT, int TM>
static int launch_mmq(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, hipStream_t st) {
    constexpr int BM = TM * 32, BN = 128;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL((k_mmq<WT, TM>), grid, dim3(256), 0, st, (const uint8_t *)w, N, K, (const uint8_t *)act, M,
                       bias, res, y, ldy, ymap);
    DFX_CHECK_LAUNCH("dfx_gemm");
    return DFX_OK;
}

// M tile (32 * TM rows) with the least row padding, larger tiles on ties.
static int pick_tm(int M, int max_tm) {
    int best = 1, best_pad = 1 << 30;
    for (int t = 1; t <= max_tm; t++) {
        const int pad = ((M + 32 * t - 1) / (32 * t)) * 32 * t;
        if (pad <= best_pad) { best = t; best_pad = pad; }
    }
    return best;
}

template <int WT>
static int dispatch_mmq(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, hipStream_t st) {
    switch (pick_tm(M, 3)) {
        case 1: return launch_mmq<WT, 1>(w, N, K, act, M, bias, res, y, ldy, ymap, st);
        case 2: return launch_mmq<WT, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, st);
        default: return launch_mmq<WT, 3>(w, N, K, act, M, bias, res, y, ldy, ymap, st);
    }
}

// Internal form: output row m goes to row ymap[m] (or m) of Y with leading dimension
// ldy; the residual is read at the same place it is written.  Split-K (F16 only)
// uses ws when it is large enough.
int dfx_gemm_ex(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                const float * bias, const float * residual, float * y, int64_t ldy, const int32_t * ymap,
                void * ws, size_t ws_bytes, void * stream) {
    if (N <= 0 || K <= 0 || M < 0 || (K % 256) || N > INT32_MAX || M > INT32_MAX || K > INT32_MAX || ldy < N) {
        dfx_set_error("dfx_gemm: bad shape M=%lld N=%lld K=%lld ldy=%lld (K must be a multiple of 256)",
                      (long long)M, (long long)N, (long long)K, (long long)ldy);
        return DFX_ERR_ARG;
    }
    if (M == 0) return DFX_OK;
    hipStream_t st = (hipStream_t)stream;
    const int n = (int)N, k = (int)K, m = (int)M;
    switch (wtype) {
        case DFX_TYPE_Q4_K: return dispatch_mmq<DFX_TYPE_Q4_K>(w, n, k, act, m, bias, residual, y, ldy, ymap, st);
        case DFX_TYPE_Q6_K: return dispatch_mmq<DFX_TYPE_Q6_K>(w, n, k, act, m, bias, residual, y, ldy, ymap, st);
        case DFX_TYPE_Q8_0: return dispatch_mmq<DFX_TYPE_Q8_0>(w, n, k, act, m, bias, residual, y, ldy, ymap, st);
        case DFX_TYPE_F16:
            switch (pick_tm(m, 4)) {
                case 1: return launch_f16<1>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st);
                case 2: return launch_f16<2>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st);
                case 3: return launch_f16<3>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st);
                default: return launch_f16<4>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st);
            }
    }
    dfx_set_error("dfx_gemm: unsupported weight type %d", wtype);
    return DFX_ERR_UNSUPPORTED;
}

extern "C" int dfx_gemm(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                        const float * bias, const float * residual, float * y, void * ws, void * stream) {
    return dfx_gemm_ex(wtype, w, N, K, act, M, bias, residual, y, N, nullptr, ws,
                       ws ? dfx_gemm_ws_bytes(M, N) : 0, stream);
}
