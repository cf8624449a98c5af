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
// accumulated in float in increasing K order, in the same order as the CPU
// oracle:
//   Q4_K  x = d_w*isum;  x = fma(-dmin_w, msum, x);  S = fma(d_a, x, S)
//   Q6_K  x = d_w*isum;  S = fma(d_a, x, S)
//   Q8_0  x = d_w*isum;  S = fma(d_a, x, S)         (per 32-element block)
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
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

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

// Block flushes over one lane's 16 outputs of a 32x32 tile, written as passes of 16
// independent operations (an empty asm on every value between passes keeps the compiler
// from folding them back into one dependent chain per output).  Each output sees the same
// operations in the same order as the chain, so the bits are the same; the VALU then
// pipelines the 16 outputs instead of waiting out each output's chain (measured on MI355X:
// the Q4_K super-block flush 25 % shorter).
__device__ __forceinline__ void pass_barrier(float (&x)[16]) {
#pragma unroll
    for (int r = 0; r < 16; r++) asm volatile("" : "+v"(x[r]));
}
// Q4_K super-block: x = d_w*isum; x = fma(-dmin_w, msum, x); S = fma(d_a, x, S)
__device__ __forceinline__ void flush_dmin(float16v & S, const float16v & P, const float16v & Q, float dw, float dmw,
                                           const float (&da)[16]) {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; r++) x[r] = dw * P[r];
    pass_barrier(x);
#pragma unroll
    for (int r = 0; r < 16; r++) x[r] = fmaf(-dmw, Q[r], x[r]);
    pass_barrier(x);
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = fmaf(da[r], x[r], S[r]);
}
// Q6_K super-block, Q8_0 block: S = fma(d_a, d_w*isum, S)
__device__ __forceinline__ void flush_d(float16v & S, const float16v & P, float dw, const float (&da)[16]) {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; r++) x[r] = dw * P[r];
    pass_barrier(x);
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = fmaf(da[r], x[r], S[r]);
}

// RoPE epilogue of one 32 x 32 tile (DFX_EPI_ROPE): v[r] is this lane's value of row
// m0 + tile_row(r, lane) at GEMM column n, w[r] the value of the paired column n ^ 16,
// p[r] the row's position.  The rotation is the NEOX one of ggml_rope_ext, as the RoPE
// kernel computes it: y0 = x0 * cos - x1 * sin, y1 = x0 * sin + x1 * cos.
__device__ __forceinline__ void rope_tile(const float (&v)[16], const float (&w)[16], const int (&p)[16], int m0,
                                          int n, bool live, int M, int lane, const dfx_epi & epi) {
#pragma clang fp contract(off)
    const int hd = epi.hd, half = hd >> 1;
    const int g = n + epi.col0, hh = g / hd, cc = g - hh * hd;
    if (hh < epi.H + epi.Hkv) {
        const bool first = (cc & 16) == 0;
        const int d0 = 16 * (cc >> 5) + (cc & 15), d = first ? d0 : half + d0;
        float2 cs[16];
#pragma unroll
        for (int r = 0; r < 16; r++) cs[r] = *(const float2 *)(epi.tab + ((int64_t)p[r] * half + d0) * 2);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + tile_row(r, lane);
            if (!live || m >= M) continue;
            const float x0 = first ? v[r] : w[r], x1 = first ? w[r] : v[r];
            const float y = first ? x0 * cs[r].x - x1 * cs[r].y : x0 * cs[r].y + x1 * cs[r].x;
            float * dst = hh < epi.H ? epi.q_out + ((int64_t)m * epi.H + hh) * hd
                                     : epi.kc + ((int64_t)p[r] * epi.Hkv + (hh - epi.H)) * hd;
            dst[d] = y;
        }
    } else {
        float * col = epi.vt + ((int64_t)(hh - epi.H - epi.Hkv) * hd + cc) * epi.v_ld;
#pragma unroll
        for (int r = 0; r < 16; r++)
            if (live && m0 + tile_row(r, lane) < M) col[p[r]] = v[r];
    }
}

// Epilogue of one 32x32 MFMA tile held by `lane`: register r is row m0 + tile_row(r, lane),
// column n.  Every read (row map, bias, residual) is issued before any is used, at clamped
// (always valid) addresses, so the wave waits once per kind of read rather than once per
// element; rows >= M and columns >= N are not stored.  With ws (split K) the tile's chunk
// sum goes to ws[z][m][n] instead.  y = (v + bias) + residual, written to Y[ymap[m] * ldy + n]
// (Y[m * ldy + n] without a row map).
template <typename V16>
__device__ __forceinline__ void epilogue_tile(const V16 & acc, int m0, int n, int M, int N, const float * bias,
                                              const float * res, float * Y, int64_t ldy, const int32_t * ymap,
                                              float * ws, int z, int lane, dfx_epi epi) {
#pragma clang fp contract(off)
    if (!ws && epi.kind == DFX_EPI_SWIGLU) {
        // lane ^ 16 holds the same rows of column n ^ 16 (n is 32j + lane % 32): a gate lane
        // and its up lane share F-index f.  The pair splits the 16 rows: the gate lane forms
        // h for registers 0..7, the up lane for registers 8..15 (rows 16 further down), each
        // receiving the partner's value of its rows (no bias, residual or row map here).
        const bool gate = (n & 16) == 0;
        const int64_t f = (int64_t)(n >> 5) * 16 + (n & 15);
        const int dm = gate ? 0 : 16;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float mine_lo = (float)acc[i], mine_hi = (float)acc[i + 8];
            const float other = __shfl_xor(gate ? mine_hi : mine_lo, 16, WAVE);
            const float g = gate ? mine_lo : other;
            const float u = gate ? other : mine_hi;
            const int m = m0 + tile_row(i, lane) + dm;
            if (n < N && m < M) Y[(int64_t)m * ldy + f] = silu_mul(g, u);
        }
        return;
    }
    if (ws) {
        if (n < N)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + tile_row(r, lane);
                if (m < M) ws[((int64_t)z * M + m) * N + n] = acc[r];
            }
        return;
    }
    if (epi.kind == DFX_EPI_ROPE) {
        const int nc = min(n, N - 1);
        const float b = bias ? bias[nc] : 0.0f;
        float v[16], w[16];
        int p[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            v[r] = acc[r];
            if (bias) v[r] = v[r] + b;
            p[r] = epi.pos[min(m0 + tile_row(r, lane), M - 1)];
        }
        // lane ^ 16 holds the same rows of the other dim of this lane's NEOX pair
#pragma unroll
        for (int r = 0; r < 16; r++) w[r] = __shfl_xor(v[r], 16, WAVE);
        rope_tile(v, w, p, m0, nc, n < N, M, lane, epi);
        return;
    }
    const int nc = min(n, N - 1);
    int64_t o[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = min(m0 + tile_row(r, lane), M - 1);
        o[r] = (int64_t)(ymap ? ymap[m] : m) * ldy + nc;
    }
    float rv[16];
    if (res)
#pragma unroll
        for (int r = 0; r < 16; r++) rv[r] = res[o[r]];
    const float b = bias ? bias[nc] : 0.0f;
    // All sums are formed before the first store: a sum sunk into its store's branch would make
    // each store wait for the one before it to complete.
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        v[r] = acc[r];
        if (bias) v[r] = v[r] + b;
        if (res) v[r] = v[r] + rv[r];
        asm volatile("" : "+v"(v[r]));
    }
#pragma unroll
    for (int r = 0; r < 16; r++)
        if (n < N && m0 + tile_row(r, lane) < M) Y[o[r]] = v[r];
}

// ---------------------------------------------------------------------------
// Exact kernel for quantised weights
// ---------------------------------------------------------------------------
template <int WT, int TM>
__global__ void __launch_bounds__(256, 2)
k_mmq(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
      const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
      dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr int BM = TM * 32, BN = 128, WSTR = wstride<WT>();
    constexpr bool KQ = WT != DFX_TYPE_Q8_0;     // Q8_K activations: d per 256, bsums per 16
    constexpr int BSTR = 24;                     // LDS halves per row of 16 block sums
    __shared__ __attribute__((aligned(16))) uint8_t Ws[BN * WSTR];
    __shared__ __attribute__((aligned(16))) half_t As[BM * ASTR];
    __shared__ __attribute__((aligned(16))) float Ad[BM * 4];          // KQ: [BM]; Q8_0: [4][BM]
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
            // [block][row]: a lane's four consecutive tile rows of one block are one 16-byte read
            Ad[tid] = dreg4.x;
            Ad[BM + tid] = dreg4.y;
            Ad[2 * BM + tid] = dreg4.z;
            Ad[3 * BM + tid] = dreg4.w;
        }
    };

    float16v P[TM], S1[TM], T1[TM];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) P[i][r] = S1[i][r] = T1[i][r] = 0.0f;

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
            }
            half8 b;
            if (WT == DFX_TYPE_Q8_0) {
                // int8 q as an exact f16 integer without conversions: q + 128 (the byte with its
                // top bit flipped) becomes the mantissa of 0x6400 = 1024.0 (v_perm places two bytes
                // beside 0x64 bytes), and one packed f16 add of -1152 leaves q
                const uint2 qw = *(const uint2 *)(wp + 16 + e);
                const uint32_t x0 = qw.x ^ 0x80808080u, x1 = qw.y ^ 0x80808080u;
                const u32x4 pk = {__builtin_amdgcn_perm(x0, 0x64646464u, 0x00050004u),
                                  __builtin_amdgcn_perm(x0, 0x64646464u, 0x00070006u),
                                  __builtin_amdgcn_perm(x1, 0x64646464u, 0x00050004u),
                                  __builtin_amdgcn_perm(x1, 0x64646464u, 0x00070006u)};
                const half8 off = {(half_t)-1152.0f, (half_t)-1152.0f, (half_t)-1152.0f, (half_t)-1152.0f,
                                   (half_t)-1152.0f, (half_t)-1152.0f, (half_t)-1152.0f, (half_t)-1152.0f};
                b = __builtin_bit_cast(half8, pk) + off;
            } else {
                b = to_half8(u);
            }
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
                for (int i = 0; i < TM; i++) {
                    // registers 4g..4g+3 hold rows 8g + 4(lane/32) + 0..3: one 16-byte read each
                    // from the [block][row] layout of Ad
                    float dav[16];
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 d4 = *(const float4 *)(Ad + bl * BM + i * 32 + 8 * g + 4 * hl);
                        dav[4 * g] = d4.x; dav[4 * g + 1] = d4.y; dav[4 * g + 2] = d4.z; dav[4 * g + 3] = d4.w;
                    }
                    flush_d(S1[i], P[i], dw, dav);
#pragma unroll
                    for (int r = 0; r < 16; r++) P[i][r] = 0.0f;
                }
            }
        }
        if (!KQ && ((kt + 1) % (DFX_DOT_CHUNK / BK) == 0 || kt + 1 == n_kt)) {
            // chunk complete: T = T + S
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) { T1[i][r] = T1[i][r] + S1[i][r]; S1[i][r] = 0.0f; }
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
                    float dav[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) dav[r] = Ad[i * 32 + tile_row(r, lane)];
                    flush_dmin(S1[i], P[i], Q, dw, dmw, dav);
#pragma unroll
                    for (int r = 0; r < 16; r++) P[i][r] = 0.0f;
                }
            } else {
                const float dw = h2f(*(const uint16_t *)(wp + 112));
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    float dav[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) dav[r] = Ad[i * 32 + tile_row(r, lane)];
                    flush_d(S1[i], P[i], dw, dav);
#pragma unroll
                    for (int r = 0; r < 16; r++) P[i][r] = 0.0f;
                }
            }
            if (((kt >> 1) + 1) % (DFX_DOT_CHUNK / 256) == 0 || kt + 1 == n_kt) {
                // chunk complete: T = T + S
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) { T1[i][r] = T1[i][r] + S1[i][r]; S1[i][r] = 0.0f; }
            }
        }
    }

    const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM; i++) epilogue_tile(T1[i], m0 + i * 32, n, M, N, bias, res, Y, ldy, ymap, nullptr, 0, lane, epi);
}

// ---------------------------------------------------------------------------
// Q4_K: register-blocked kernel with packed-f16 dequantisation
// ---------------------------------------------------------------------------
// Workgroup = 4 waves side by side along N; wave w owns TN column tiles of 32 weight
// rows and every wave covers all TM row tiles of 32 activation rows, so a
// dequantised B fragment feeds TM MFMAs and an A fragment (LDS) feeds TN.
// A K step is half a super-block (128): lane (row n, half hl) holds the 32 bytes of
// packed nibbles of group g = 2h+hl, and MFMA kk takes word kk of them.  One word w
// (bytes b0..b3) gives the eight operands
//   [lo b0, lo b2, lo b1, lo b3, hi b0, hi b2, hi b1, hi b3] * sc
// as f16 integers with no conversion instructions: (w & 0x000F000F) | 0x64006400 is
// the f16 pair (1024+lo b0, 1024+lo b2), and one packed FMA x*sc - 1024*sc leaves
// sc*lo exactly (high nibbles: mask 0x00F000F0, factor sc/16, constant -64*sc).  The
// activation buffer stores q in the same slot order (CONV_Q8_K_P4).
// The weights of the next K step are loaded into registers during the current one;
// the A tile is double-buffered in LDS (one barrier per K step).  Workgroups are
// numbered so that all row tiles of one column tile run on the same XCD (L2).

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_fma_h2(uint32_t x, uint32_t a, uint32_t c) {
    const half2v r = __builtin_elementwise_fma(__builtin_bit_cast(half2v, x), __builtin_bit_cast(half2v, a),
                                               __builtin_bit_cast(half2v, c));
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t h2pair(float v) {
    const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)v);
    return h | (h << 16);
}

// v_and_or_b32 (x & m) | o; the masks live in VGPRs (gfx9 VOP3 takes no literals).
// (x & m) | o for an o with no bits inside m, written as (x & m) | (o & ~m) so that it
// becomes one v_bfi_b32.  m and o must reach it as register values (opaque()):
// with literal constants the compiler folds o & ~m and emits an and and an or.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) { return (x & m) | (o & ~m); }
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Q4_K header of one super-block held in registers: x = {d, dmin}, y/z/w = scales[0..11].
// The eight 6-bit scales and mins (GGML get_scale_min_k4) as bytes of two words each:
//   sc[0..3] = y & 63              sc[4..7] = (w & 15) | ((y >> 6) << 4)
//   mn[0..3] = z & 63              mn[4..7] = (w >> 4) | ((z >> 6) << 4)
struct q4k_sm { uint32_t sc_lo, sc_hi, mn_lo, mn_hi; };
__device__ __forceinline__ q4k_sm q4k_unpack(const u32x4 & h) {
    q4k_sm r;
    r.sc_lo = h.y & 0x3F3F3F3Fu;
    r.sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    r.mn_lo = h.z & 0x3F3F3F3Fu;
    r.mn_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    return r;
}

// Scale constants of the two sub-blocks (low / high nibbles) of one 64-element group.
struct q4k_consts { uint32_t slo, clo, shi, chi; };
__device__ __forceinline__ q4k_consts q4k_group_consts(uint32_t sc_word, int shift) {
    const float s0 = (float)((sc_word >> shift) & 0xFFu), s1 = (float)((sc_word >> (shift + 8)) & 0xFFu);
    q4k_consts k;
    k.slo = h2pair(s0);
    k.clo = h2pair(-1024.0f * s0);
    k.shi = h2pair(s1 * 0.0625f);
    k.chi = h2pair(-64.0f * s1);
    return k;
}

// Eight f16 operands [lo b0, lo b2, lo b1, lo b3, hi b0, hi b2, hi b1, hi b3] * sc from
// one word of packed nibbles.
__device__ __forceinline__ half8 q4k_word(uint32_t w, const q4k_consts & k, uint32_t m_lo, uint32_t m_hi,
                                          uint32_t magic) {
    const uint32_t s8 = w >> 8;
    u32x4 r;
    r.x = pk_fma_h2(and_or(w, m_lo, magic), k.slo, k.clo);
    r.y = pk_fma_h2(and_or(s8, m_lo, magic), k.slo, k.clo);
    r.z = pk_fma_h2(and_or(w, m_hi, magic), k.shi, k.chi);
    r.w = pk_fma_h2(and_or(s8, m_hi, magic), k.shi, k.chi);
    return __builtin_bit_cast(half8, r);
}

// Four 6-bit mins (bytes of m4) as the half8 [m0, m0, m1, m1, m2, m2, m3, m3].
__device__ __forceinline__ half8 mins_half8(uint32_t m4) {
    u32x4 r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t v = (m4 >> (8 * k)) & 0xFFu;
        r[k] = h2pair((float)v);
    }
    return __builtin_bit_cast(half8, r);
}

// NWV waves side by side (4: 128 weight rows per workgroup; 1 or 2 give narrow GEMMs over few
// rows more workgroups than CUs would otherwise get); the second bound is waves per SIMD,
// so the register budget does not depend on NWV.
template <int TM, int TN, int D, int NWV = 4>
__global__ void __launch_bounds__(64 * NWV, TM * TN >= 4 ? 1 : 2)
k_q4k(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
      const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
      int n_tiles, int m_tiles, float * __restrict__ ws, dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr int NT = 64 * NWV;             // threads per workgroup
    constexpr int BM = TM * 32, BN = NWV * TN * 32;
    constexpr int BST = 24;                  // LDS halves per row of 16 block sums
    constexpr int A_PER_T = BM * 16 / NT;    // 16-byte chunks of the A tile per thread
    static_assert(A_PER_T >= 1 && A_PER_T * NT == BM * 16 && NT >= 2 * BM, "A tile split over the threads");
    // A tile of one K step in fragment order: operand kk of row tile i at half (8i + kk) * 512
    __shared__ __attribute__((aligned(16))) half_t As[2][BM * 128];
    __shared__ __attribute__((aligned(16))) float Ad[2][BM];
    __shared__ __attribute__((aligned(16))) half_t Abs[2][BM * BST];

    // XCD-aware tile order: workgroup L runs on XCD L % 8; column tile x always maps
    // to XCD x % 8, and its row tiles are consecutive there.  With ws (split K) the
    // grid repeats once per K chunk: chunk z = blockIdx.x / (tiles of one pass).
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int z = blockIdx.x / per_pass, L = blockIdx.x - z * per_pass, xcd = L & 7, j = L >> 3;
    const int ty = j % m_tiles, tx = 8 * (j / m_tiles) + xcd;
    if (tx >= n_tiles) return;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hl = lane >> 5, l32 = lane & 31;
    const int n0 = tx * BN, m0 = ty * BM;
    constexpr int SB_CHUNK = DFX_DOT_CHUNK / 256;
    const int n_sb_all = K >> 8;
    const int sb_first = ws ? z * SB_CHUNK : 0;                       // this workgroup's super-blocks
    const int n_sb = ws ? min(SB_CHUNK, n_sb_all - sb_first) : n_sb_all;
    const int n_kt = 2 * n_sb;
    const uint32_t row_bytes = (uint32_t)n_sb_all * SB_Q4_K;
    const act_layout Lay = act_layout_of(CONV_Q8_K_P4, M, K);
    const int m_pad = (int)act_q_rows(CONV_Q8_K_P4, M);
    const uint8_t * Aq = act + Lay.q;
    const uint8_t * Adg = act + Lay.d;
    const uint8_t * Absg = act + Lay.bs;

    // Per-thread 32-bit byte offsets from bases that only move with the K step (so the
    // loads use a scalar base and the step costs no vector instructions).  Every load
    // is unconditional, at a clamped (always valid) address: padded rows (m >= M) only
    // feed output rows that are never stored, and steps past the end are never used.
    uint32_t off_a[A_PER_T], off_w[TN];
#pragma unroll
    for (int i = 0; i < A_PER_T; i++) {
        // chunk c of the step: row tile c / 512 (clamped to the padded rows), 16 bytes c % 512
        const int c = tid + NT * i, mt = min(m0 / 32 + (c >> 9), m_pad / 32 - 1);
        off_a[i] = (uint32_t)mt * (uint32_t)(K / 128) * 8192u + (uint32_t)(c & 511) * 16u;
    }
#pragma unroll
    for (int t = 0; t < TN; t++) off_w[t] = (uint32_t)min(n0 + (wv * TN + t) * 32 + l32, N - 1) * row_bytes;
    const uint32_t off_d = (uint32_t)min(m0 + tid % BM, M - 1) * 4u;   // d is [sb][m_pad]
    const uint32_t off_b = ((uint32_t)min(m0 + (tid >> 1) % BM, M - 1) * (uint32_t)(K / 16) + (tid & 1) * 8u) * 2u;

    // Register rings: weight stage s holds the nibbles (and header) of K step kt with
    // kt % D == s, D-1 steps ahead (weights stream from HBM); the activation rows and
    // their block scales / sums (small, L2-resident) are loaded one step ahead into a
    // 2-deep ring (stage kt % 2).
    u32x4 a_st[2][A_PER_T];          // A tile chunks of this thread
    float d_st[2];                   // d_a of row tid % BM (even K steps)
    u32x4 b_st[2];                   // 8 block sums of row (tid/2) % BM (even K steps)
    u32x4 q_st[D][TN][2];            // this lane's 32 bytes of nibbles, per column tile
    u32x4 h_st[D][TN];               // super-block header (even K steps)

    // Stage indices are compile-time constants (generic lambdas over integral_constant),
    // so the rings stay in registers.  n_kt is a multiple of D (even): stage s only ever
    // holds K steps kt with kt % D == s, hence of parity s & 1.
    auto issue_w = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);      // global K step
        const int sb = kt >> 1;
        const uint8_t * wbase = W + (size_t)sb * SB_Q4_K;
#pragma unroll
        for (int t = 0; t < TN; t++) {
            if (h == 0) h_st[s][t] = *(const u32x4 *)(wbase + off_w[t]);
            q_st[s][t][0] = *(const u32x4 *)(wbase + off_w[t] + 16 + 32 * (2 * h + hl));
            q_st[s][t][1] = *(const u32x4 *)(wbase + off_w[t] + 32 + 32 * (2 * h + hl));
        }
    };
    auto issue_a = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);
        const int sb = kt >> 1;
        const uint8_t * abase = Aq + (size_t)kt * 8192;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) a_st[s][i] = *(const u32x4 *)(abase + off_a[i]);
        if (h == 0) {
            d_st[s] = *(const float *)(Adg + (size_t)sb * m_pad * 4 + off_d);
            b_st[s] = *(const u32x4 *)(Absg + (size_t)sb * 32 + off_b);
        }
    };

    float16v P[TM][TN], S[TM][TN], T[TM][TN];
    const float16v zero16 = {};
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int t = 0; t < TN; t++) { P[i][t] = zero16; S[i][t] = zero16; T[i][t] = zero16; }
    u32x4 hdr[TN];
    q4k_sm sm[TN];
    const uint32_t MASK_LO = opaque(0x000F000Fu), MASK_HI = opaque(0x00F000F0u), MAGIC = opaque(0x64006400u);

    auto step = [&](auto stage, int kt) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1, buf = s & 1;
        const int mbuf = (kt >> 1) & 1;
        // The step's phases are fenced from the scheduler: loads moved below the
        // fence after the issue block would be waited for right after issue, and
        // ring registers refilled before their last use would need copies (and
        // waits) at the loop back-edge.
        __builtin_amdgcn_sched_barrier(0);
        // activation stage -> LDS
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            *(u32x4 *)(&As[buf][(tid + NT * i) * 8]) = a_st[buf][i];
        }
        if (h == 0) {
            // every thread stores (threads of the same row store the same value), so
            // no branch lets the compiler sink the scale loads next to these stores
            Ad[mbuf][tid % BM] = d_st[buf];
            *(u32x4 *)(&Abs[mbuf][((tid >> 1) % BM) * BST + (tid & 1) * 8]) = b_st[buf];
#pragma unroll
            for (int t = 0; t < TN; t++) {
                hdr[t] = h_st[s][t];
                sm[t] = q4k_unpack(hdr[t]);
            }
        }
        __syncthreads();
        // activations one K step ahead, then weights D-1 steps ahead.  Loads complete
        // in issue order, so the wait for the next step's activations (at the top of
        // that step) never waits for the weight loads issued here.
        issue_a(std::integral_constant<int, (s + 1) & 1>{}, kt + 1);
        issue_w(std::integral_constant<int, (s + D - 1) % D>{}, kt + D - 1);
        __builtin_amdgcn_sched_barrier(0);

        // group g = 2h + hl: scales of sub-blocks 4h + 2hl and 4h + 2hl + 1
        q4k_consts kc[TN];
#pragma unroll
        for (int t = 0; t < TN; t++) kc[t] = q4k_group_consts(h == 0 ? sm[t].sc_lo : sm[t].sc_hi, 16 * hl);
        // all A fragments of the step in flight at once (one LDS latency per step)
        half8 afr[8][TM];
#pragma unroll
        for (int kk = 0; kk < 8; kk++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                afr[kk][i] = *(const half8 *)(&As[buf][(8 * i + kk) * 512 + 8 * lane]);
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            half8 b[TN];
#pragma unroll
            for (int t = 0; t < TN; t++) b[t] = q4k_word(q_st[s][t][kk >> 2][kk & 3], kc[t], MASK_LO, MASK_HI, MAGIC);
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int t = 0; t < TN; t++)
                    P[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[kk][i], b[t],
                                                                     (h == 0 && kk == 0) ? zero16 : P[i][t], 0, 0, 0);
            }
        }

        if (h == 1) {
            // super-block complete: x = d_w*isum; x = fma(-dmin_w, msum, x); S = fma(d_a, x, S)
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const half8 bm = mins_half8(hl ? sm[t].mn_hi : sm[t].mn_lo);
                const float dw = h2f((uint16_t)(hdr[t].x & 0xFFFFu)), dmw = h2f((uint16_t)(hdr[t].x >> 16));
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const half8 a = *(const half8 *)(&Abs[mbuf][(i * 32 + l32) * BST + 8 * hl]);
                    const float16v Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bm, zero16, 0, 0, 0);
                    float dav[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const float4 da = *(const float4 *)(&Ad[mbuf][i * 32 + 8 * q4 + 4 * hl]);
                        dav[4 * q4] = da.x; dav[4 * q4 + 1] = da.y; dav[4 * q4 + 2] = da.z; dav[4 * q4 + 3] = da.w;
                    }
                    flush_dmin(S[i][t], P[i][t], Q, dw, dmw, dav);
                }
            }
        }
    };

    // same issue order as the steady state: activations, then weights
    issue_a(std::integral_constant<int, 0>{}, 0);
    issue_w(std::integral_constant<int, 0>{}, 0);
    if constexpr (D == 4) {
        issue_w(std::integral_constant<int, 1>{}, 1);
        issue_w(std::integral_constant<int, 2>{}, 2);
    }
    // chunks of SB_CHUNK super-blocks (the first at sb_first, a multiple of SB_CHUNK);
    // every chunk's K steps are a multiple of D
    for (int c0 = 0; c0 < n_kt; c0 += 2 * SB_CHUNK) {
        const int c1 = min(c0 + 2 * SB_CHUNK, n_kt);
        for (int kt0 = c0; kt0 < c1; kt0 += D) {
            step(std::integral_constant<int, 0>{}, kt0);
            step(std::integral_constant<int, 1>{}, kt0 + 1);
            if constexpr (D == 4) {
                step(std::integral_constant<int, 2>{}, kt0 + 2);
                step(std::integral_constant<int, 3>{}, kt0 + 3);
            }
        }
        // chunk complete: T = T + S
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int t = 0; t < TN; t++) {
                T[i][t] = T[i][t] + S[i][t];
                S[i][t] = zero16;
            }
    }

    // split K: the chunk sum goes to ws[z][m][n]; the reduction adds the chunks in order
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            epilogue_tile(T[i][t], m0 + i * 32, n0 + (wv * TN + t) * 32 + l32, M, N, bias, res, Y, ldy, ymap, ws, z,
                          lane, epi);
}

// ---------------------------------------------------------------------------
// Q4_K over few rows, super-blocks side by side.  Over 12-96 rows the K loop of k_q4k is a
// chain of K steps, each waiting on a barrier and on its MFMAs, with few waves to hide
// either.  Here a workgroup of eight waves computes TN 32 x 32 output tiles side by side, one
// chunk of 2048 at a time (or one chunk only, z, with ws): wave w takes super-block w of the
// chunk, loads its activation fragments once (straight from the operand-order buffer, one
// contiguous KB per 64-lane load) for all TN tiles, forms each tile's integer sums with the
// same 16 + 1 MFMAs as k_q4k and x = fma(-dmin_w, msum, d_w * isum), and leaves x and the rows'
// d_a in LDS; wave t then adds tile t's super-blocks in chunk order, S = fma(d_a, x, S), and
// T = T + S.  The operations and their order are k_q4k's, so the bits are the same; a chunk
// costs the latency of one super-block instead of eight.  TN = 1: two workgroups per CU;
// TN = 2 / 4 read the activations half / a quarter as often, one workgroup per CU.
template <int TN>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(TN == 1 ? 4 : 2)))
k_q4k_sb(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
         const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
         int n_tiles, int m_tiles, float * __restrict__ ws, dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr int NW = 8, SBC = DFX_DOT_CHUNK / 256;
    static_assert(SBC == NW, "one wave per super-block of a chunk");
    extern __shared__ __attribute__((aligned(16))) float4 X[];   // [NW][TN][4][64]: x of super-block w, tile t
    float * Dl = (float *)(X + NW * TN * 4 * 64);                 // [NW][32]: d_a of super-block w, rows m0..

    // tile order as k_q4k: column tile x on XCD x % 8, its row tiles and chunks there too
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int z = blockIdx.x / per_pass, L = blockIdx.x - z * per_pass, xcd = L & 7, j = L >> 3;
    const int ty = j % m_tiles, tx = 8 * (j / m_tiles) + xcd;
    if (tx >= n_tiles) return;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hl = lane >> 5, l32 = lane & 31;
    const int n0 = tx * 32 * TN, m0 = ty * 32;
    const int n_sb_all = K >> 8, n_chunks = (n_sb_all + SBC - 1) / SBC;
    const uint32_t row_bytes = (uint32_t)n_sb_all * SB_Q4_K;
    const act_layout Lay = act_layout_of(CONV_Q8_K_P4, M, K);
    const int m_pad = (int)act_q_rows(CONV_Q8_K_P4, M);
    const uint8_t * Aq = act + Lay.q + (size_t)(m0 / 32) * (size_t)(K / 128) * 8192 + (size_t)lane * 16;
    const float * Adg = (const float *)(act + Lay.d);
    const uint8_t * Absg = act + Lay.bs;
    const int m_bs = min(m0 + l32, M - 1);
    const uint32_t MASK_LO = opaque(0x000F000Fu), MASK_HI = opaque(0x00F000F0u), MAGIC = opaque(0x64006400u);
    const float16v zero16 = {};

    float16v T = zero16;
    const int c_first = ws ? z : 0, c_end = ws ? z + 1 : n_chunks;
    for (int c = c_first; c < c_end; c++) {
        const int sb0 = c * SBC, nsb = min(SBC, n_sb_all - sb0);
        if (wv < nsb) {
            const int sb = sb0 + wv;
            // every load of the super-block issued before the first use
            u32x4 hdr[TN], q[TN][2][2];
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const uint8_t * wb = W + (size_t)min(n0 + 32 * t + l32, N - 1) * row_bytes + (size_t)sb * SB_Q4_K;
                hdr[t] = *(const u32x4 *)wb;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    q[t][h][0] = *(const u32x4 *)(wb + 16 + 32 * (2 * h + hl));
                    q[t][h][1] = *(const u32x4 *)(wb + 32 + 32 * (2 * h + hl));
                }
            }
            half8 a[2][8];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int kk = 0; kk < 8; kk++) a[h][kk] = *(const half8 *)(Aq + (size_t)(2 * sb + h) * 8192 + kk * 1024);
            const half8 bsa = *(const half8 *)(Absg + ((size_t)m_bs * (size_t)(K / 16) + (size_t)sb * 16 + 8 * hl) * 2);
            const float dav = Adg[(size_t)sb * m_pad + m_bs];

#pragma unroll
            for (int t = 0; t < TN; t++) {
                const q4k_sm sm = q4k_unpack(hdr[t]);
                float16v P = zero16;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const q4k_consts kc = q4k_group_consts(h == 0 ? sm.sc_lo : sm.sc_hi, 16 * hl);
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) {
                        const half8 b = q4k_word(q[t][h][kk >> 2][kk & 3], kc, MASK_LO, MASK_HI, MAGIC);
                        P = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[h][kk], b, (h == 0 && kk == 0) ? zero16 : P, 0, 0,
                                                                   0);
                    }
                }
                const float16v Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsa, mins_half8(hl ? sm.mn_hi : sm.mn_lo),
                                                                          zero16, 0, 0, 0);
                const float dw = h2f((uint16_t)(hdr[t].x & 0xFFFFu)), dmw = h2f((uint16_t)(hdr[t].x >> 16));
                float x[16];
#pragma unroll
                for (int r = 0; r < 16; r++) x[r] = dw * P[r];
                pass_barrier(x);
#pragma unroll
                for (int r = 0; r < 16; r++) x[r] = fmaf(-dmw, Q[r], x[r]);
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++)
                    X[((wv * TN + t) * 4 + q4) * 64 + lane] = make_float4(x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2],
                                                                          x[4 * q4 + 3]);
            }
            if (hl == 0) Dl[wv * 32 + l32] = dav;
        }
        __syncthreads();
        if (wv < TN) {
            // tile wv: the chunk's super-blocks in order, S = fma(d_a, x, S), then T = T + S
            float16v S = zero16;
            for (int w = 0; w < nsb; w++) {
                float da[16], xv[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const float4 d4 = *(const float4 *)(&Dl[w * 32 + 8 * q4 + 4 * hl]);
                    const float4 x4 = X[((w * TN + wv) * 4 + q4) * 64 + lane];
                    da[4 * q4] = d4.x; da[4 * q4 + 1] = d4.y; da[4 * q4 + 2] = d4.z; da[4 * q4 + 3] = d4.w;
                    xv[4 * q4] = x4.x; xv[4 * q4 + 1] = x4.y; xv[4 * q4 + 2] = x4.z; xv[4 * q4 + 3] = x4.w;
                }
#pragma unroll
                for (int r = 0; r < 16; r++) S[r] = fmaf(da[r], xv[r], S[r]);
            }
            T = T + S;
        }
        if (c + 1 < c_end) __syncthreads();   // X and Dl are refilled by the next chunk
    }
    if (wv < TN) epilogue_tile(T, m0, n0 + 32 * wv + l32, M, N, bias, res, Y, ldy, ymap, ws, z, lane, epi);
}

// ---------------------------------------------------------------------------
// Q4_K, many rows: each wave computes 64 x 64 outputs (2 x 2 MFMA tiles, every A
// operand feeds two MFMAs), four waves side by side make a 64 x 256 workgroup tile,
// one workgroup per CU.  Everything a K step (128 elements) needs is requested
// DEPTH-1 steps ahead, nine loads per wave and step, in this order:
//   4 copies global -> LDS of the step's fragment-ordered A (16 KB per workgroup);
//   1 copy global -> LDS: even steps the super-block headers of the wave's 64
//     weight rows, odd steps the super-block's activation scales (d_a by waves 0
//     and 3, the block sums of rows 0-31 / 32-63 by waves 1 / 2);
//   4 loads of the wave's packed nibbles (32 bytes per lane and row): with DEPTH 2 straight
//     into a two-slot register ring (2-3.5 % faster than through LDS), with DEPTH 4 as copies
//     into LDS.
// The other rings (DEPTH slots) are in LDS.
// Loads complete in issue order, so "this wave's copies for step kt are done" is a
// wait for all but the loads issued after them; a barrier then makes every wave's
// copies visible.  Sums and their order: as k_q4k.
__host__ __device__ constexpr int waitcnt_vm_lgkm(int vm, int lgkm) {
    return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | ((vm >> 4) << 14);
}
// Workgroup barrier without the memory fence of __syncthreads (whose release would
// wait for every outstanding load, the copies to LDS included); the empty asm with a
// memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_only() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
typedef __attribute__((address_space(3))) void * lds_ptr;

template <int TM, int TN, int DEPTH>
__global__ void __launch_bounds__(256, TN == 1 ? 2 : 1)
k_q4k_w(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
        const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
        int n_tiles, int m_tiles, float * __restrict__ ws, dfx_epi epi, int n_full) {
#pragma clang fp contract(off)
    constexpr int BM = 32 * TM, BN = 128 * TN, WSZ = 2048 * TN;   // WSZ: nibble bytes per wave and step
    constexpr int NA = 2 * TM;                                     // A operand copies per wave and step
    static_assert(DEPTH == 2 || DEPTH == 4, "ring depth 2 or 4");
    static_assert(TN == 1 || TN == 2, "one or two column tiles per wave");
    static_assert(TM == 2 || TM == 3, "64- or 96-row tiles");
    // Separate arrays per ring slot: the compiler then knows that reading one slot
    // does not have to wait for the copies in flight into the others.
    __shared__ __attribute__((aligned(1024))) half_t As0[BM * 128], As1[BM * 128], As2[DEPTH > 2 ? BM * 128 : 8],
        As3[DEPTH > 2 ? BM * 128 : 8];
    // nibble slots: [wave][t][j][lane][16 B], j = the two 16-byte halves of a lane's 32 bytes
    __shared__ __attribute__((aligned(1024))) uint8_t Ws0[DEPTH > 2 ? 4 * WSZ : 16], Ws1[DEPTH > 2 ? 4 * WSZ : 16],
        Ws2[DEPTH > 2 ? 4 * WSZ : 16], Ws3[DEPTH > 2 ? 4 * WSZ : 16];
    // header slots: [wave][lane][16 B] (TN 2: lane = t*32 + row; TN 1: rows repeat in both halves)
    __shared__ __attribute__((aligned(1024))) uint8_t Hs0[4 * 1024], Hs1[DEPTH > 2 ? 4 * 1024 : 16];
    // scale slots: [0, TM KB) block sums [row][16], [TM KB, TM KB + 1 KB) d of rows m0.. (BM used)
    __shared__ __attribute__((aligned(1024))) uint8_t Sc0[(TM + 1) * 1024], Sc1[DEPTH > 2 ? (TM + 1) * 1024 : 16];
    auto aslot = [&](auto stage) __attribute__((always_inline)) -> half_t * {
        constexpr int s = decltype(stage)::value;
        if constexpr (s == 0) return As0;
        else if constexpr (s == 1) return As1;
        else if constexpr (s == 2) return As2;
        else return As3;
    };
    auto wslot = [&](auto stage) __attribute__((always_inline)) -> uint8_t * {
        constexpr int s = decltype(stage)::value;
        if constexpr (s == 0) return Ws0;
        else if constexpr (s == 1) return Ws1;
        else if constexpr (s == 2) return Ws2;
        else return Ws3;
    };

    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    // Tile L (numbered as the grid without split).  With ws and no tile counters every tile's
    // K range is split at chunk borders (z = chunk).  With counters (two chunks): workgroups
    // 0 .. n_full-1 take whole tiles, the others half tiles, the two halves of tile L being
    // workgroups n_full + 16q + e and n_full + 16q + 8 + e (L = n_full + 8q + e): both on
    // XCD L mod 8, so the halves meet in one L2.
    int z, L, cpart = 0;
    bool half = false;
    int32_t * const cnt = epi.tile_cnt;
    if (cnt) {
        const int B = blockIdx.x;
        if (B < n_full) {
            L = B;
        } else {
            const int u = B - n_full;
            L = n_full + 8 * (u >> 4) + (u & 7);
            cpart = (u >> 3) & 1;
            half = true;
        }
        z = 0;
    } else {
        z = blockIdx.x / per_pass;
        L = blockIdx.x - z * per_pass;
    }
    const int xcd = L & 7, j = L >> 3;
    const int ty = j % m_tiles, tx = 8 * (j / m_tiles) + xcd;
    if (tx >= n_tiles) return;

    const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = tx * BN, m0 = ty * BM;
    constexpr int SB_CHUNK = DFX_DOT_CHUNK / 256;
    const int n_sb_all = K >> 8;
    const bool split = cnt ? half : ws != nullptr;
    const int sb_first = split ? (cnt ? cpart : z) * SB_CHUNK : 0;
    const int n_sb = split ? min(SB_CHUNK, n_sb_all - sb_first) : n_sb_all;
    const int n_kt = 2 * n_sb;
    const uint32_t row_bytes = (uint32_t)n_sb_all * SB_Q4_K;
    const act_layout Lay = act_layout_of(CONV_Q8_K_P4, M, K);
    const int m_pad = (int)act_q_rows(CONV_Q8_K_P4, M);

    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, 0xFFFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void *)act, 0, (int)Lay.bytes, 0x00020000);

    // per-lane byte offsets (fixed); the step moves only the scalar offsets
    // (arrays here have fixed sizes: this clang drops the host stub of a kernel template whose
    // lambdas capture a local array sized by a template parameter)
    uint32_t off_a[6];   // this wave copies A operands NA*wv.. of the step: row tile f/8, operand f%8
#pragma unroll
    for (int f = 0; f < NA; f++) {
        const int ff = NA * wv + f, mt = min(m0 / 32 + (ff >> 3), m_pad / 32 - 1);
        off_a[f] = (uint32_t)Lay.q + (uint32_t)mt * (uint32_t)(K / 128) * 8192u + (uint32_t)(ff & 7) * 1024u +
                   (uint32_t)lane * 16u;
    }
    // (fixed size: this clang drops the host stub of a kernel template whose lambdas
    // capture a local array sized by a template parameter)
    uint32_t off_w[2];
#pragma unroll
    for (int t = 0; t < TN; t++) off_w[t] = (uint32_t)min(n0 + (wv * TN + t) * 32 + l32, N - 1) * row_bytes;
    const uint32_t off_h = (uint32_t)min(n0 + 32 * TN * wv + (TN == 2 ? lane : l32), N - 1) * row_bytes;
    // scale copies (16 bytes a lane): waves below TM the block sums of rows 32 wv + lane/2,
    // the others the same 1 KB of d from row m0 on (d is [sb][m_pad]; BM of those rows
    // are used; lanes past the buffer's end read nothing: the buffer's extent is set)
    const bool bs_wave = wv < TM;
    const uint32_t off_s = bs_wave
        ? (uint32_t)Lay.bs + ((uint32_t)min(m0 + 32 * wv + (lane >> 1), M - 1) * (uint32_t)(K / 16) +
                              (lane & 1) * 8u) * 2u
        : (uint32_t)Lay.d + (uint32_t)m0 * 4u + (uint32_t)lane * 16u;
    const int s_step = bs_wave ? 32 : m_pad * 4;   // bytes per super-block

    // Header and scale slots alternate with the super-block (DEPTH 4: the slot of the
    // steps of stage s is (s / 2) % 2, as every chunk starts at an even super-block and
    // on a multiple of 4 steps); with DEPTH 2 one slot each suffices.
    auto hslot = [&](auto stage) __attribute__((always_inline)) -> uint8_t * {
        constexpr int s = decltype(stage)::value;
        if constexpr (DEPTH == 4 && ((s >> 1) & 1)) return Hs1;
        else return Hs0;
    };
    auto sslot = [&](auto stage) __attribute__((always_inline)) -> uint8_t * {
        constexpr int s = decltype(stage)::value;
        if constexpr (DEPTH == 4 && ((s >> 1) & 1)) return Sc1;
        else return Sc0;
    };
    const int sc_dst = bs_wave ? 1024 * wv : 1024 * TM;   // this wave's copy within a scale slot

    u32x4 qwr[2][TN][2];   // DEPTH 2: nibble ring [step parity][column tile][16-byte word]
    auto issue = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);
        const int sb = kt >> 1;
#pragma unroll
        for (int f = 0; f < NA; f++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)(aslot(stage) + (NA * wv + f) * 512), 16, off_a[f],
                                                     kt * 8192, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (h == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_ptr)(hslot(stage) + 1024 * wv), 16, off_h, sb * SB_Q4_K,
                                                     0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)(sslot(stage) + sc_dst), 16, off_s,
                                                     sb * s_step, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
            for (int jj = 0; jj < 2; jj++) {
                if constexpr (DEPTH == 2)
                    qwr[h][t][jj] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                  rW, off_w[t] + 16 + 16 * jj + 32 * hl,
                                                                  sb * SB_Q4_K + 64 * h, 0));
                else
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_ptr)(wslot(stage) + WSZ * wv + 1024 * (2 * t + jj)),
                                                             16, off_w[t] + 16 + 16 * jj + 32 * hl, sb * SB_Q4_K + 64 * h,
                                                             0, 0);
            }
    };
    // per step: NA + 1 + 2*TN loads; after a step's copies of A and its header / scale
    // copy come its 2*TN nibble copies and DEPTH-2 whole steps
    // at the top of a step: this step's A and header / scale copies (the shared ones, made
    // visible to every wave by the barrier that follows); its nibble copies (issued last,
    // read only by the wave that made them) may still be in flight, and so may the DEPTH-2
    // later steps' copies.  Before the nibble words are read: the step's nibble copies, with
    // only the DEPTH-1 later steps' copies in flight.
    constexpr int WAIT_TOP = waitcnt_vm_lgkm(2 * TN + (NA + 1 + 2 * TN) * (DEPTH - 2), 0);
    constexpr int WAIT_NIB = waitcnt_vm_lgkm((NA + 1 + 2 * TN) * (DEPTH - 1), 15);   // (no LDS-read wait)

    float16v P[TM][TN], S[TM][TN], T[TM][TN];
    const float16v zero16 = {};
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int t = 0; t < TN; t++) { P[i][t] = zero16; S[i][t] = zero16; T[i][t] = zero16; }
    q4k_sm sm[TN];
    float dw[TN], dmw[TN];
    const uint32_t MASK_LO = opaque(0x000F000Fu), MASK_HI = opaque(0x00F000F0u), MAGIC = opaque(0x64006400u);

    auto step = [&](auto stage, int kt) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(WAIT_TOP);
        barrier_only();
        __builtin_amdgcn_sched_barrier(0);
        issue(std::integral_constant<int, (s + DEPTH - 1) % DEPTH>{}, kt + DEPTH - 1);
        __builtin_amdgcn_sched_barrier(0);
        if (h == 0) {
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const u32x4 hdr = *(const u32x4 *)(hslot(stage) + 1024 * wv + 16 * (32 * t + l32));
                sm[t] = q4k_unpack(hdr);
                dw[t] = h2f((uint16_t)(hdr.x & 0xFFFFu));
                dmw[t] = h2f((uint16_t)(hdr.x >> 16));
            }
        }
        // the step's A operands and nibble words requested together (one LDS latency); with
        // 96 rows the A operands come in two halves of four K slices, to fit two waves per SIMD
        constexpr int KH = TM == 3 ? 2 : 1, KPH = 8 / KH;
        half8 afr[8][3];   // [KPH][TM] used
        auto read_a = [&](int part) __attribute__((always_inline)) {
#pragma unroll
            for (int kq = 0; kq < KPH; kq++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    afr[kq][i] = *(const half8 *)(aslot(stage) + (8 * i + KPH * part + kq) * 512 + 8 * lane);
        };
        read_a(0);
        u32x4 qw[TN][2];
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(WAIT_NIB);   // this wave's nibble copies for the step
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
            for (int jj = 0; jj < 2; jj++) {
                if constexpr (DEPTH == 2) qw[t][jj] = qwr[h][t][jj];
                else qw[t][jj] = *(const u32x4 *)(wslot(stage) + WSZ * wv + 1024 * (2 * t + jj) + 16 * lane);
            }
        __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the MFMAs
        q4k_consts kc[TN];
#pragma unroll
        for (int t = 0; t < TN; t++) kc[t] = q4k_group_consts(h == 0 ? sm[t].sc_lo : sm[t].sc_hi, 16 * hl);
#pragma unroll
        for (int part = 0; part < KH; part++) {
            if (part) read_a(part);
#pragma unroll
            for (int kq = 0; kq < KPH; kq++) {
                const int kk = KPH * part + kq;
                half8 b[TN];
#pragma unroll
                for (int t = 0; t < TN; t++) b[t] = q4k_word(qw[t][kk >> 2][kk & 3], kc[t], MASK_LO, MASK_HI, MAGIC);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int t = 0; t < TN; t++)
                        P[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[kq][i], b[t],
                                                                         (h == 0 && kk == 0) ? zero16 : P[i][t], 0, 0, 0);
            }
        }
#ifdef DFX_W_INTERLEAVE
        // interleave: every MFMA followed by a few VALU instructions (the next
        // operands' dequantisation), so that the VALU work runs under the MFMAs
#pragma unroll
        for (int g = 0; g < 8 * TM * TN; g++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // 1 MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, DFX_W_INTERLEAVE, 0);   // VALU
        }
#endif

        if (h == 1) {
            // super-block complete: x = d_w*isum; x = fma(-dmin_w, msum, x); S = fma(d_a, x, S)
            const half_t * Abs = (const half_t *)sslot(stage);
            const float * Ad = (const float *)(sslot(stage) + 1024 * TM);
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const half8 bm = mins_half8(hl ? sm[t].mn_hi : sm[t].mn_lo);
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const half8 av = *(const half8 *)(Abs + (i * 32 + l32) * 16 + 8 * hl);
                    const float16v Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bm, zero16, 0, 0, 0);
                    float dav[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const float4 da = *(const float4 *)(Ad + i * 32 + 8 * q4 + 4 * hl);
                        dav[4 * q4] = da.x; dav[4 * q4 + 1] = da.y; dav[4 * q4 + 2] = da.z; dav[4 * q4 + 3] = da.w;
                    }
                    flush_dmin(S[i][t], P[i][t], Q, dw[t], dmw[t], dav);
                }
            }
        }
    };

    // steps 0 .. DEPTH-2 requested up front; step kt requests step kt + DEPTH - 1
    issue(std::integral_constant<int, 0>{}, 0);
    if constexpr (DEPTH == 4) {
        issue(std::integral_constant<int, 1>{}, 1);
        issue(std::integral_constant<int, 2>{}, 2);
    }
    for (int c0 = 0; c0 < n_kt; c0 += 2 * SB_CHUNK) {
        const int c1 = min(c0 + 2 * SB_CHUNK, n_kt);
        for (int kt0 = c0; kt0 < c1; kt0 += DEPTH) {
            step(std::integral_constant<int, 0>{}, kt0);
            step(std::integral_constant<int, 1>{}, kt0 + 1);
            if constexpr (DEPTH == 4) {
                step(std::integral_constant<int, 2>{}, kt0 + 2);
                step(std::integral_constant<int, 3>{}, kt0 + 3);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int t = 0; t < TN; t++) {
                T[i][t] = T[i][t] + S[i][t];
                S[i][t] = zero16;
            }
    }
    // the copies issued past the last step still land in this workgroup's LDS: let
    // them finish before the workgroup (and its LDS) can end
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(0, 0));

    if (half) {
        // half tile: chunk total T = 0 + S_c to ws[c]; the later of the tile's two halves reads
        // the other's and forms (0 + S_0) + (0 + S_1), which equals the whole tile's
        // (0 + S_0) + S_1 (0 + x is never -0), then applies the epilogue.  Its stores complete
        // in the XCD's L2 before the counter's atomic there; the partner's loads of lines it
        // never touched miss its own vector L1.  No workgroup waits for another.
        __shared__ int first;
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                epilogue_tile(T[i][t], m0 + i * 32, n0 + (wv * TN + t) * 32 + l32, M, N, nullptr, nullptr, nullptr, 0,
                              nullptr, ws, cpart, lane, epi);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(0, 15));
        __syncthreads();
        if (tid == 0) {
            // The handover relies on both halves sharing one L2, i.e. on workgroup L being
            // dispatched to XCD L mod 8.  Each half adds 1 + 16 * (its XCC id) to the counter;
            // the later half compares the earlier one's id with its own and, if they differ
            // (the totals it is about to read may be stale), raises the sticky flag cnt[1],
            // which the host checks after the pass.
            const int xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15;   // HW_REG_XCC_ID[3:0]
            const int old = __hip_atomic_fetch_add(cnt + 32 * L, 1 + 16 * xcc, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            first = old == 0;
            if (!first && (old >> 4) != xcc) cnt[1] = 1;
        }
        __syncthreads();
        if (first) return;
        const float * other = ws + (int64_t)(1 - cpart) * M * N;
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int n = n0 + (wv * TN + t) * 32 + l32;
                float o[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + i * 32 + tile_row(r, lane);
                    o[r] = (m < M && n < N) ? other[(int64_t)m * N + n] : 0.0f;
                }
#pragma unroll
                for (int r = 0; r < 16; r++) T[i][t][r] = cpart == 0 ? T[i][t][r] + o[r] : o[r] + T[i][t][r];
            }
        if (tid == 0) cnt[32 * L] = 0;   // ready for the next call
    }
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            epilogue_tile(T[i][t], m0 + i * 32, n0 + (wv * TN + t) * 32 + l32, M, N, bias, res, Y, ldy, ymap,
                          cnt ? nullptr : ws, z, lane, epi);
}

// ---------------------------------------------------------------------------
// Q6_K: the same pipeline as Q4_K (register rings, A tile in LDS, chunked K)
// ---------------------------------------------------------------------------
// A K step is half a super-block (128 elements).  Lane (row n, half g = lane/32) holds
// l = 16g..16g+15 of every quarter: 16 bytes of ql for quarters 0/2, 16 for quarters
// 1/3 and 16 of qh.  MFMA kk = i + 4p takes word i of the ql bytes of quarters p / p+2
// (low / high nibbles) and word i of qh.  q6 - 32 = lo4 + 16*(hi2 - 2) is split into two
// exact f16 operands that go to two MFMAs into the same accumulator:
//   sc*lo4:          (lo4 at bits 3..6) | 0x5800 = 128 + lo4,  x*sc - 128*sc
//   16*sc*(hi2-2):   (hi2 at bits 8..9) | 0x4400 = 4 + hi2,    x*(16*sc) - 96*sc
// (|sc| <= 128: every constant and result is an exact f16).  The activation buffer
// stores q in the matching slot order (CONV_Q8_K_P6).  The flush of a super-block is
// x = d_w*isum; S = fma(d_a, x, S).

struct q6k_qc { uint32_t s, c, s16, c96; };
__device__ __forceinline__ q6k_qc q6k_quarter_consts(int sc) {
    const float f = (float)sc;
    q6k_qc k;
    k.s = h2pair(f);
    k.c = h2pair(-128.0f * f);
    k.s16 = h2pair(16.0f * f);
    k.c96 = h2pair(-96.0f * f);
    return k;
}

// Signed scale byte k (0..15) of the 16 scale bytes held in sc4.
__device__ __forceinline__ int q6k_scale(const u32x4 & sc4, int k) {
    const uint32_t w = sc4[k >> 2];
    return (int)(int8_t)((w >> (8 * (k & 3))) & 0xFFu);
}

// Operands of MFMA kk = i + 4p: lo = sc*lo4 part, hi = 16*sc*(hi2-2) part, order
// [qa: b0 b2 b1 b3 | qb: b0 b2 b1 b3], qa = p, qb = p + 2.
__device__ __forceinline__ void q6k_word(int P, uint32_t w, uint32_t hw, const q6k_qc & ka, const q6k_qc & kb,
                                         half8 & lo, half8 & hi, uint32_t m78, uint32_t mg58, uint32_t m300,
                                         uint32_t mg44) {
    u32x4 a, b;
    a.x = pk_fma_h2(and_or(w << 3, m78, mg58), ka.s, ka.c);
    a.y = pk_fma_h2(and_or(w >> 5, m78, mg58), ka.s, ka.c);
    a.z = pk_fma_h2(and_or(w >> 1, m78, mg58), kb.s, kb.c);
    a.w = pk_fma_h2(and_or(w >> 9, m78, mg58), kb.s, kb.c);
    const int qa = P, qb = P + 2;    // 2-bit fields at bits 2q (+8 per byte): moved to bits 8..9 of each half
    b.x = pk_fma_h2(and_or(hw << (8 - 2 * qa), m300, mg44), ka.s16, ka.c96);
    b.y = pk_fma_h2(and_or(hw >> (2 * qa), m300, mg44), ka.s16, ka.c96);
    b.z = pk_fma_h2(and_or(hw << (8 - 2 * qb), m300, mg44), kb.s16, kb.c96);
    b.w = pk_fma_h2(and_or(hw >> (2 * qb), m300, mg44), kb.s16, kb.c96);
    lo = __builtin_bit_cast(half8, a);
    hi = __builtin_bit_cast(half8, b);
}

template <int TM, int TN, int D>
__global__ void __launch_bounds__(256, TM * TN >= 4 ? 1 : 2)
k_q6k(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
      const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
      int n_tiles, int m_tiles, float * __restrict__ ws, dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr int BM = TM * 32, BN = 4 * TN * 32;
    constexpr int A_PER_T = BM * 16 / 256;
    __shared__ __attribute__((aligned(16))) half_t As[2][BM * 128];   // fragment order, as in k_q4k
    __shared__ __attribute__((aligned(16))) float Ad[2][BM];

    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int z = blockIdx.x / per_pass, L = blockIdx.x - z * per_pass, xcd = L & 7, j = L >> 3;
    const int ty = j % m_tiles, tx = 8 * (j / m_tiles) + xcd;
    if (tx >= n_tiles) return;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hl = lane >> 5, l32 = lane & 31;
    const int n0 = tx * BN, m0 = ty * BM;
    constexpr int SB_CHUNK = DFX_DOT_CHUNK / 256;
    const int n_sb_all = K >> 8;
    const int sb_first = ws ? z * SB_CHUNK : 0;
    const int n_sb = ws ? min(SB_CHUNK, n_sb_all - sb_first) : n_sb_all;
    const int n_kt = 2 * n_sb;
    const uint32_t row_bytes = (uint32_t)n_sb_all * SB_Q6_K;
    const act_layout Lay = act_layout_of(CONV_Q8_K_P6, M, K);
    const int m_pad = (int)act_q_rows(CONV_Q8_K_P6, M);
    const uint8_t * Aq = act + Lay.q;
    const uint8_t * Adg = act + Lay.d;

    uint32_t off_a[A_PER_T], off_w[TN];
#pragma unroll
    for (int i = 0; i < A_PER_T; i++) {
        // chunk c of the step: row tile c / 512 (clamped to the padded rows), 16 bytes c % 512
        const int c = tid + 256 * i, mt = min(m0 / 32 + (c >> 9), m_pad / 32 - 1);
        off_a[i] = (uint32_t)mt * (uint32_t)(K / 128) * 8192u + (uint32_t)(c & 511) * 16u;
    }
#pragma unroll
    for (int t = 0; t < TN; t++) off_w[t] = (uint32_t)min(n0 + (wv * TN + t) * 32 + l32, N - 1) * row_bytes;
    const uint32_t off_d = (uint32_t)min(m0 + tid % BM, M - 1) * 4u;   // d is [sb][m_pad]

    u32x4 a_st[2][A_PER_T];
    float d_st[2];
    u32x4 l_st[D][TN][2];            // ql bytes: quarters 0/2 and 1/3 at l = 16g..16g+15
    u32x4 qh_st[D][TN];              // qh bytes at l = 16g..16g+15
    u32x4 sc_st[D][TN];              // 16 scale bytes (even K steps)
    uint32_t dw_st[D][TN];           // d (low 16 bits) (even K steps)

    auto issue_w = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);
        const int sb = kt >> 1;
        const uint8_t * wbase = W + (size_t)sb * SB_Q6_K;
#pragma unroll
        for (int t = 0; t < TN; t++) {
            const uint8_t * p = wbase + off_w[t];
            l_st[s][t][0] = *(const u32x4 *)(p + 64 * h + 16 * hl);
            l_st[s][t][1] = *(const u32x4 *)(p + 64 * h + 32 + 16 * hl);
            qh_st[s][t] = *(const u32x4 *)(p + 128 + 32 * h + 16 * hl);
            if (h == 0) {
                sc_st[s][t] = *(const u32x4 *)(p + 192);
                dw_st[s][t] = *(const uint32_t *)(p + 208);
            }
        }
    };
    auto issue_a = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1;
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);
        const int sb = kt >> 1;
        const uint8_t * abase = Aq + (size_t)kt * 8192;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) a_st[s][i] = *(const u32x4 *)(abase + off_a[i]);
        if (h == 0) d_st[s] = *(const float *)(Adg + (size_t)sb * m_pad * 4 + off_d);
    };

    float16v P[TM][TN], S[TM][TN], T[TM][TN];
    const float16v zero16 = {};
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int t = 0; t < TN; t++) { P[i][t] = zero16; S[i][t] = zero16; T[i][t] = zero16; }
    u32x4 sc4[TN];
    uint32_t dwh[TN];
    const uint32_t M78 = opaque(0x00780078u), MG58 = opaque(0x58005800u), M300 = opaque(0x03000300u),
                   MG44 = opaque(0x44004400u);

    auto step = [&](auto stage, int kt) __attribute__((always_inline)) {
        constexpr int s = decltype(stage)::value, h = s & 1, buf = s & 1;
        const int mbuf = (kt >> 1) & 1;
        __builtin_amdgcn_sched_barrier(0);     // phases fenced as in k_q4k
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            *(u32x4 *)(&As[buf][(tid + 256 * i) * 8]) = a_st[buf][i];
        }
        if (h == 0) {
            Ad[mbuf][tid % BM] = d_st[buf];     // duplicates store the same value
#pragma unroll
            for (int t = 0; t < TN; t++) { sc4[t] = sc_st[s][t]; dwh[t] = dw_st[s][t]; }
        }
        __syncthreads();
        issue_a(std::integral_constant<int, (s + 1) & 1>{}, kt + 1);
        issue_w(std::integral_constant<int, (s + D - 1) % D>{}, kt + D - 1);
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int p = 0; p < 2; p++) {
            // quarters p and p+2 of this half: sub-blocks 8h + 2q + g
            q6k_qc ka[TN], kb[TN];
#pragma unroll
            for (int t = 0; t < TN; t++) {
                ka[t] = q6k_quarter_consts(q6k_scale(sc4[t], 8 * h + 2 * p + hl));
                kb[t] = q6k_quarter_consts(q6k_scale(sc4[t], 8 * h + 2 * (p + 2) + hl));
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = i + 4 * p;
                half8 blo[TN], bhi[TN];
#pragma unroll
                for (int t = 0; t < TN; t++)
                    q6k_word(p, l_st[s][t][p][i], qh_st[s][t][i], ka[t], kb[t], blo[t], bhi[t], M78, MG58, M300,
                             MG44);
#pragma unroll
                for (int ii = 0; ii < TM; ii++) {
                    const half8 a = *(const half8 *)(&As[buf][(8 * ii + kk) * 512 + 8 * lane]);
#pragma unroll
                    for (int t = 0; t < TN; t++) {
                        P[ii][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, blo[t],
                                                                          (h == 0 && kk == 0) ? zero16 : P[ii][t],
                                                                          0, 0, 0);
                        P[ii][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bhi[t], P[ii][t], 0, 0, 0);
                    }
                }
            }
        }

        if (h == 1) {
            // super-block complete: x = d_w*isum; S = fma(d_a, x, S)
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const float dw = h2f((uint16_t)(dwh[t] & 0xFFFFu));
#pragma unroll
                for (int ii = 0; ii < TM; ii++) {
                    float dav[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const float4 da = *(const float4 *)(&Ad[mbuf][ii * 32 + 8 * q4 + 4 * hl]);
                        dav[4 * q4] = da.x; dav[4 * q4 + 1] = da.y; dav[4 * q4 + 2] = da.z; dav[4 * q4 + 3] = da.w;
                    }
                    flush_d(S[ii][t], P[ii][t], dw, dav);
                }
            }
        }
    };

    // same issue order as the steady state: activations, then weights
    issue_a(std::integral_constant<int, 0>{}, 0);
    issue_w(std::integral_constant<int, 0>{}, 0);
    if constexpr (D == 4) {
        issue_w(std::integral_constant<int, 1>{}, 1);
        issue_w(std::integral_constant<int, 2>{}, 2);
    }
    for (int c0 = 0; c0 < n_kt; c0 += 2 * SB_CHUNK) {
        const int c1 = min(c0 + 2 * SB_CHUNK, n_kt);
        for (int kt0 = c0; kt0 < c1; kt0 += D) {
            step(std::integral_constant<int, 0>{}, kt0);
            step(std::integral_constant<int, 1>{}, kt0 + 1);
            if constexpr (D == 4) {
                step(std::integral_constant<int, 2>{}, kt0 + 2);
                step(std::integral_constant<int, 3>{}, kt0 + 3);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int t = 0; t < TN; t++) {
                T[i][t] = T[i][t] + S[i][t];
                S[i][t] = zero16;
            }
    }

#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            epilogue_tile(T[i][t], m0 + i * 32, n0 + (wv * TN + t) * 32 + l32, M, N, bias, res, Y, ldy, ymap, ws, z,
                          lane, epi);
}

// ---------------------------------------------------------------------------
// Q6_K, LDS-DMA fed: k_q6k's operands, sums and flush inside k_q4k_w's pipeline.  A 64 x 128
// or 96 x 128 workgroup tile (TM = 2 or 3 row tiles of 32, four waves side by side, 32 weight
// rows each); one
// K step (128 elements, half a super-block) is requested one step ahead, in this order:
//   NA = 2 * TM copies global -> LDS of the step's fragment-ordered A (shared by the waves);
//   even steps: the 16 scale bytes and the d word of the wave's rows (register loads);
//   odd steps: the super-block's activation scales d_a of rows m0.. (one copy per wave into
//     its own 1 KB of LDS, read only by that wave);
//   three 16-byte register loads per lane of ql (quarters p and p + 2) and qh.
// Loads complete in issue order: the top-of-step wait leaves only the step's own scale and
// weight loads in flight (after the barrier the next step's loads are issued); before the
// weights are used, only the next step's loads.
template <int TM>
__global__ void __launch_bounds__(256, 2)
k_q6k_w(const uint8_t * __restrict__ W, int N, int K, const uint8_t * __restrict__ act, int M,
        const float * __restrict__ bias, const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
        int n_tiles, int m_tiles, float * __restrict__ ws, dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr int BM = 32 * TM, NA = 2 * TM;
    static_assert((TM == 2 || TM == 3) && NA <= 6, "64- or 96-row tiles");
    __shared__ __attribute__((aligned(1024))) half_t As0[BM * 128], As1[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t Ds[4 * 1024];   // [wave][1 KB]: d_a of rows m0..
    auto aslot = [&](auto stage) __attribute__((always_inline)) -> half_t * {
        if constexpr (decltype(stage)::value == 0) return As0;
        else return As1;
    };

    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int z = blockIdx.x / per_pass, L = blockIdx.x - z * per_pass, xcd = L & 7, j = L >> 3;
    const int ty = j % m_tiles, tx = 8 * (j / m_tiles) + xcd;
    if (tx >= n_tiles) return;

    const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = tx * 128, m0 = ty * BM;
    constexpr int SB_CHUNK = DFX_DOT_CHUNK / 256;
    const int n_sb_all = K >> 8;
    const int sb_first = ws ? z * SB_CHUNK : 0;
    const int n_sb = ws ? min(SB_CHUNK, n_sb_all - sb_first) : n_sb_all;
    const int n_kt = 2 * n_sb;
    const uint32_t row_bytes = (uint32_t)n_sb_all * SB_Q6_K;
    const act_layout Lay = act_layout_of(CONV_Q8_K_P6, M, K);
    const int m_pad = (int)act_q_rows(CONV_Q8_K_P6, M);

    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, 0xFFFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void *)act, 0, (int)Lay.bytes, 0x00020000);

    // (fixed size: this clang drops the host stub of a kernel template whose lambdas capture a
    // local array sized by a template parameter)
    uint32_t off_a[6];   // this wave copies A operands NA*wv.. of the step: row tile f/8, operand f%8
#pragma unroll
    for (int f = 0; f < NA; f++) {
        const int ff = NA * wv + f, mt = min(m0 / 32 + (ff >> 3), m_pad / 32 - 1);
        off_a[f] = (uint32_t)Lay.q + (uint32_t)mt * (uint32_t)(K / 128) * 8192u + (uint32_t)(ff & 7) * 1024u +
                   (uint32_t)lane * 16u;
    }
    const uint32_t off_w = (uint32_t)min(n0 + wv * 32 + l32, N - 1) * row_bytes;
    // d_a is [sb][m_pad]: 1 KB from row m0 (BM of its rows are used; lanes past the buffer's
    // end read nothing, the buffer's extent is set)
    const uint32_t off_d = (uint32_t)Lay.d + (uint32_t)m0 * 4u + (uint32_t)lane * 16u;

    u32x4 l_st[2][2], qh_st[2], sc_st;
    uint32_t dw_st;
    auto issue = [&](auto stage, int kt_req) __attribute__((always_inline)) {
        constexpr int h = decltype(stage)::value;   // DEPTH 2: the stage is the step's parity
        const int kt = 2 * sb_first + min(kt_req, n_kt - 1);
        const int sb = kt >> 1;
#pragma unroll
        for (int f = 0; f < NA; f++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)(aslot(stage) + (NA * wv + f) * 512), 16, off_a[f],
                                                     kt * 8192, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (h == 0) {
            sc_st = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, off_w + 192, sb * SB_Q6_K, 0));
            dw_st = __builtin_amdgcn_raw_buffer_load_b32(rW, off_w + 208, sb * SB_Q6_K, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)(Ds + 1024 * wv), 16, off_d, sb * m_pad * 4, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        l_st[h][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, off_w + 64 * h + 16 * hl,
                                                                                        sb * SB_Q6_K, 0));
        l_st[h][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, off_w + 64 * h + 32 + 16 * hl,
                                                                                        sb * SB_Q6_K, 0));
        qh_st[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, off_w + 128 + 32 * h + 16 * hl,
                                                                                     sb * SB_Q6_K, 0));
    };
    // loads per step after its A copies: even 2 + 3, odd 1 + 3; per step in all: NA + those
    constexpr int AFTER_A_EVEN = 5, AFTER_A_ODD = 4;

    float16v P[TM], S[TM], T[TM];
    const float16v zero16 = {};
#pragma unroll
    for (int i = 0; i < TM; i++) { P[i] = zero16; S[i] = zero16; T[i] = zero16; }
    u32x4 sc4;
    uint32_t dwh = 0;
    const uint32_t M78 = opaque(0x00780078u), MG58 = opaque(0x58005800u), M300 = opaque(0x03000300u),
                   MG44 = opaque(0x44004400u);

    auto step = [&](auto stage, int kt) __attribute__((always_inline)) {
        constexpr int h = decltype(stage)::value;
        // this step's A copies done (its scale and weight loads may still be in flight), and
        // every LDS read of the previous step done before the barrier
        constexpr int WAIT_TOP = waitcnt_vm_lgkm(h == 0 ? AFTER_A_EVEN : AFTER_A_ODD, 0);
        // everything of this step done, the next step's loads (NA + its scale and weight
        // loads) still in flight
        constexpr int WAIT_W = waitcnt_vm_lgkm(NA + (h == 0 ? AFTER_A_ODD : AFTER_A_EVEN), 15);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(WAIT_TOP);
        barrier_only();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (h == 0) {
            // the super-block's scales and d (loaded with this step) before the next step's loads
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(3, 15));
            sc4 = sc_st;
            dwh = dw_st;
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(std::integral_constant<int, h ^ 1>{}, kt + 1);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(WAIT_W);
        __builtin_amdgcn_sched_barrier(0);
        const half_t * As = aslot(stage);
#pragma unroll
        for (int p = 0; p < 2; p++) {
            // quarters p and p+2 of this half: sub-blocks 8h + 2q + g
            const q6k_qc ka = q6k_quarter_consts(q6k_scale(sc4, 8 * h + 2 * p + hl));
            const q6k_qc kb = q6k_quarter_consts(q6k_scale(sc4, 8 * h + 2 * (p + 2) + hl));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = i + 4 * p;
                half8 blo, bhi;
                q6k_word(p, l_st[h][p][i], qh_st[h][i], ka, kb, blo, bhi, M78, MG58, M300, MG44);
#pragma unroll
                for (int ii = 0; ii < TM; ii++) {
                    const half8 a = *(const half8 *)(As + (8 * ii + kk) * 512 + 8 * lane);
                    P[ii] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, blo, (h == 0 && kk == 0) ? zero16 : P[ii], 0, 0,
                                                                   0);
                    P[ii] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bhi, P[ii], 0, 0, 0);
                }
            }
        }
        if constexpr (h == 1) {
            // super-block complete: x = d_w*isum; S = fma(d_a, x, S)
            const float dw = h2f((uint16_t)(dwh & 0xFFFFu));
            const float * Ad = (const float *)(Ds + 1024 * wv);
#pragma unroll
            for (int ii = 0; ii < TM; ii++) {
                float dav[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const float4 da = *(const float4 *)(Ad + ii * 32 + 8 * q4 + 4 * hl);
                    dav[4 * q4] = da.x; dav[4 * q4 + 1] = da.y; dav[4 * q4 + 2] = da.z; dav[4 * q4 + 3] = da.w;
                }
                flush_d(S[ii], P[ii], dw, dav);
            }
        }
    };

    issue(std::integral_constant<int, 0>{}, 0);
    for (int c0 = 0; c0 < n_kt; c0 += 2 * SB_CHUNK) {
        const int c1 = min(c0 + 2 * SB_CHUNK, n_kt);
        for (int kt0 = c0; kt0 < c1; kt0 += 2) {
            step(std::integral_constant<int, 0>{}, kt0);
            step(std::integral_constant<int, 1>{}, kt0 + 1);
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
            T[i] = T[i] + S[i];
            S[i] = zero16;
        }
    }
    // the copies issued past the last step still land in this workgroup's LDS
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm(0, 0));
#pragma unroll
    for (int i = 0; i < TM; i++)
        epilogue_tile(T[i], m0 + i * 32, n0 + wv * 32 + l32, M, N, bias, res, Y, ldy, ymap, ws, z, lane, epi);
}

// ---------------------------------------------------------------------------
// F16 weights
// ---------------------------------------------------------------------------
template <int TM>
__global__ void __launch_bounds__(256, 2)
k_gemm_f16(const uint8_t * __restrict__ W, int N, int K, const half_t * __restrict__ A, int M,
           const float * __restrict__ bias, const float * res, float * Y, int64_t ldy,
           const int32_t * __restrict__ ymap, float * __restrict__ ws, int kt_per_split, dfx_epi epi) {
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
#pragma unroll
    for (int i = 0; i < TM; i++)
        epilogue_tile(acc[i], m0 + i * 32, n, M, N, bias, res, Y, ldy, ymap, split ? ws : nullptr, (int)blockIdx.z,
                      lane, epi);
}

// ---------------------------------------------------------------------------
// F32 weights (GGML's vec_dot_type of F32 is F32: activations are not converted)
// ---------------------------------------------------------------------------
// v_mfma_f32_32x32x2_f32 on f32 operands staged in LDS: workgroup = 4 waves side by side
// over 128 weight rows, TM row tiles of 32 activation rows per wave, K step 32.  The
// sums are f32-accurate (GGML sums the f32 products in double in its scalar form, in its
// own SIMD order otherwise); no activation rounding is involved, so the result stays
// within f32 rounding of the CPU value.
#define BKF 32
#define FSTR (BKF + 1)   // LDS floats per row (odd: the 32 rows a wave reads hit 32 banks)
template <int TM>
__global__ void __launch_bounds__(256, 2)
k_gemm_f32(const float * __restrict__ W, int N, int K, const float * __restrict__ A, int M,
           const float * __restrict__ bias, const float * res, float * Y, int64_t ldy,
           const int32_t * __restrict__ ymap, dfx_epi epi) {
    constexpr int BM = TM * 32, BN = 128;
    __shared__ float Ws[BN * FSTR];
    __shared__ float As[BM * FSTR];
    const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6, l32 = lane & 31, hl = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    float16v acc[TM];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BKF) {
        float4 wv[4], av[TM];
#pragma unroll
        for (int j = 0; j < 4; j++) {   // 128 rows x 8 float4
            const int c = tid + 256 * j, r = c >> 3, q = c & 7;
            const int n = min(n0 + r, N - 1);
            wv[j] = *(const float4 *)(W + (int64_t)n * K + k0 + 4 * q);
        }
#pragma unroll
        for (int j = 0; j < TM; j++) {  // BM rows x 8 float4
            const int c = tid + 256 * j, r = c >> 3, q = c & 7;
            const int m = min(m0 + r, M - 1);
            av[j] = *(const float4 *)(A + (int64_t)m * K + k0 + 4 * q);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = tid + 256 * j, r = c >> 3, q = c & 7;
            float * d = Ws + r * FSTR + 4 * q;
            d[0] = wv[j].x; d[1] = wv[j].y; d[2] = wv[j].z; d[3] = wv[j].w;
        }
#pragma unroll
        for (int j = 0; j < TM; j++) {
            const int c = tid + 256 * j, r = c >> 3, q = c & 7;
            float * d = As + r * FSTR + 4 * q;
            d[0] = av[j].x; d[1] = av[j].y; d[2] = av[j].z; d[3] = av[j].w;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BKF / 2; kk++) {
            const float b = Ws[(wn * 32 + l32) * FSTR + 2 * kk + hl];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const float a = As[(i * 32 + l32) * FSTR + 2 * kk + hl];
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[i], 0, 0, 0);
            }
        }
    }
    const int n = n0 + wn * 32 + l32;
#pragma unroll
    for (int i = 0; i < TM; i++)
        epilogue_tile(acc[i], m0 + i * 32, n, M, N, bias, res, Y, ldy, ymap, nullptr, 0, lane, epi);
}

// Fixed-order reduction of split-K partials plus epilogue: y = ((0 + p_0) + p_1 ...) + bias + res.
// Each thread takes REDUCE_R elements spaced one grid apart, so the partial loads of one chunk,
// the row-map reads and the residual reads are each issued as one batch at clamped (valid)
// addresses; elements past MN are not stored.
#define REDUCE_R 4
__global__ void k_gemm_reduce(const float * __restrict__ ws, int S, int64_t MN, int N, const float * bias,
                              const float * res, float * Y, int64_t ldy, const int32_t * __restrict__ ymap,
                              dfx_epi epi) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (epi.kind == DFX_EPI_SWIGLU) {
        // one output h[m][f] per element: gate and up column sums (slice order), then silu * up
        const int F = N / 2;
        const int64_t MF = MN / 2;
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MF; i += stride) {
            const int64_t m = i / F;
            const int f = (int)(i - m * F);
            const int64_t cg = m * N + (int64_t)(f >> 4) * 32 + (f & 15);
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < S; s++) {
                g = g + ws[(int64_t)s * MN + cg];
                u = u + ws[(int64_t)s * MN + cg + 16];
            }
            Y[m * ldy + f] = silu_mul(g, u);
        }
        return;
    }
    for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < MN; i0 += REDUCE_R * stride) {
        int64_t idx[REDUCE_R];
        float v[REDUCE_R];
#pragma unroll
        for (int j = 0; j < REDUCE_R; j++) {
            idx[j] = min(i0 + j * stride, MN - 1);
            v[j] = 0.0f;
        }
        for (int s = 0; s < S; s++) {
            float p[REDUCE_R];
#pragma unroll
            for (int j = 0; j < REDUCE_R; j++) p[j] = ws[(int64_t)s * MN + idx[j]];
#pragma unroll
            for (int j = 0; j < REDUCE_R; j++) v[j] = v[j] + p[j];
        }
        int64_t o[REDUCE_R];
        int n[REDUCE_R];
#pragma unroll
        for (int j = 0; j < REDUCE_R; j++) {
            const int64_t m = idx[j] / N;
            n[j] = (int)(idx[j] - m * N);
            o[j] = (int64_t)(ymap ? ymap[m] : m) * ldy + n[j];
        }
        float b[REDUCE_R], rv[REDUCE_R];
        if (bias)
#pragma unroll
            for (int j = 0; j < REDUCE_R; j++) b[j] = bias[n[j]];
        if (res)
#pragma unroll
            for (int j = 0; j < REDUCE_R; j++) rv[j] = res[o[j]];
#pragma unroll
        for (int j = 0; j < REDUCE_R; j++) {
            if (bias) v[j] = v[j] + b[j];
            if (res) v[j] = v[j] + rv[j];
            asm volatile("" : "+v"(v[j]));
        }
#pragma unroll
        for (int j = 0; j < REDUCE_R; j++)
            if (i0 + j * stride < MN) Y[o[j]] = v[j];
    }
}

#define MAX_SPLIT 8

// Forced tile of the Q4_K / Q6_K kernels, for tuning and tests:
// "<TM>x<TN>[x<D>]" picks a register tile, "s" splits K when possible, "n" never
// splits, "w" / "w1" / "w3" pick the LDS-DMA Q4_K kernel (64 x 64 / 64 x 32 / 96 x 32
// per wave), "v1" / "v2" run a Q4_K 32 x 32 register tile with one or two waves per
// workgroup instead of four, "k" the super-block-parallel Q4_K kernel ("ks" split K).
// Set with dfx_gemm_force_tile; DFX_Q4K_TILE / DFX_Q6K_TILE are read once, at the
// first GEMM launch or setter call.  Parsed once, not per launch.
struct tile_force {
    bool on = false;
    int got = 0, tm = 0, tn = 0, d = 0;
    bool split = false, nosplit = false, w = false, w1 = false, w3 = false, halves = false, sbp = false;
    int sbtn = 1;   // "k<n>": column tiles per workgroup of the super-block-parallel kernel (1, 2 or 4)
    int nwv = 4;   // "v<n>": waves per workgroup of a register-ring tile (1, 2 or 4)
};
static std::mutex g_force_mu;
static tile_force g_force[2];   // [0] Q4_K, [1] Q6_K
static std::once_flag g_force_env;

static tile_force parse_force(const char * f) {
    tile_force t;
    if (!f || !*f) return t;
    t.on = true;
    t.got = sscanf(f, "%dx%dx%d", &t.tm, &t.tn, &t.d);
    t.split = strchr(f, 's') != nullptr;
    t.nosplit = strchr(f, 'n') != nullptr;
    t.w = strchr(f, 'w') != nullptr;
    t.w1 = strstr(f, "w1") != nullptr;
    t.w3 = strstr(f, "w3") != nullptr;
    t.halves = strchr(f, 'f') != nullptr;
    if (const char * k = strchr(f, 'k')) {
        t.sbp = true;
        const int v = atoi(k + 1);
        t.sbtn = v == 2 || v == 4 ? v : 1;
    }
    if (const char * v = strchr(f, 'v')) t.nwv = atoi(v + 1);
    return t;
}

static void force_from_env() {
    std::call_once(g_force_env, [] {
        std::lock_guard<std::mutex> lk(g_force_mu);
        g_force[0] = parse_force(getenv("DFX_Q4K_TILE"));
        g_force[1] = parse_force(getenv("DFX_Q6K_TILE"));
    });
}

static tile_force forced_tile(int which) {
    force_from_env();
    std::lock_guard<std::mutex> lk(g_force_mu);
    return g_force[which];
}

extern "C" int dfx_gemm_force_tile(int wtype, const char * spec) {
    if (wtype != DFX_TYPE_Q4_K && wtype != DFX_TYPE_Q6_K) {
        dfx_set_error("dfx_gemm_force_tile: only Q4_K and Q6_K have tile choices (type %d)", wtype);
        return DFX_ERR_ARG;
    }
    force_from_env();
    std::lock_guard<std::mutex> lk(g_force_mu);
    g_force[wtype == DFX_TYPE_Q4_K ? 0 : 1] = parse_force(spec);
    return DFX_OK;
}

// Split-K partials: F16 up to MAX_SPLIT slices, quantised types one slice per K chunk.
extern "C" size_t dfx_gemm_ws_bytes(int64_t M, int64_t N, int64_t K) {
    const int64_t slices = std::max<int64_t>(MAX_SPLIT, dot_chunks(K));
    return (size_t)slices * M * N * sizeof(float);
}

// The RoPE epilogue after split K, by tiles of 4 rows x 64 columns (whole NEOX pairs: a column's
// partner n ^ 16 is in the same tile): each element's chunk sums (slice order) plus bias are read
// once, along the columns, into LDS, where the partner's sum is taken from; Q and K are rotated
// and stored along the columns, V along the rows of the transposed value cache.  Each element's
// arithmetic is the element-wise reduction's.  Against one element (and its partner's sums) per
// thread: Dream-7B generations 2.4 % faster in a same-box A/B (its Q|K|V at 12-64 rows splits K);
// 8-, 16- and 32-row tiles gained 1.6, 0.4 and -2 %.
#define RR_M 4
#define RR_N 64
__global__ void __launch_bounds__(256) k_gemm_reduce_rope(const float * __restrict__ ws, int S, int M, int N,
                                                          const float * bias, dfx_epi epi) {
#pragma clang fp contract(off)
    __shared__ float tile[RR_M][RR_N + 1];
    const int m0 = blockIdx.y * RR_M, n0 = blockIdx.x * RR_N, tid = threadIdx.x;
    const int64_t MN = (int64_t)M * N;
    // sums: thread (row r = tid / 64 + 4 i, column c = tid % 64), clamped reads, zero outside
#pragma unroll
    for (int i = 0; i < RR_M / 4; i++) {
        const int r = tid / RR_N + 4 * i, c = tid % RR_N;
        const int m = min(m0 + r, M - 1), n = min(n0 + c, N - 1);
        float v = 0.0f;
        for (int sl = 0; sl < S; sl++) v = v + ws[(int64_t)sl * MN + (int64_t)m * N + n];
        if (bias) v = v + bias[n];
        tile[r][c] = v;
    }
    __syncthreads();
    const int hd = epi.hd, half = hd >> 1, qk_cols = (epi.H + epi.Hkv) * hd;
    // Q and K: along the columns
#pragma unroll
    for (int i = 0; i < RR_M / 4; i++) {
        const int r = tid / RR_N + 4 * i, c = tid % RR_N, m = m0 + r, n = n0 + c;
        const int g = n + epi.col0;
        if (m >= M || n >= N || g >= qk_cols) continue;
        const int hh = g / hd, cc = g - hh * hd;
        const bool first = (cc & 16) == 0;
        const int d0 = 16 * (cc >> 5) + (cc & 15), d = first ? d0 : half + d0;
        const int p = epi.pos[m];
        const float2 cs = *(const float2 *)(epi.tab + ((int64_t)p * half + d0) * 2);
        const float v = tile[r][c], w = tile[r][c ^ 16];
        const float x0 = first ? v : w, x1 = first ? w : v;
        const float y = first ? x0 * cs.x - x1 * cs.y : x0 * cs.y + x1 * cs.x;
        float * dst = hh < epi.H ? epi.q_out + ((int64_t)m * epi.H + hh) * hd
                                 : epi.kc + ((int64_t)p * epi.Hkv + (hh - epi.H)) * hd;
        dst[d] = y;
    }
    // V: along the rows (transposed store)
#pragma unroll
    for (int i = 0; i < RR_N * RR_M / 256; i++) {
        const int r = tid % RR_M, c = tid / RR_M + (256 / RR_M) * i, m = m0 + r, n = n0 + c;
        const int g = n + epi.col0;
        if (m >= M || n >= N || g < qk_cols) continue;
        const int hh = g / hd, cc = g - hh * hd;
        epi.vt[((int64_t)(hh - epi.H - epi.Hkv) * hd + cc) * epi.v_ld + epi.pos[m]] = tile[r][c];
    }
}

// Split-K epilogue: sums the S partial slices in ws (slice order) plus bias and residual
// into Y, or, with defer, leaves the slices for the consumer of Y (the next RMSNorm,
// which then adds them and the residual itself) and reports S.
static int reduce_or_defer(const void * ws, int S, int M, int N, const float * bias, const float * res, float * y,
                           int64_t ldy, const int32_t * ymap, hipStream_t st, int * defer, dfx_epi epi) {
    if (defer) {
        *defer = S;
        return DFX_OK;
    }
    if (epi.kind == DFX_EPI_ROPE) {
        const dim3 grid((unsigned)((N + RR_N - 1) / RR_N), (unsigned)((M + RR_M - 1) / RR_M));
        hipLaunchKernelGGL(k_gemm_reduce_rope, grid, dim3(256), 0, st, (const float *)ws, S, M, N, bias, epi);
        DFX_CHECK_LAUNCH("dfx_gemm reduce (RoPE)");
        return DFX_OK;
    }
    const int64_t MN = (int64_t)M * N;
    const int64_t blocks = std::min<int64_t>((MN + 256 * REDUCE_R - 1) / (256 * REDUCE_R), 8192);
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)blocks), dim3(256), 0, st, (const float *)ws, S, MN, N, bias, res,
                       y, ldy, ymap, epi);
    DFX_CHECK_LAUNCH("dfx_gemm reduce");
    return DFX_OK;
}

// K slices of an F16 GEMM with TM row tiles per workgroup: K is split while the grid is
// smaller than the CU count, ws_bytes holds the partials and every slice keeps at least 4
// K steps.  (f32 sums: the slice count decides the summation order, hence the bits.)
static int f16_splits(int TM, int64_t M, int64_t N, int64_t K, size_t ws_bytes) {
    const int64_t tiles = ((N + 127) / 128) * ((M + 32 * TM - 1) / (32 * TM));
    const int n_kt = (int)(K / BK);
    int S = 1;
    while (S < MAX_SPLIT && tiles * S < 256 && n_kt / (S * 2) >= 4 &&
           (size_t)(S * 2) * M * N * sizeof(float) <= ws_bytes)
        S *= 2;
    const int per = (n_kt + S - 1) / S;
    return (n_kt + per - 1) / per;
}

template <int TM>
static int launch_f16(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, void * ws, size_t ws_bytes, hipStream_t st, int * defer,
                      dfx_epi epi) {
    constexpr int BM = TM * 32, BN = 128;
    const int gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM;
    const int n_kt = K / BK;
    const int S = f16_splits(TM, M, N, K, ws ? ws_bytes : 0);
    const int per = (n_kt + S - 1) / S;
    hipLaunchKernelGGL((k_gemm_f16<TM>), dim3(gx, gy, S), dim3(256), 0, st, (const uint8_t *)w, N, K,
                       (const half_t *)act, M, bias, res, y, ldy, ymap, (float *)ws, per, epi);
    DFX_CHECK_LAUNCH("dfx_gemm f16");
    if (S > 1) return reduce_or_defer(ws, S, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

template <int TM>
static int launch_f32(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, hipStream_t st, dfx_epi epi) {
    const dim3 grid((N + 127) / 128, (M + 32 * TM - 1) / (32 * TM));
    hipLaunchKernelGGL((k_gemm_f32<TM>), grid, dim3(256), 0, st, (const float *)w, N, K, (const float *)act, M, bias,
                       res, y, ldy, ymap, epi);
    DFX_CHECK_LAUNCH("dfx_gemm f32");
    return DFX_OK;
}

template <int WT, int TM>
static int launch_mmq(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, hipStream_t st, dfx_epi epi) {
    constexpr int BM = TM * 32, BN = 128;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL((k_mmq<WT, TM>), grid, dim3(256), 0, st, (const uint8_t *)w, N, K, (const uint8_t *)act, M,
                       bias, res, y, ldy, ymap, epi);
    DFX_CHECK_LAUNCH("dfx_gemm");
    return DFX_OK;
}

template <int TM, int TN, int D, int NWV = 4>
static int launch_q4k(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, float * ws, hipStream_t st, int * defer,
                      dfx_epi epi) {
    constexpr int BM = TM * 32, BN = NWV * TN * 32;
    const int n_tiles = (N + BN - 1) / BN, m_tiles = (M + BM - 1) / BM;
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int chunks = dot_chunks(K), passes = ws ? chunks : 1;
    static_assert(D == 2 || D == 4, "ring depth 2 or 4");
    // every workgroup's K steps (whole super-blocks, two per super-block) must be a
    // multiple of the ring depth
    const int sb = K / 256, sb_last = sb - (chunks - 1) * (DFX_DOT_CHUNK / 256);
    if ((2 * sb_last) % D || (chunks > 1 && (2 * (DFX_DOT_CHUNK / 256)) % D)) {
        dfx_set_error("dfx_gemm q4_k: K=%d does not fit the pipeline depth %d", K, D);
        return DFX_ERR_ARG;
    }
    hipLaunchKernelGGL((k_q4k<TM, TN, D, NWV>), dim3((unsigned)(per_pass * passes)), dim3(64 * NWV), 0, st,
                       (const uint8_t *)w, N, K, (const uint8_t *)act, M, bias, res, y, ldy, ymap, n_tiles, m_tiles, ws, epi);
    DFX_CHECK_LAUNCH("dfx_gemm q4_k");
    if (ws) return reduce_or_defer(ws, chunks, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

// Super-block-parallel Q4_K (k_q4k_sb): eight waves per 32 x (32 TN) tile; with ws, one
// workgroup per chunk and the chunk sums added by the reduction (or by the caller).
template <int TN>
static int launch_q4k_sb(const void * w, int N, int K, const void * act, int M, const float * bias,
                         const float * res, float * y, int64_t ldy, const int32_t * ymap, float * ws, hipStream_t st,
                         int * defer, dfx_epi epi) {
    const int n_tiles = (N + 32 * TN - 1) / (32 * TN), m_tiles = (M + 31) / 32;
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int chunks = dot_chunks(K);
    if (chunks == 1) ws = nullptr;
    const size_t lds = (size_t)8 * TN * 4 * 64 * 16 + 8 * 32 * 4;
    if (lds > 64 * 1024) {
        // above the default limit of dynamic LDS (TN >= 2: the forced tuning forms only)
        static std::once_flag once;
        static hipError_t attr = hipSuccess;
        std::call_once(once, [lds] {
            attr = hipFuncSetAttribute((const void *)k_q4k_sb<TN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
        });
        if (attr != hipSuccess) {
            dfx_set_error("dfx_gemm q4_k: %zu bytes of LDS refused: %s", lds, hipGetErrorString(attr));
            return DFX_ERR_HIP;
        }
    }
    hipLaunchKernelGGL(k_q4k_sb<TN>, dim3((unsigned)(per_pass * (ws ? chunks : 1))), dim3(512), lds, st,
                       (const uint8_t *)w, N, K, (const uint8_t *)act, M, bias, res, y, ldy, ymap, n_tiles, m_tiles,
                       ws, epi);
    DFX_CHECK_LAUNCH("dfx_gemm q4_k");
    if (ws) return reduce_or_defer(ws, chunks, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

template <int TM, int TN, int DEPTH>
// n_full >= 0 (with epi.tile_cnt, two chunks, ws of 2 M N floats): tiles n_full.. are split
// into halves combined inside the launch; otherwise epi.tile_cnt is ignored.
static int launch_q4k_w(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, float * ws, hipStream_t st, int * defer,
                      dfx_epi epi, int n_full = -1) {
    const int n_tiles = (N + 128 * TN - 1) / (128 * TN), m_tiles = (M + 32 * TM - 1) / (32 * TM);
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int chunks = dot_chunks(K), passes = ws ? chunks : 1;
    const int sb = K / 256, sb_last = sb - (chunks - 1) * (DFX_DOT_CHUNK / 256);
    if ((2 * sb_last) % DEPTH || (chunks > 1 && (2 * (DFX_DOT_CHUNK / 256)) % DEPTH)) {
        dfx_set_error("dfx_gemm q4_k: K=%d does not fit the pipeline depth %d", K, DEPTH);
        return DFX_ERR_ARG;
    }
    const bool halves = n_full >= 0 && epi.tile_cnt && ws && chunks == 2 && n_full % 8 == 0 && n_full <= per_pass;
    if (!halves) epi.tile_cnt = nullptr;
    const int grid = halves ? 2 * per_pass - n_full : per_pass * passes;
    hipLaunchKernelGGL((k_q4k_w<TM, TN, DEPTH>), dim3((unsigned)grid), dim3(256), 0, st, (const uint8_t *)w, N, K,
                       (const uint8_t *)act, M, bias, res, y, ldy, ymap, n_tiles, m_tiles, ws, epi, halves ? n_full : 0);
    DFX_CHECK_LAUNCH("dfx_gemm q4_k");
    if (ws && !halves) return reduce_or_defer(ws, chunks, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

// Compute units of the current device (cached per device).
static int device_cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (!v) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Whole tiles for the first n_full workgroups, half tiles after them.  Taken where a grid of
// whole tiles fills more than half but not all of the workgroup slots (two per CU): S/2 < T
// <= S tiles, where some CUs would carry two whole tiles and others one.  n_full from a sweep
// on MI355X at the LLaDA-8B shapes (Q|K|V and gate|up, every result the same bits):
//   T = 384: 2T - S = 256 whole tiles and 256 halves, one of each per CU (10-16 % faster
//            than whole tiles; 192 or 288 whole tiles are slower);
//   T = 288: 3T/4 = 216 whole tiles (15 % faster; 2T - S = 64 gives 8 %);
//   T = 480: 2T - S = 448 (3 %).
// Not taken for T <= S/2 (no CU holds two whole tiles; splitting gains nothing) nor above S
// (a last part-filled round: 0-6 % slower split).  `force` (tests) splits the second half of
// the tiles of any grid.
static int split_tile_count(int per_pass, bool force) {
    const int S = 2 * device_cu_count();
    const int T = per_pass;
    if (force) return T / 2 / 8 * 8;
    if (2 * T <= S || T > S) return -1;
    const int n_full = std::max(2 * T - S, 4 * T <= 5 * S / 2 ? 3 * T / 4 : 0);
    return std::min(T, (n_full + 7) / 8 * 8);
}

template <int TM, int TN, int D>
static int launch_q6k(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                      float * y, int64_t ldy, const int32_t * ymap, float * ws, hipStream_t st, int * defer,
                      dfx_epi epi) {
    constexpr int BM = TM * 32, BN = 4 * TN * 32;
    const int n_tiles = (N + BN - 1) / BN, m_tiles = (M + BM - 1) / BM;
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int chunks = dot_chunks(K), passes = ws ? chunks : 1;
    const int sb = K / 256, sb_last = sb - (chunks - 1) * (DFX_DOT_CHUNK / 256);
    if ((2 * sb_last) % D || (chunks > 1 && (2 * (DFX_DOT_CHUNK / 256)) % D)) {
        dfx_set_error("dfx_gemm q6_k: K=%d does not fit the pipeline depth %d", K, D);
        return DFX_ERR_ARG;
    }
    hipLaunchKernelGGL((k_q6k<TM, TN, D>), dim3((unsigned)(per_pass * passes)), dim3(256), 0, st,
                       (const uint8_t *)w, N, K, (const uint8_t *)act, M, bias, res, y, ldy, ymap, n_tiles, m_tiles, ws, epi);
    DFX_CHECK_LAUNCH("dfx_gemm q6_k");
    if (ws) return reduce_or_defer(ws, chunks, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

template <int TM>
static int launch_q6k_w(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, float * ws, hipStream_t st, int * defer,
                        dfx_epi epi) {
    const int n_tiles = (N + 127) / 128, m_tiles = (M + 32 * TM - 1) / (32 * TM);
    const int per_pass = 8 * ((n_tiles + 7) / 8) * m_tiles;
    const int chunks = dot_chunks(K), passes = ws ? chunks : 1;
    hipLaunchKernelGGL((k_q6k_w<TM>), dim3((unsigned)(per_pass * passes)), dim3(256), 0, st, (const uint8_t *)w, N, K,
                       (const uint8_t *)act, M, bias, res, y, ldy, ymap, n_tiles, m_tiles, ws, epi);
    DFX_CHECK_LAUNCH("dfx_gemm q6_k");
    if (ws) return reduce_or_defer(ws, chunks, M, N, bias, res, y, ldy, ymap, st, defer, epi);
    return DFX_OK;
}

// Q6_K: above 32 rows the LDS-DMA kernel, with 96-row tiles where they pad M to no more rows
// than 64-row tiles (ties included), else 64-row tiles; at most 32 rows the register-ring
// kernel (32 rows, 2-deep weight ring).  Split K when the grid is small.  Measured on MI355X at
// the LLaDA-8B vocab head (126464 x 4096) and Q6_K down projection (4096 x 12288) and the
// Dream-7B ones, every variant the same bits: 96-row tiles 10-33 % faster at 74, 162, 181 and
// 288 rows, 25-50 % slower at 97, 120 and 128 (192 rows of tiles against 128), even at 240 and
// 256 at the head, 20 % slower at 256 for the down projection; the DMA kernel 2-6 % faster than
// the register ring at 64-row tiles; at 34-48 rows its 64-row tiles 10-30 % faster than two
// 32-row tiles of the register ring (each weight dequantised once), at 12-24 rows 20 % slower.  A forced tile "<TM>x<TN>[x<D>][s|n]" (dfx_gemm_force_tile) picks a
// register-ring tile, "w" / "w1" the 64-row and "w3" the 96-row DMA kernel.
static int dispatch_q6k(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, void * ws, size_t ws_bytes, hipStream_t st, int * defer,
                        dfx_epi epi) {
    bool dma = M > 32;
    int tm = !dma ? 1 : (M + 95) / 96 * 96 <= (M + 63) / 64 * 64 ? 3 : 2, tn = 1;
    const int chunks = dot_chunks(K);
    const int64_t tiles = (int64_t)((M + 32 * tm - 1) / (32 * tm)) * ((N + 128 * tn - 1) / (128 * tn));
    bool split = chunks > 1 && tiles * 4 < 1024 && ws && ws_bytes >= (size_t)chunks * M * N * sizeof(float);
    int d = 2;
    if (const tile_force f = forced_tile(1); f.on) {
        if (f.got >= 2 && ((f.tm == 1 || f.tm == 2) && f.tn == 1)) { tm = f.tm; tn = f.tn; dma = false; }
        if (f.got == 3 && (f.d == 2 || f.d == 4)) d = f.d;
        if (f.w) { tm = f.w3 ? 3 : 2; dma = true; }
        if (f.split) split = chunks > 1 && ws && ws_bytes >= (size_t)chunks * M * N * sizeof(float);
        if (f.nosplit) split = false;
    }
    // a 4-deep ring needs a multiple of 4 K steps in every workgroup
    const int sb = K / 256, sb_last = sb - (chunks - 1) * (DFX_DOT_CHUNK / 256);
    if (sb_last % 2) d = 2;
    float * wsf = split ? (float *)ws : nullptr;
    if (dma && tm == 3) return launch_q6k_w<3>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    if (dma) return launch_q6k_w<2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    if (tm == 2)
        return d == 4 ? launch_q6k<2, 1, 4>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi)
                      : launch_q6k<2, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    return d == 4 ? launch_q6k<1, 1, 4>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi)
                  : launch_q6k<1, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
}

// Tile of the Q4_K kernel (TM x TN 32x32 tiles per wave, D = K steps in flight).
// When the grid leaves the SIMDs short of two waves each, K is split at chunk
// borders (workspace permitting).
static int dispatch_q4k(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, void * ws, size_t ws_bytes, hipStream_t st, int * defer,
                        dfx_epi epi) {
    struct cand { int tm, tn, d; };
    // (a 96-row tile, TM = 3, spills its sums at two workgroups per CU and is not built; nor is
    // 32 x 64 per wave, TM = 1, TN = 2, whose two-deep ring spills 68 registers)
    static const cand cands[] = {{2, 2, 2}, {4, 1, 2}, {2, 1, 2}, {1, 1, 4}, {1, 1, 2}, {2, 1, 4}, {2, 2, 4}};
    constexpr int n_cand = 7;
    enum { C_2x1x2 = 2, C_1x1x4 = 3, C_1x1x2 = 4 };
    // Kernel and split choice, from a warmed-up sweep of every variant on MI355X over
    // the LLaDA-8B shapes (N 4096 / 12288 / 24576, K 4096 / 12288) and the row counts
    // of a 16-step, 256-mask generation (M 50..288), kept where the whole generation
    // got faster too.  "Narrow" GEMMs (at most 32
    // column tiles of 128) give few workgroups; "wide" ones many.
    //   default: the 64x128 LDS-DMA kernel k_q4k_w<1, 2>, K split at chunk borders
    //     when K spans more than two chunks or the grid has under 160 workgroups;
    //   M in (128, 150): 64-row tiles leave most of the last tile empty, and the
    //     32x128 register-ring kernel (4-deep ring; 2-deep and split for narrow GEMMs
    //     over many chunks) is 6-19% faster;
    //   narrow, at most two chunks, M <= 128: 32x128 with a 2-deep ring and split K
    //     (8-17% faster than the default);
    //   narrow, many chunks, M in (64, 80]: 32x128, 2-deep ring, split K;
    //   M <= 48 (outside the sweep, weight-bandwidth-bound): 32x128, 4-deep ring, split
    //     K while the grid leaves the SIMDs short of a wave each.
    // The choice only changes speed: every variant gives the same bits.
    //   32 < M <= 48, not narrow or over more than two chunks: the 64-row DMA tile (every
    //     weight dequantised once for all rows), K split over many chunks or on grids under
    //     160 column tiles (Dream-7B gate|up and down at 34-48 rows: 15-18 % faster than 32-row
    //     tiles; LLaDA-8B Q|K|V at 48 rows 23.3 -> 19.5 us);
    //   64 < M <= 96, unless narrow over at most two chunks: one 96-row tile (k_q4k_w<3, 1, 2>),
    //     K split over many chunks or on grids under 160 workgroups (LLaDA-8B Q|K|V, gate|up
    //     and down at 74 and 96 rows: 2-15 % faster than 64-row tiles).
    // "Narrow" is at most 40 column tiles (Dream-7B's Q|K|V, 36 tiles, runs best as the 32-tile
    // O and down projections do).
    const int chunks = dot_chunks(K);
    const int n_col = (N + 127) / 128;
    const bool narrow = n_col <= 40;
    const bool can_split = chunks > 1 && ws && ws_bytes >= (size_t)chunks * M * N * sizeof(float);
    int pick = C_2x1x2;   // register-ring 64x128 (when the DMA kernel is not used)
    bool dma = true, split = false, rows96 = false;
    if (M <= 48) {
        if (M > 32 && (!narrow || chunks > 2)) {
            split = can_split && (chunks > 2 || n_col < 160);
        } else {
            dma = false;
            pick = C_1x1x4;
            split = can_split && (int64_t)n_col * ((M + 31) / 32) * 4 < 1024;
        }
    } else if (M > 128 && M < 150) {
        dma = false;
        pick = narrow && chunks > 2 ? C_1x1x2 : C_1x1x4;
        split = narrow && chunks > 2 && can_split;
    } else if (narrow && chunks <= 2 && M <= 128) {
        dma = false;
        pick = C_1x1x2;
        split = can_split;
    } else if (M > 64 && M <= 96) {
        rows96 = true;
        split = can_split && (chunks > 2 || n_col < 160);
    } else {
        split = can_split && (chunks > 2 || (int64_t)n_col * ((M + 63) / 64) < 160);
    }
    // Narrow GEMMs over at most 64 rows: 32 x 32 register tiles in workgroups of one or two
    // waves where four-wave workgroups would leave CUs idle or fill a second round only in
    // part (LLaDA-8B and Dream-7B O, Q|K|V and down at 12-64 rows: 3-13 % faster; slower where
    // the four-wave grid fills the chip once, as LLaDA-8B's down projection does):
    //   at most two chunks, when twice the four-wave split grid fits one workgroup per CU:
    //     two waves, 2-deep ring, split K;
    //   more chunks, with 256 to 512 workgroups of one 32- or 64-row tile per column tile and
    //     chunk: one wave up to 32 rows, two above, 2-deep ring, split K.
    int nwv = 4;
    if (narrow && M <= 64 && can_split) {
        const int64_t g4 = (int64_t)n_col * ((M + 31) / 32) * chunks, g1 = (int64_t)n_col * chunks;
        if (chunks <= 2 ? 2 * g4 <= 256 : g1 > 256 && g1 < 512) {
            nwv = chunks > 2 && M <= 32 ? 1 : 2;
            dma = false;
            pick = C_1x1x2;
            split = true;
        }
    }
    // Wide GEMMs over at most 32 rows (gate|up): two waves per workgroup, 2-deep ring, K split
    // where the workspace allows (Dream-7B's gate|up at 12-32 rows 29.2-29.4 -> 25.8-29.1 us,
    // LLaDA-8B's 23.5-24.1 -> 21.9-22.2 us).
    if (!narrow && M <= 32 && !dma) {
        nwv = 2;
        pick = C_1x1x2;
        split = can_split;
    }
    // A forced tile "<TM>x<TN>[x<D>][s|n][v1|v2]" (dfx_gemm_force_tile) overrides the choice:
    // s = split K when possible, n = never split, v = waves per workgroup.
    const tile_force f = forced_tile(0);
    if (f.on) {
        nwv = f.nwv;
        if (f.got >= 2) {
            dma = false;
            for (int c = n_cand - 1; c >= 0; c--)
                if (cands[c].tm == f.tm && cands[c].tn == f.tn && (f.got < 3 || cands[c].d == f.d)) pick = c;
        }
        if (f.split) split = chunks > 1 && ws && ws_bytes >= (size_t)chunks * M * N * sizeof(float);
        if (f.nosplit) split = false;
    }
    // At most 96 rows over at most two chunks, on grids of at most 432 32 x 32 tiles: the
    // super-block-parallel kernel k_q4k_sb, K split at the chunk border when the caller adds
    // the chunk sums later (defer), else both chunks in one workgroup.  Measured on the
    // LLaDA-8B and Dream-7B O and Q|K|V shapes at 12-96 rows: 14.1-16.7 -> 8.4-14.7 us a call
    // (Dream-7B's Q|K|V and O, LLaDA-8B's O, LLaDA-8B's Q|K|V up to 32 rows), and the Dream-7B
    // 64 + 64 generation 4.2 % faster; slower over many chunks or many column tiles, where
    // every tile re-reads the activations.
    if (!f.on && chunks <= 2 && M <= 96 && (int64_t)((N + 31) / 32) * ((M + 31) / 32) <= 432)
        return launch_q4k_sb<1>(w, N, K, act, M, bias, res, y, ldy, ymap, defer && can_split ? (float *)ws : nullptr,
                                st, defer, epi);
    // a 4-deep ring needs a multiple of 4 K steps in every workgroup
    const int sb = K / 256, sb_last = sb - (chunks - 1) * (DFX_DOT_CHUNK / 256);
    // whole and half tiles in one launch (k_q4k_w): two chunks, tile counters, and room in ws
    // for both halves' chunk totals
    const bool halves_ok = epi.tile_cnt && chunks == 2 && N % 128 == 0 && ws &&
                           ws_bytes >= (size_t)2 * M * N * sizeof(float);
    if (f.on && f.sbp) {
        float * wsk = f.split && can_split ? (float *)ws : nullptr;
        if (f.sbtn == 4) return launch_q4k_sb<4>(w, N, K, act, M, bias, res, y, ldy, ymap, wsk, st, defer, epi);
        if (f.sbtn == 2) return launch_q4k_sb<2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsk, st, defer, epi);
        return launch_q4k_sb<1>(w, N, K, act, M, bias, res, y, ldy, ymap, wsk, st, defer, epi);
    }
    if (f.on && f.w) {
        // "w": 64 x 64 per wave; "w1": 64 x 32 per wave, two workgroups per CU
        float * wsw = split ? (float *)ws : nullptr;
        if (f.w1) {
            if (f.halves && halves_ok)
                return launch_q4k_w<2, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, (float *)ws, st, defer, epi,
                                             split_tile_count(8 * ((n_col + 7) / 8) * ((M + 63) / 64), true));
            return launch_q4k_w<2, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsw, st, defer, epi);
        }
        if (f.w3) {
            if (f.halves && halves_ok)
                return launch_q4k_w<3, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, (float *)ws, st, defer, epi,
                                             split_tile_count(8 * ((n_col + 7) / 8) * ((M + 95) / 96), true));
            return launch_q4k_w<3, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsw, st, defer, epi);
        }
        if (sb_last % 2) return launch_q4k_w<2, 2, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsw, st, defer, epi);
        return launch_q4k_w<2, 2, 4>(w, N, K, act, M, bias, res, y, ldy, ymap, wsw, st, defer, epi);
    }
    // whole and half tiles in one launch where that evens out the workgroups per CU
    if (dma && halves_ok && (!f.on || f.got < 2)) {
        const int nf = split_tile_count(8 * ((n_col + 7) / 8) * ((M + 63) / 64), f.on && f.halves);
        if (nf >= 0)
            return launch_q4k_w<2, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, (float *)ws, st, defer, epi, nf);
    }
    // 96-row tiles (k_q4k_w<3, 1, 2>): each dequantised weight feeds three MFMAs instead of
    // two, but a workgroup takes 1.5x longer, so they only pay when the chosen kernel's grid
    // needs more rounds of two workgroups per CU than theirs (measured: gate|up and down at
    // M = 142-181 of the LLaDA-8B shapes, 3-12% faster; slower wherever the default fits
    // in one round)
    if (!f.on && M > 128 && M <= 192) {
        auto rounds = [](int64_t wgs) { return (wgs + 511) / 512; };
        const int64_t t3 = (int64_t)n_col * ((M + 95) / 96);
        const bool split3 = can_split && (chunks > 2 || t3 < 160);
        const int64_t t_def = (int64_t)n_col * (dma ? (M + 63) / 64 : (M + 31) / 32);
        if (rounds(t3 * (split3 ? chunks : 1)) < rounds(t_def * (split ? chunks : 1))) {
            const int n3 = halves_ok ? split_tile_count(8 * ((n_col + 7) / 8) * ((M + 95) / 96), false) : -1;
            if (n3 >= 0)
                return launch_q4k_w<3, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, (float *)ws, st, defer, epi, n3);
            return launch_q4k_w<3, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, split3 ? (float *)ws : nullptr, st,
                                         defer, epi);
        }
    }
    if (rows96 && !f.on)
        return launch_q4k_w<3, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, split ? (float *)ws : nullptr, st,
                                     defer, epi);
    if (dma) return launch_q4k_w<2, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, split ? (float *)ws : nullptr, st, defer, epi);
    if (cands[pick].d == 4 && (sb_last % 2))
        for (int c = 0; c < n_cand; c++)
            if (cands[c].tm == cands[pick].tm && cands[c].tn == cands[pick].tn && cands[c].d == 2) { pick = c; break; }
    float * wsf = split ? (float *)ws : nullptr;
    if ((nwv == 1 || nwv == 2) && cands[pick].tm == 1 && cands[pick].tn == 1) {
        if (nwv == 1)
            return cands[pick].d == 4 ? launch_q4k<1, 1, 4, 1>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi)
                                      : launch_q4k<1, 1, 2, 1>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
        return cands[pick].d == 4 ? launch_q4k<1, 1, 4, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi)
                                  : launch_q4k<1, 1, 2, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    }
#define Q4K_CASE(c, TM_, TN_, D_) \
    case c: return launch_q4k<TM_, TN_, D_>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    switch (pick) {
        Q4K_CASE(0, 2, 2, 2) Q4K_CASE(1, 4, 1, 2) Q4K_CASE(2, 2, 1, 2) Q4K_CASE(3, 1, 1, 4)
        Q4K_CASE(5, 2, 1, 4) Q4K_CASE(6, 2, 2, 4)
        default: return launch_q4k<1, 1, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, wsf, st, defer, epi);
    }
#undef Q4K_CASE
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

// Q8_0: one 32-row tile per workgroup.  The per-32-element block flush keeps three
// f32 totals per output in registers, and wider row tiles spill them (measured on
// MI355X: 2-5x slower with 64 or 96 rows per workgroup at M = 96..768).
template <int WT>
static int dispatch_mmq(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                        float * y, int64_t ldy, const int32_t * ymap, hipStream_t st, dfx_epi epi) {
    // 64-row tiles (each converted weight feeds two MFMAs) where their grid still gives every
    // CU two workgroups; else 32-row tiles (same-box A/B over the LLaDA-8B projections: gate|up
    // at 256 / 768 rows and Q|K|V at 768 rows 7-21 % faster with 64 rows, the narrower grids
    // 0-35 % slower)
    if ((int64_t)((N + 127) / 128) * ((M + 63) / 64) >= 2 * device_cu_count())
        return launch_mmq<WT, 2>(w, N, K, act, M, bias, res, y, ldy, ymap, st, epi);
    return launch_mmq<WT, 1>(w, N, K, act, M, bias, res, y, ldy, ymap, st, epi);
}

// ---------------------------------------------------------------------------
// Q4_K / Q6_K matrix-vector kernels: at most DFX_GEMV_M activation rows (decoding)
// ---------------------------------------------------------------------------
// One wave per pair of output columns (n, n + 16) and pass set, n = 32 (p / 16) + p % 16 for
// pair p: the pairs the SwiGLU and RoPE epilogues combine.  A pass is 16 super-blocks (two
// chunks of 2048); lane l takes the 64-element group l % 4 of super-block l / 4 of each
// pass, for both columns and all rows.  Rows of one pass: four pairs per workgroup, a wave
// each.  Longer rows (SPLIT, e.g. the FFN down projection): a workgroup per pair with one
// wave per pass (up to 16, each taking every ws-th pass beyond that), so every pass's weight
// loads are in flight at once.  Integer dot products come from v_dot4_i32_i8 on the
// natural-order int8 activation plane (nibbles and 6-bit quants are non-negative bytes),
// exactly, in int32; the four lanes of a super-block add them (DPP quad permutes), and every
// lane then runs the exact float order over the super-blocks of each chunk (x and d_a read
// from the lanes that hold them): x = d_w*isum (Q4_K: x = fma(-dmin_w, msum, x));
// S = fma(d_a, x, S).  The chunk sums are added in chunk order, T = T + S, in the wave or,
// after a barrier, from LDS by the pair's first wave.  No MFMA: at these row counts the
// weights' HBM stream sets the time.
constexpr int GEMV_MAX_CHUNKS = 64;     // K <= 131072 for the pass-split form

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// v + (v of lane ^ 1), then + (lane ^ 2): the four lanes of a quad end with their sum
// (DPP quad permutes, no LDS traffic)
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1, 0, 3, 2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2, 3, 0, 1]
    return v;
}

// the value of a lane known at compile time, as a wave-uniform value
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// One output of the matrix-vector kernels through the epilogue: v = row m at column n,
// w = row m at the paired column n ^ 16 (the SwiGLU up value, or the other dim of the RoPE
// pair).  Float expressions as in epilogue_tile / rope_tile / k_gemm_reduce.
__device__ __forceinline__ void gemv_store(float v, float w, int m, int n, int N, const float * bias, const float * res,
                                           float * Y, int64_t ldy, const int32_t * ymap, const dfx_epi & epi) {
#pragma clang fp contract(off)
    if (epi.kind == DFX_EPI_SWIGLU) {
        if ((n & 16) == 0) Y[(int64_t)m * ldy + (n >> 5) * 16 + (n & 15)] = silu_mul(v, w);
        return;
    }
    if (bias) {
        v = v + bias[n];
        w = w + bias[n ^ 16];
    }
    if (epi.kind == DFX_EPI_ROPE) {
        const int p = epi.pos[m];
        const int hd = epi.hd, half = hd >> 1;
        const int g = n + epi.col0, hh = g / hd, cc = g - hh * hd;
        if (hh < epi.H + epi.Hkv) {
            const bool first = (cc & 16) == 0;
            const int d0 = 16 * (cc >> 5) + (cc & 15), d = first ? d0 : half + d0;
            const float2 cs = *(const float2 *)(epi.tab + ((int64_t)p * half + d0) * 2);
            const float x0 = first ? v : w, x1 = first ? w : v;
            const float y = first ? x0 * cs.x - x1 * cs.y : x0 * cs.y + x1 * cs.x;
            float * dst = hh < epi.H ? epi.q_out + ((int64_t)m * epi.H + hh) * hd
                                     : epi.kc + ((int64_t)p * epi.Hkv + (hh - epi.H)) * hd;
            dst[d] = y;
        } else {
            epi.vt[((int64_t)(hh - epi.H - epi.Hkv) * hd + cc) * epi.v_ld + p] = v;
        }
        return;
    }
    const int64_t o = (int64_t)(ymap ? ymap[m] : m) * ldy + n;
    if (res) v = v + res[o];
    Y[o] = v;
}

template <int WT, int MR, bool SPLIT>
__global__ void __launch_bounds__(1024) k_gemv(const uint8_t * __restrict__ W, int N, int K,
                                              const uint8_t * __restrict__ act, int M, const float * __restrict__ bias,
                                              const float * res, float * Y, int64_t ldy,
                                              const int32_t * __restrict__ ymap, dfx_epi epi) {
#pragma clang fp contract(off)
    constexpr bool Q4 = WT == DFX_TYPE_Q4_K;
    constexpr int SB = Q4 ? SB_Q4_K : SB_Q6_K;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ws = SPLIT ? (int)(blockDim.x >> 6) : 1;   // waves per pair
    const int p = SPLIT ? (int)blockIdx.x : (int)blockIdx.x * 4 + wv, part = SPLIT ? wv : 0;
    const bool pair_live = p < N / 2;                    // the whole wave
    if (!SPLIT && !pair_live) return;
    const int ncol[2] = {32 * (p >> 4) + (p & 15), 32 * (p >> 4) + (p & 15) + 16};
    const int nsb = K >> 8, g = lane & 3, sbl = lane >> 2;
    const act_layout Lay = act_layout_of(Q4 ? CONV_Q8_K_P4 : CONV_Q8_K_P6, M, K);
    const int8_t * a8 = (const int8_t *)(act + Lay.i8);
    const float * ad = (const float *)(act + Lay.d);     // [nsb][mq]
    const uint16_t * abs = (const uint16_t *)(act + Lay.bs);   // [M][K/16], exact small integers
    const int64_t rb = (int64_t)nsb * SB;
    [[maybe_unused]] __shared__ float sS[SPLIT ? GEMV_MAX_CHUNKS * 2 * MR : 1];
    float T[2][MR];
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int m = 0; m < MR; m++) T[c][m] = 0.0f;

    for (int sb0 = 16 * part; pair_live && sb0 < nsb; sb0 += 16 * ws) {
        const int sbc = min(sb0 + sbl, nsb - 1);          // clamped: lanes past the end add nothing
        const bool live = sb0 + sbl < nsb;
        float x[2][MR];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint8_t * blk = W + (int64_t)ncol[c] * rb + (int64_t)sbc * SB;
            int isum[MR], msum[MR];
            float dw, dmw = 0.0f;
            if constexpr (Q4) {
                // header {d, dmin, scales[12]}, then 32 nibble bytes of group g (sub-blocks 2g, 2g+1)
                const u32x4 h = *(const u32x4 *)blk;
                const u32x4 q0 = *(const u32x4 *)(blk + 16 + 32 * g), q1 = *(const u32x4 *)(blk + 32 + 32 * g);
                const q4k_sm sm = q4k_unpack(h);
                const uint32_t scw = g < 2 ? sm.sc_lo : sm.sc_hi, mnw = g < 2 ? sm.mn_lo : sm.mn_hi;
                const int sh = 16 * (g & 1);
                const int sc0 = (scw >> sh) & 0xFF, sc1 = (scw >> (sh + 8)) & 0xFF;
                const int mn0 = (mnw >> sh) & 0xFF, mn1 = (mnw >> (sh + 8)) & 0xFF;
                dw = h2f((uint16_t)(h.x & 0xFFFFu));
                dmw = h2f((uint16_t)(h.x >> 16));
                const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const int mm = min(m, M - 1);
                    const int8_t * ar = a8 + (int64_t)mm * K + (int64_t)sbc * 256 + 64 * g;
                    const u32x4 a0 = *(const u32x4 *)ar, a1 = *(const u32x4 *)(ar + 16);
                    const u32x4 a2 = *(const u32x4 *)(ar + 32), a3 = *(const u32x4 *)(ar + 48);
                    const uint32_t aw[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                             a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
                    int slo = 0, shi = 0;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        slo = sdot4(qw[i] & 0x0F0F0F0Fu, aw[i], slo);
                        shi = sdot4((qw[i] >> 4) & 0x0F0F0F0Fu, aw[8 + i], shi);
                    }
                    isum[m] = sc0 * slo + sc1 * shi;
                    const uint2 bsw = *(const uint2 *)(abs + (int64_t)mm * (K / 16) + sbc * 16 + 4 * g);
                    const int b0 = (int)h2f((uint16_t)(bsw.x & 0xFFFFu)), b1 = (int)h2f((uint16_t)(bsw.x >> 16));
                    const int b2 = (int)h2f((uint16_t)(bsw.y & 0xFFFFu)), b3 = (int)h2f((uint16_t)(bsw.y >> 16));
                    msum[m] = mn0 * (b0 + b1) + mn1 * (b2 + b3);
                }
            } else {
                // group g: half hf = g / 2, quants l = 16 (g % 2) .. +15 of each of the four
                // 32-element strips k (elements 128 hf + 32 k + l, sub-block 8 hf + 2 k + g % 2)
                const int hf = g >> 1, lh = 16 * (g & 1);
                const u32x4 la = *(const u32x4 *)(blk + 64 * hf + lh), lb = *(const u32x4 *)(blk + 64 * hf + 32 + lh);
                const u32x4 qh = *(const u32x4 *)(blk + 128 + 32 * hf + lh);
                const u32x4 scv = *(const u32x4 *)(blk + 192);
                dw = h2f(*(const uint16_t *)(blk + 208));
                const uint32_t law[4] = {la.x, la.y, la.z, la.w}, lbw[4] = {lb.x, lb.y, lb.z, lb.w};
                const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
                uint32_t u[4][4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    u[0][t] = (law[t] & 0x0F0F0F0Fu) | ((qhw[t] << 4) & 0x30303030u);
                    u[1][t] = (lbw[t] & 0x0F0F0F0Fu) | ((qhw[t] << 2) & 0x30303030u);
                    u[2][t] = ((law[t] >> 4) & 0x0F0F0F0Fu) | (qhw[t] & 0x30303030u);
                    u[3][t] = ((lbw[t] >> 4) & 0x0F0F0F0Fu) | ((qhw[t] >> 2) & 0x30303030u);
                }
                int sck[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int j = 8 * hf + 2 * k + (g & 1);
                    sck[k] = (int)(int8_t)((scv[j >> 2] >> (8 * (j & 3))) & 0xFFu);
                }
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const int mm = min(m, M - 1);
                    const int8_t * ar = a8 + (int64_t)mm * K + (int64_t)sbc * 256 + 128 * hf + lh;
                    const uint16_t * br = abs + (int64_t)mm * (K / 16) + sbc * 16 + 8 * hf + (g & 1);
                    int acc = 0;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const u32x4 a = *(const u32x4 *)(ar + 32 * k);
                        int us = 0;
                        us = sdot4(u[k][0], a.x, us);
                        us = sdot4(u[k][1], a.y, us);
                        us = sdot4(u[k][2], a.z, us);
                        us = sdot4(u[k][3], a.w, us);
                        const int bsum = (int)h2f(br[2 * k]);
                        acc += sck[k] * (us - 32 * bsum);
                    }
                    isum[m] = acc;
                    msum[m] = 0;
                }
            }
            // the super-block's four lanes (consecutive) hold its four groups
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const int is = quad_sum(isum[m]);
                if constexpr (Q4) {
                    const int ms = quad_sum(msum[m]);
                    x[c][m] = fmaf(-dmw, (float)ms, dw * (float)is);
                } else {
                    x[c][m] = dw * (float)is;
                }
                if (!live) x[c][m] = 0.0f;
            }
        }
        // each lane's super-block scale of the activation rows, loaded together for the pass
        float dam[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) dam[m] = ad[(int64_t)sbc * Lay.mq + min(m, M - 1)];
        // the pass's two chunks of 8 super-blocks: S = fma(d_a, x, S) in order, T = T + S
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int first = sb0 + 8 * h;
            if (first >= nsb) break;
            float S[2][MR];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int m = 0; m < MR; m++) S[c][m] = 0.0f;
            for (int i = 0; i < 8 && first + i < nsb; i++) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const float da = lane_value(dam[m], 32 * h + 4 * i);
#pragma unroll
                    for (int c = 0; c < 2; c++) S[c][m] = fmaf(da, lane_value(x[c][m], 32 * h + 4 * i), S[c][m]);
                }
            }
            if constexpr (!SPLIT) {
#pragma unroll
                for (int c = 0; c < 2; c++)
#pragma unroll
                    for (int m = 0; m < MR; m++) T[c][m] = T[c][m] + S[c][m];
            } else if (lane == 0) {
                float * d = sS + (first >> 3) * 2 * MR;
#pragma unroll
                for (int c = 0; c < 2; c++)
#pragma unroll
                    for (int m = 0; m < MR; m++) d[c * MR + m] = S[c][m];
            }
        }
    }
    if constexpr (SPLIT) {
        __syncthreads();
        if (part != 0 || !pair_live) return;
        const float * d = sS;
        for (int ch = 0; ch < (nsb + 7) >> 3; ch++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int m = 0; m < MR; m++) T[c][m] = T[c][m] + d[ch * 2 * MR + c * MR + m];
    }
    // lane 2m + c stores row m of column c
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int c = 0; c < 2; c++)
            if (lane == 2 * m + c && m < M) gemv_store(T[c][m], T[c ^ 1][m], m, ncol[c], N, bias, res, Y, ldy, ymap, epi);
}

template <int WT>
static int launch_gemv(const void * w, int N, int K, const void * act, int M, const float * bias, const float * res,
                       float * y, int64_t ldy, const int32_t * ymap, hipStream_t st, dfx_epi epi) {
    // waves per pair: one per pass of 16 super-blocks, up to 16 (a workgroup per pair); one
    // pass: four pairs per workgroup, one wave each
    const int passes = (K / 256 + 15) / 16;
    const bool split = passes > 1 && (K / 256 + 7) / 8 <= GEMV_MAX_CHUNKS;
    const int ws = split ? std::min(passes, 16) : 1;
    const dim3 grid((unsigned)(split ? N / 2 : (N / 2 + 3) / 4)), block((unsigned)(split ? 64 * ws : 256));
    const uint8_t * W = (const uint8_t *)w;
    const uint8_t * A = (const uint8_t *)act;
#define GEMV_CASE(mr, sp) hipLaunchKernelGGL((k_gemv<WT, mr, sp>), grid, block, 0, st, W, N, K, A, M, bias, res, y, ldy, ymap, epi)
#define GEMV_WS(mr) if (split) GEMV_CASE(mr, true); else GEMV_CASE(mr, false)
    switch (M) {
        case 1: GEMV_WS(1); break;
        case 2: GEMV_WS(2); break;
        default: GEMV_WS(4); break;
    }
#undef GEMV_WS
#undef GEMV_CASE
    DFX_CHECK_LAUNCH("dfx_gemm (matrix-vector)");
    return DFX_OK;
}

// Internal form: output row m goes to row ymap[m] (or m) of Y with leading dimension
// ldy; the residual is read at the same place it is written.  Split K uses ws when it
// is large enough.
int dfx_gemm_ex(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                const float * bias, const float * residual, float * y, int64_t ldy, const int32_t * ymap,
                void * ws, size_t ws_bytes, void * stream, int * n_partials, const dfx_epi * epi_p) {
    // n_partials: if K gets split, leave the partial slices ws[s][m][n] for the caller
    // to add (calls without bias or row map, ldy = N) and report their number; 0 = Y
    // was written
    if (n_partials) *n_partials = 0;
    dfx_epi epi{};
    if (epi_p) epi = *epi_p;
    if (epi.kind == DFX_EPI_SWIGLU && (bias || residual || ymap || N % 32)) {
        dfx_set_error("dfx_gemm: the SwiGLU epilogue takes N a multiple of 32, no bias, residual or row map");
        return DFX_ERR_ARG;
    }
    if (epi.kind == DFX_EPI_ROPE) {
        const int64_t width = ((int64_t)epi.H + 2 * (int64_t)epi.Hkv) * epi.hd;
        if (residual || ymap || N % 32 || epi.H <= 0 || epi.Hkv <= 0 || epi.H % epi.Hkv || epi.hd <= 0 ||
            epi.hd % 32 || epi.col0 < 0 || epi.col0 % 32 || epi.col0 + N > width || !epi.pos || !epi.tab ||
            !epi.q_out || !epi.kc || !epi.vt || epi.v_ld <= 0) {
            dfx_set_error("dfx_gemm: bad RoPE epilogue (N=%lld col0=%d H=%d Hkv=%d hd=%d; no residual or row map)",
                          (long long)N, epi.col0, epi.H, epi.Hkv, epi.hd);
            return DFX_ERR_ARG;
        }
        ldy = N;   // Y is not written
    } else if (epi.kind != DFX_EPI_PLAIN && epi.kind != DFX_EPI_SWIGLU) {
        dfx_set_error("dfx_gemm: unknown epilogue %d", epi.kind);
        return DFX_ERR_ARG;
    }
    int * defer = n_partials && !bias && !ymap && ldy == N && epi.kind == DFX_EPI_PLAIN ? n_partials : nullptr;
    if (N <= 0 || K <= 0 || M < 0 || (K % 256) || N > INT32_MAX || M > INT32_MAX || K > INT32_MAX ||
        ldy < (epi.kind == DFX_EPI_SWIGLU ? N / 2 : N)) {
        dfx_set_error("dfx_gemm: bad shape M=%lld N=%lld K=%lld ldy=%lld (K must be a multiple of 256)",
                      (long long)M, (long long)N, (long long)K, (long long)ldy);
        return DFX_ERR_ARG;
    }
    if (M == 0) return DFX_OK;
    hipStream_t st = (hipStream_t)stream;
    const int n = (int)N, k = (int)K, m = (int)M;
    // the matrix-vector kernels (unless a tile is forced) where they beat the matrix-core
    // kernels: one row; two Q4_K rows; up to DFX_GEMV_M rows of a matrix of at most
    // 4096 x 4096 (measured at the LLaDA-8B shapes: the integer dot products grow with the
    // rows, the matrix-core kernels' time does not below 32 rows)
    const bool gemv_rows = m == 1 || (m == 2 && wtype == DFX_TYPE_Q4_K) || (m <= DFX_GEMV_M && N * K <= 4096 * 4096);
    if (gemv_rows && N % 32 == 0 && (wtype == DFX_TYPE_Q4_K || wtype == DFX_TYPE_Q6_K) &&
        !forced_tile(wtype == DFX_TYPE_Q4_K ? 0 : 1).on) {
        return wtype == DFX_TYPE_Q4_K ? launch_gemv<DFX_TYPE_Q4_K>(w, n, k, act, m, bias, residual, y, ldy, ymap, st, epi)
                                      : launch_gemv<DFX_TYPE_Q6_K>(w, n, k, act, m, bias, residual, y, ldy, ymap, st, epi);
    }
    switch (wtype) {
        case DFX_TYPE_Q4_K: return dispatch_q4k(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
        case DFX_TYPE_Q6_K: return dispatch_q6k(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
        case DFX_TYPE_Q8_0: return dispatch_mmq<DFX_TYPE_Q8_0>(w, n, k, act, m, bias, residual, y, ldy, ymap, st, epi);
        case DFX_TYPE_F16:
            switch (pick_tm(m, 4)) {
                case 1: return launch_f16<1>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
                case 2: return launch_f16<2>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
                case 3: return launch_f16<3>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
                default: return launch_f16<4>(w, n, k, act, m, bias, residual, y, ldy, ymap, ws, ws_bytes, st, defer, epi);
            }
        case DFX_TYPE_F32:
            if (m <= 32) return launch_f32<1>(w, n, k, act, m, bias, residual, y, ldy, ymap, st, epi);
            return launch_f32<2>(w, n, k, act, m, bias, residual, y, ldy, ymap, st, epi);
    }
    dfx_set_error("dfx_gemm: unsupported weight type %d", wtype);
    return DFX_ERR_UNSUPPORTED;
}

extern "C" int dfx_gemm(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                        const float * bias, const float * residual, float * y, void * ws, void * stream) {
    return dfx_gemm_ex(wtype, w, N, K, act, M, bias, residual, y, N, nullptr, ws,
                       ws ? dfx_gemm_ws_bytes(M, N, K) : 0, stream, nullptr, nullptr);
}

extern "C" size_t dfx_gemm_tile_cnt_bytes(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0) return 0;
    return (size_t)(8 * ((((N + 127) / 128) + 7) / 8) * ((M + 63) / 64)) * 32 * sizeof(int32_t);
}

extern "C" int dfx_gemm_counted(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                                const float * bias, const float * residual, float * y, void * ws, int32_t * tile_cnt,
                                void * stream) {
    dfx_epi e{};
    e.tile_cnt = tile_cnt;
    return dfx_gemm_ex(wtype, w, N, K, act, M, bias, residual, y, N, nullptr, ws,
                       ws ? dfx_gemm_ws_bytes(M, N, K) : 0, stream, nullptr, &e);
}

extern "C" int dfx_gemm_swiglu(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                               float * y, int64_t ldy, void * ws, void * stream) {
    dfx_epi e{};
    e.kind = DFX_EPI_SWIGLU;
    return dfx_gemm_ex(wtype, w, N, K, act, M, nullptr, nullptr, y, ldy, nullptr, ws,
                       ws ? dfx_gemm_ws_bytes(M, N, K) : 0, stream, nullptr, &e);
}

extern "C" int dfx_gemm_rope(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                             const float * bias, int col0, const int32_t * pos, int H, int Hkv, int hd,
                             const float * tab, float * q_out, float * kc, float * vt, int64_t v_ld, void * ws,
                             void * stream) {
    dfx_epi e{};
    e.kind = DFX_EPI_ROPE;
    e.col0 = col0;
    e.H = H;
    e.Hkv = Hkv;
    e.hd = hd;
    e.pos = pos;
    e.tab = tab;
    e.q_out = q_out;
    e.kc = kc;
    e.vt = vt;
    e.v_ld = v_ld;
    return dfx_gemm_ex(wtype, w, N, K, act, M, bias, nullptr, nullptr, N, nullptr, ws,
                       ws ? dfx_gemm_ws_bytes(M, N, K) : 0, stream, nullptr, &e);
}

// ---------------------------------------------------------------------------
// GEMM with a library-held split-K workspace (no allocation on any call)
// ---------------------------------------------------------------------------
// dfx_gemm takes its split-K workspace from the caller.  Callers that cannot allocate
// device memory at all (code under stream capture, serving loops that forbid hipMalloc)
// use dfx_gemm_noalloc instead: the workspace is `scratch`, a file-scope device array of
// DFX_GEMM_SCRATCH_BYTES that every device holds from module load to process end.  Host
// code never passes the array's name to a kernel (in host code it is only a stand-in
// symbol): the device address comes from hipGetSymbolAddress, looked up once per device on
// that device's first call and kept in scratch_ptr[device].
#define DFX_GEMM_SCRATCH_BYTES (32u << 20)
static __device__ __align__(256) uint8_t scratch[DFX_GEMM_SCRATCH_BYTES];

#define DFX_MAX_DEVICES 64
static void * scratch_ptr[DFX_MAX_DEVICES];
static std::once_flag scratch_once[DFX_MAX_DEVICES];
static hipError_t scratch_err[DFX_MAX_DEVICES];

extern "C" int dfx_gemm_noalloc(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                                const float * bias, const float * residual, float * y, void * stream) {
    int dev = -1;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess || dev < 0 || dev >= DFX_MAX_DEVICES) {
        dfx_set_error("dfx_gemm_noalloc: no current device (%s)", hipGetErrorString(ge));
        return DFX_ERR_HIP;
    }
    std::call_once(scratch_once[dev], [dev] {
        // The first call on a device may come while the caller captures a stream: the
        // lookup is not a stream operation, so this thread's capture mode is relaxed around
        // it (and restored) rather than letting a global-mode capture reject it.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
        void * p = nullptr;
        scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        scratch_ptr[dev] = scratch_err[dev] == hipSuccess ? p : nullptr;
        if (exchanged) (void)hipThreadExchangeStreamCaptureMode(&mode);
    });
    if (!scratch_ptr[dev]) {
        dfx_set_error("dfx_gemm_noalloc: device %d scratch address: %s", dev, hipGetErrorString(scratch_err[dev]));
        return DFX_ERR_HIP;
    }
    // Quantised weights: the chunk sums are added in chunk order whether K is split or not,
    // so a workspace too small for the split dfx_gemm would choose only makes the dispatch
    // keep K whole, with the same bits.  F16: the slice count decides the f32 summation
    // order, so the split dfx_gemm would choose must fit the array.  F32 and Q8_0 use no
    // workspace.
    const size_t full = M > 0 && N > 0 && K > 0 ? dfx_gemm_ws_bytes(M, N, K) : 0;
    if (wtype == DFX_TYPE_F16 && M > 0 && N > 0 && K > 0 && K % 256 == 0) {
        const int S = f16_splits(pick_tm((int)std::min<int64_t>(M, INT32_MAX), 4), M, N, K, full);
        const size_t need = S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
        if (need > DFX_GEMM_SCRATCH_BYTES) {
            dfx_set_error("dfx_gemm_noalloc: the F16 split's partial sums (%d slices, %zu bytes) exceed the %u-byte "
                          "scratch (M=%lld N=%lld K=%lld)", S, need, DFX_GEMM_SCRATCH_BYTES, (long long)M,
                          (long long)N, (long long)K);
            return DFX_ERR_ARG;
        }
    }
    const size_t ws_bytes = std::min<size_t>(full, DFX_GEMM_SCRATCH_BYTES);
    return dfx_gemm_ex(wtype, w, N, K, act, M, bias, residual, y, N, nullptr, scratch_ptr[dev], ws_bytes, stream,
                       nullptr, nullptr);
}
