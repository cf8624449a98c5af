// k_attn.hip — NEOX RoPE + KV-cache store, and bidirectional attention.
//
// The inter-step cache lives in HBM per layer as kc[pos][n_head_kv][head_dim] and the
// transposed vt[n_head_kv][head_dim][capacity] (f32); the attention reads four
// consecutive keys of one value column with one 16-byte load.  The reference keeps
// it expanded to n_head (src/diffuse-cache.h:23-26)
// and concatenates [cached ‖ active] keys (src/diffuse-graph.cpp:524-525); here the
// active rows are scattered into the cache first and every query attends over the
// cache in position order.  Softmax without a mask is invariant to key order, and
// the GQA repeat (src/diffuse-graph.cpp:84-95) is the index h / n_rep.
#include "dfx_device.h"

#include <algorithm>
#include <atomic>

// One workgroup per (32-row tile, head of Q|K|V), head size HD.  Q and K heads: wave
// w rotates rows w, w+4, .., w+28 of the tile; HD/8 lanes share a row, each rotating
// four consecutive pairs (i, i + HD/2) with 16-byte loads and stores; all rows' loads
// are issued before any arithmetic.  V heads: the tile passes through LDS so that the
// transposed store vt[kvh][dim][p] takes consecutive positions from consecutive lanes.
#define ROPE_RT 32
template <int HD>
__global__ void __launch_bounds__(256) k_rope_store(const float * __restrict__ qkv, const int32_t * __restrict__ pos,
                                                    int M, int H, int Hkv, const float * __restrict__ tab,
                                                    float * __restrict__ q_out, float * __restrict__ kc,
                                                    float * __restrict__ vt, int64_t v_ld) {
#pragma clang fp contract(off)
    constexpr int HALF = HD / 2;
    constexpr int RPW = ROPE_RT / 4;                        // rows per wave
    __shared__ float vtile[ROPE_RT * (HD + 1)];
    const int heads = H + 2 * Hkv;
    const int hh = blockIdx.y, m0 = blockIdx.x * ROPE_RT;
    const int rows = min(ROPE_RT, M - m0);
    const int64_t ld = (int64_t)heads * HD;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (hh < H + Hkv) {
        constexpr int LPR = HALF / 4;          // lanes per row, four pairs each
        constexpr int RPI = 64 / LPR;          // rows per pass of the wave
        constexpr int NIT = RPW / RPI;         // passes
        static_assert(HALF % 4 == 0 && 64 % LPR == 0 && NIT >= 1 && RPW % RPI == 0, "head size");
        const int lr = lane / LPR, j4 = 4 * (lane % LPR);
        int p[NIT];
        float4 a[NIT], b[NIT], c01[NIT], c23[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int m = m0 + min(wv + 4 * (it * RPI + lr), rows - 1);   // clamped: duplicates are not stored
            p[it] = pos[m];
            const float * src = qkv + m * ld + (int64_t)hh * HD + j4;
            a[it] = *(const float4 *)src;
            b[it] = *(const float4 *)(src + HALF);
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const float * cs = tab + ((int64_t)p[it] * HALF + j4) * 2;   // (cos, sin) of pairs j4 .. j4+3
            c01[it] = *(const float4 *)cs;
            c23[it] = *(const float4 *)(cs + 4);
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int r = wv + 4 * (it * RPI + lr);
            if (r >= rows) continue;
            const int m = m0 + r;
            const float x0[4] = {a[it].x, a[it].y, a[it].z, a[it].w}, x1[4] = {b[it].x, b[it].y, b[it].z, b[it].w};
            const float c[4] = {c01[it].x, c01[it].z, c23[it].x, c23[it].z};
            const float sn[4] = {c01[it].y, c01[it].w, c23[it].y, c23[it].w};
            float y0[4], y1[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                // ggml_rope_ext NEOX: rotate (i, i + n_dims/2) by theta_i(p)
                y0[k] = x0[k] * c[k] - x1[k] * sn[k];
                y1[k] = x0[k] * sn[k] + x1[k] * c[k];
            }
            float * dst = hh < H ? q_out + ((int64_t)m * H + hh) * HD : kc + ((int64_t)p[it] * Hkv + (hh - H)) * HD;
            *(float4 *)(dst + j4) = make_float4(y0[0], y0[1], y0[2], y0[3]);
            *(float4 *)(dst + HALF + j4) = make_float4(y1[0], y1[1], y1[2], y1[3]);
        }
    } else {
        const int kvh = hh - H - Hkv;
        constexpr int LS = HD + 1;
#pragma unroll
        for (int k = 0; k < ROPE_RT * HD / 256; k++) {
            const int e = threadIdx.x + 256 * k, r = e / HD, i = e % HD;
            if (r < rows) vtile[r * LS + i] = qkv[(int64_t)(m0 + r) * ld + (int64_t)hh * HD + i];
        }
        __syncthreads();
        // thread -> position r = tid % 32 (fixed), dimensions i = tid / 32 + 8k
        const int r = threadIdx.x & 31;
        if (r < rows) {
            const int p = pos[m0 + r];
#pragma unroll
            for (int k = 0; k < HD / 8; k++) {
                const int i = (threadIdx.x >> 5) + 8 * k;
                vt[((int64_t)kvh * HD + i) * v_ld + p] = vtile[r * LS + i];
            }
        }
    }
}

// Both attention kernels follow the reference op for op (src/diffuse-graph.cpp:107-114
// with GGML soft_max):
//   s = dot(k, q) * (1/sqrtf(hd));  max;  e = exp(s - max);  sum in double;
//   p = e * (float)(1/sum);  out = sum_n v_n * p_n.
// f32 x f32 products are exact in f64; the dot products and the P.V sums are
// accumulated in f64 and rounded to float once.  f64 addition is not associative,
// so the float result depends on the summation order only when two orders' f64
// sums fall on either side of a float rounding boundary: measured about one
// element in 10^6-10^7 differing by one float ulp from a sequential f64 sum.
// exp is correctly rounded.

typedef double double4v __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte load at an always valid address; `keep` false gives zeros.  Written without
// a branch around the load: a conditional load compiles to four predicated dword loads
// under their own branches, each waited for on its own.
__device__ __forceinline__ float4 ld4_or0(const float * p, bool keep) {
    const f32x4 v = *(const f32x4 *)p;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const f32x4 r = keep ? v : z;
    return make_float4(r.x, r.y, r.z, r.w);
}

// Causal mask (src/ar-graph.cpp:70-88): with q_pos0 >= 0, query row r sits at position
// q_pos0 + r and sees the keys lo..hi, hi = its position, lo = hi - window + 1 with a
// window (> 0), else 0.  q_pos0 < 0: every key is visible.  Rows past M (tile padding)
// take the last row's range, so every row keeps a visible key.
struct key_range { int lo, hi; };
__device__ __forceinline__ key_range row_keys(int row, int M, int n_keys, int q_pos0, int window) {
    if (q_pos0 < 0) return {0, n_keys - 1};
    const int hi = min(q_pos0 + min(row, M - 1), n_keys - 1);
    return {window > 0 ? max(hi - window + 1, 0) : 0, hi};
}

// v_mfma_f64_16x16x4f64: D[16][16] += A[16][4] B[4][16].
// Lane l supplies A[l%16][l/16] and B[l/16][l%16]; it holds D[l/16 + 4i][l%16], i < 4.
__device__ __forceinline__ double4v mfma_f64(double a, double b, double4v c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Matrix-core attention: one head and 16 query rows per workgroup of NW waves.
// Phase 1: S = Q K^T on the f64 MFMA; each wave takes key tiles of 16 (t = wave + NW j),
// the next tiles' keys are loaded while the current one multiplies (KR-slot ring), and
// the head dims are reduced in four independent accumulation chains (dims 16s+4g+c to
// MFMA c for step s), added at the end as (c0 + c1) + (c2 + c3).
// Phase 2: softmax, one wave per row, scores resident in LDS.
// Phase 3: O = P V on the f64 MFMA; wave w owns head-dim columns 16w+16 NW ct+(0..15),
// keys are the reduction: lane group g supplies keys 16s+4g+c to MFMA c, read as one
// float4 of the transposed value cache, four key steps ahead; two chains (c even / odd).
// Every output element's sums are the same for every NW: the wave count only decides which
// wave computes them.  With eight waves (and at most 128 VGPRs) two workgroups share a CU
// at four waves per SIMD, and each workgroup finishes in about half the time of four waves.
// Workgroups are numbered so that all query tiles of head h run on XCD h % 8.  With vs = 2
// (grids that leave CUs idle) each query tile runs as two workgroups that both form the scores
// and probabilities and take half of the value columns each (phase 3 on half the waves): the
// same operations for every output element, so the same bits.
template <int HD, int KR, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 4 : 1)))
k_attn_mfma(const float * __restrict__ q, const float * __restrict__ kc, const float * __restrict__ vt, int64_t v_ld,
            int M, int n_keys, int H, int Hkv, int sstride, int q_tiles, int q_pos0, int window,
            float * __restrict__ out, int vs) {
#pragma clang fp contract(off)
    extern __shared__ float S[];       // [16][sstride] scores, then probabilities
    constexpr int SS = HD / 16;        // reduction steps of 16 head dims
    constexpr int CT = HD / (16 * NW); // phase-3 column tiles per wave
    static_assert(CT >= 1 && CT * 16 * NW == HD, "head dims split evenly over the waves");
    const int L = blockIdx.x, xcd = L & 7, j = L >> 3, slots = q_tiles * vs;
    const int h = 8 * (j / slots) + xcd, qt = (j % slots) / vs, part = (j % slots) % vs;
    if (h >= H) return;
    const int kvh = h / (H / Hkv);
    const int q0 = qt * 16;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool pv = (wv * vs) / NW == part;   // this wave's value columns are this workgroup's
    const int li = lane & 15, lg = lane >> 4;
    const int64_t kvstride = (int64_t)Hkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int ntiles = (n_keys + 15) >> 4;

    // ---- phase 1
    float4 qf[SS];
    {
        const int row = q0 + li;
        const float * qr = q + ((int64_t)min(row, M - 1) * H + h) * HD + 4 * lg;
#pragma unroll
        for (int s = 0; s < SS; s++) qf[s] = ld4_or0(qr + 16 * s, row < M);
    }
    const float * kbase = kc + (int64_t)kvh * HD + 4 * lg;
    auto load_k = [&](float4 (&kf)[SS], int t) {
        const int n = 16 * t + li;
        const float * kr = kbase + (int64_t)min(n, n_keys - 1) * kvstride;
#pragma unroll
        for (int s = 0; s < SS; s++) kf[s] = ld4_or0(kr + 16 * s, n < n_keys);
    };
    // key tiles t = wv + NW j in a KR-slot register ring, KR - 1 tiles in flight ahead
    // of the one being multiplied (slot roles fixed by unrolling, so no copies)
    float4 kr[KR][SS];
    auto tile = [&](float4 (&kf)[SS], int t) __attribute__((always_inline)) {
        double4v a[4] = {0.0, 0.0, 0.0, 0.0};      // four independent chains: MFMA c of each step
#pragma unroll
        for (int s = 0; s < SS; s++) {
            const float kb[4] = {kf[s].x, kf[s].y, kf[s].z, kf[s].w};
            float qa[4] = {qf[s].x, qf[s].y, qf[s].z, qf[s].w};
            if constexpr (NW == 8) {
                // converted to double at each use, not once for the whole kernel: the 64
                // VGPRs of a hoisted double copy do not fit four waves per SIMD
#pragma unroll
                for (int c = 0; c < 4; c++) asm volatile("" : "+v"(qa[c]));
            }
#pragma unroll
            for (int c = 0; c < 4; c++) a[c] = mfma_f64((double)qa[c], (double)kb[c], a[c]);
        }
        const double4v acc = (a[0] + a[1]) + (a[2] + a[3]);
        const int n = 16 * t + li;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // masked keys score -inf: weight exactly 0 in the sums below
            const key_range kr = row_keys(q0 + lg + 4 * i, M, n_keys, q_pos0, window);
            S[(lg + 4 * i) * sstride + n] = n >= kr.lo && n <= kr.hi ? (float)acc[i] * scale : -INFINITY;
        }
    };
#pragma unroll
    for (int u = 0; u < KR; u++)
        if (wv + NW * u < ntiles) load_k(kr[u], wv + NW * u);
    for (int t0 = wv; t0 < ntiles; t0 += NW * KR) {
#pragma unroll
        for (int u = 0; u < KR; u++) {
            const int t = t0 + NW * u;
            if (t < ntiles) {
                tile(kr[u], t);
                if (t + NW * KR < ntiles) load_k(kr[u], t + NW * KR);
            }
        }
    }
    __syncthreads();

    // The first value steps of phase 3 are loaded here, so that their latency passes under the
    // softmax.  Value column of this lane for column tile ct: 16*wv + 16*NW*ct + li; keys
    // 16s+4g..+3.
    const float * vb = vt + ((int64_t)kvh * HD + 16 * wv + li) * v_ld + 4 * lg;
    auto load_v = [&](float4 (&vf)[CT], int s) {
        const int n = 16 * s + 4 * lg;                 // first of this lane's 4 keys
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const float * p = vb + (int64_t)16 * NW * ct * v_ld + 16 * min(s, ntiles - 1);
            // v_ld and n are multiples of 4 and n_keys <= v_ld: the load stays in the row;
            // keys past the end of the sequence count as 0
            const f32x4 v = *(const f32x4 *)p;
            vf[ct] = make_float4(n < n_keys ? v.x : 0.0f, n + 1 < n_keys ? v.y : 0.0f, n + 2 < n_keys ? v.z : 0.0f,
                                 n + 3 < n_keys ? v.w : 0.0f);
        }
    };
    constexpr int PV = 4;                           // value steps in flight
    float4 vq[PV][CT];
    if (pv)
#pragma unroll
        for (int u = 0; u < PV; u++) load_v(vq[u], u);

    // ---- phase 2: the wave's RPW rows (wv, wv + NW, ..) together, four keys per lane and
    // row at a time, so that RPW * 4 exponentials and the rows' reductions are in flight at
    // once.  Each lane sums its keys lane, lane + 64, .. in increasing order and the lanes
    // are added by the xor butterfly, one row as another.
    {
        constexpr int RPW = 16 / NW;
        float mx[RPW];
#pragma unroll
        for (int q = 0; q < RPW; q++) mx[q] = -INFINITY;
        for (int n0 = lane; n0 < n_keys; n0 += 256)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int n = n0 + 64 * u;
#pragma unroll
                for (int q = 0; q < RPW; q++)
                    if (n < n_keys) mx[q] = fmaxf(mx[q], S[(wv + NW * q) * sstride + n]);
            }
#pragma unroll
        for (int q = 0; q < RPW; q++) mx[q] = wave_max(mx[q]);
        double sum[RPW];
#pragma unroll
        for (int q = 0; q < RPW; q++) sum[q] = 0.0;
        for (int n0 = lane; n0 < n_keys; n0 += 256) {
            float e[RPW][4];
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int q = 0; q < RPW; q++) {
                    const int n = min(n0 + 64 * u, n_keys - 1);
                    e[q][u] = (float)exp((double)(S[(wv + NW * q) * sstride + n] - mx[q]));
                }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int n = n0 + 64 * u;
                if (n < n_keys)
#pragma unroll
                    for (int q = 0; q < RPW; q++) {
                        S[(wv + NW * q) * sstride + n] = e[q][u];
                        sum[q] += (double)e[q][u];
                    }
            }
        }
        float inv[RPW];
#pragma unroll
        for (int q = 0; q < RPW; q++) {
            sum[q] = wave_sum_d(sum[q]);
            inv[q] = (float)(1.0 / sum[q]);
        }
        for (int n0 = lane; n0 < n_keys; n0 += 256)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int n = n0 + 64 * u;
                if (n < n_keys)
#pragma unroll
                    for (int q = 0; q < RPW; q++) S[(wv + NW * q) * sstride + n] *= inv[q];
            }
#pragma unroll
        for (int q = 0; q < RPW; q++)
            for (int n = n_keys + lane; n < 16 * ntiles; n += 64) S[(wv + NW * q) * sstride + n] = 0.0f;
    }
    __syncthreads();

    // ---- phase 3
    if (!pv) return;
    double4v o[CT][2];                              // chains: column tile x MFMA parity
#pragma unroll
    for (int ct = 0; ct < CT; ct++) o[ct][0] = o[ct][1] = 0.0;
    for (int s0 = 0; s0 < ntiles; s0 += PV) {
#pragma unroll
        for (int u = 0; u < PV; u++) {
            const int s = s0 + u;
            if (s < ntiles) {
                float4 vcur[CT];
#pragma unroll
                for (int ct = 0; ct < CT; ct++) vcur[ct] = vq[u][ct];
                load_v(vq[u], s + PV);
                const float4 pf = *(const float4 *)(S + li * sstride + 16 * s + 4 * lg);
                const float pa[4] = {pf.x, pf.y, pf.z, pf.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const double a = (double)pa[c];
#pragma unroll
                    for (int ct = 0; ct < CT; ct++) {
                        const float vv[4] = {vcur[ct].x, vcur[ct].y, vcur[ct].z, vcur[ct].w};
                        o[ct][c & 1] = mfma_f64(a, (double)vv[c], o[ct][c & 1]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = q0 + lg + 4 * i;
        if (row >= M) continue;
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
            out[(int64_t)row * H * HD + (int64_t)h * HD + 16 * wv + 16 * NW * ct + li] =
                (float)(o[ct][0][i] + o[ct][1][i]);
    }
}

// ---- split-bf16 matrix-core attention (the default)
//
// Every f32 operand x is split into three bf16 parts, x = hi + mid + lo with
// hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid) (each rounded to nearest,
// each difference exact in f32), and a product x*y is taken as the six terms down to
// 2^-16 of it: hi*hi into one f32 sum and hi*mid + mid*hi + hi*lo + lo*hi + mid*mid
// into a second, whose values are 2^-8 of the first, so its own rounding is far below
// f32's.  What is left out (mid*lo, lo*mid, lo*lo and lo's rounding) is below 2^-25 of
// |x*y|: the products are as accurate as f32 ones, on the bf16 MFMA.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

struct bf16x3 {
    bf16x8 h, m, l;
};

__device__ __forceinline__ bf16x3 split_bf16x8(f32x4 a, f32x4 b) {
    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16x3 r;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const f32x2 v = {x[e], x[e + 1]};
        const bf16x2 h = __builtin_convertvector(v, bf16x2);
        const f32x2 r1 = v - __builtin_convertvector(h, f32x2);
        const bf16x2 m = __builtin_convertvector(r1, bf16x2);
        const bf16x2 l = __builtin_convertvector(r1 - __builtin_convertvector(m, f32x2), bf16x2);
        r.h[e] = h[0];
        r.h[e + 1] = h[1];
        r.m[e] = m[0];
        r.m[e + 1] = m[1];
        r.l[e] = l[0];
        r.l[e + 1] = l[1];
    }
    return r;
}

// D = big + low at the end.
struct split_acc {
    float16v big, low;
};

__device__ __forceinline__ void mfma_split(const bf16x3 & a, const bf16x3 & b, split_acc & d) {
    d.big = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.h, d.big, 0, 0, 0);
    d.low = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.m, b.m, d.low, 0, 0, 0);
    d.low = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.l, d.low, 0, 0, 0);
    d.low = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.l, b.h, d.low, 0, 0, 0);
    d.low = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.m, d.low, 0, 0, 0);
    d.low = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.m, b.h, d.low, 0, 0, 0);
}

__device__ __forceinline__ float16v split_sum(const split_acc & d) { return d.big + d.low; }

// max / sum over the 8 lanes of an aligned lane group
__device__ __forceinline__ float group8_max(float v) {
    for (int o = 4; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}
__device__ __forceinline__ double group8_sum_d(double v) {
    for (int o = 4; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// One head and 32 query rows per workgroup (4 waves, two workgroups per CU), the
// softmax of the reference (src/diffuse-graph.cpp:107-114 with GGML soft_max:
// s = dot(k, q) * (1/sqrtf(hd)), e = exp(s - max), sum in double, p = e * (float)(1/sum))
// with f32 exp.
// v_mfma_f32_32x32x16_bf16: lane l supplies A[l%32][8*(l/32) + e] and B[8*(l/32) + e][l%32],
// e < 8, and holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r < 16.
// Phase 1: S = Q K^T, key tiles of 32 (t = wave + 4j); the query fragments stay in
// registers; each half tile of keys (64 head dims) is loaded while the other multiplies.
// Phase 2: softmax with the scores resident in LDS, wave w taking rows 8w..8w+7 at once,
// eight lanes per row.
// Phase 3: O = P V: wave w owns output columns 32*(w % CT)..+31 and key steps of 16
// s = w / CT (mod 4 / CT); with HD = 64 two waves share a column tile and their sums
// are added through LDS.
// Workgroups are numbered so that all query tiles of head h run on XCD h % 8.
#define ATTN_QT 32
template <int HD>
__global__ void __launch_bounds__(256, 2) k_attn_split(const float * __restrict__ q, const float * __restrict__ kc,
                                                       const float * __restrict__ vt, int64_t v_ld, int M, int n_keys,
                                                       int H, int Hkv, int sstride, int q_tiles,
                                                       float * __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ float S[];       // [32][sstride] scores, then probabilities; [2][64][16] partial sums
    constexpr int QS = HD / 16;        // reduction steps of 16 head dims
    constexpr int HS = QS / 2;         // steps per half tile
    constexpr int CT = HD / 32;        // 32-column output tiles
    constexpr int KW = 4 / CT;         // waves per output tile (key-step interleave)
    const int L = blockIdx.x, xcd = L & 7, j = L >> 3;
    const int h = 8 * (j / q_tiles) + xcd, qt = j % q_tiles;
    if (h >= H) return;
    const int kvh = h / (H / Hkv);
    const int q0 = qt * ATTN_QT;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l32 = lane & 31, hl = lane >> 5;
    const int64_t kvstride = (int64_t)Hkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int ntiles = (n_keys + 31) >> 5;

    // ---- phase 1
    bf16x3 qs[QS];
    {
        const int row = q0 + l32;
        const float * qr = q + ((int64_t)min(row, M - 1) * H + h) * HD + 8 * hl;
#pragma unroll
        for (int s = 0; s < QS; s++) {
            const float4 a = ld4_or0(qr + 16 * s, row < M), b = ld4_or0(qr + 16 * s + 4, row < M);
            qs[s] = split_bf16x8(f32x4{a.x, a.y, a.z, a.w}, f32x4{b.x, b.y, b.z, b.w});
        }
    }
    const float * kbase = kc + (int64_t)kvh * HD + 8 * hl;
    // steps HS*half .. HS*half + HS-1 of key tile t: lane holds key 32t + l32, dims 16s + 8hl .. +7
    auto load_kh = [&](f32x4 (&kf)[2 * HS], int t, int half) __attribute__((always_inline)) {
        const int n = 32 * t + l32;
        const float * kr = kbase + (int64_t)min(n, n_keys - 1) * kvstride + 16 * HS * half;
#pragma unroll
        for (int s = 0; s < HS; s++) {
            const float4 a = ld4_or0(kr + 16 * s, n < n_keys), b = ld4_or0(kr + 16 * s + 4, n < n_keys);
            kf[2 * s] = f32x4{a.x, a.y, a.z, a.w};
            kf[2 * s + 1] = f32x4{b.x, b.y, b.z, b.w};
        }
    };
    auto mul_half = [&](const f32x4 (&kf)[2 * HS], int half, split_acc & d) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < HS; s++) mfma_split(qs[HS * half + s], split_bf16x8(kf[2 * s], kf[2 * s + 1]), d);
    };
    f32x4 k0[2 * HS], k1[2 * HS];
    if (wv < ntiles) {
        load_kh(k0, wv, 0);
        load_kh(k1, wv, 1);
    }
    for (int t = wv; t < ntiles; t += 4) {
        split_acc d = {};
        mul_half(k0, 0, d);
        if (t + 4 < ntiles) load_kh(k0, t + 4, 0);
        mul_half(k1, 1, d);
        if (t + 4 < ntiles) load_kh(k1, t + 4, 1);
        const float16v acc = split_sum(d);
#pragma unroll
        for (int r = 0; r < 16; r++)
            S[(8 * (r >> 2) + 4 * hl + (r & 3)) * sstride + 32 * t + l32] = acc[r] * scale;
    }
    __syncthreads();

    // ---- phase 2: keys >= n_keys (up to the 32-key tile) get probability 0
    {
        float * sr = S + (8 * wv + (lane >> 3)) * sstride;
        const int c0 = 4 * (lane & 7), nk32 = 32 * ntiles;
        float mx = -INFINITY;
        for (int n = c0; n < nk32; n += 32) {
            const f32x4 v = *(const f32x4 *)(sr + n);
            mx = fmaxf(mx, fmaxf(fmaxf(n < n_keys ? v.x : -INFINITY, n + 1 < n_keys ? v.y : -INFINITY),
                                 fmaxf(n + 2 < n_keys ? v.z : -INFINITY, n + 3 < n_keys ? v.w : -INFINITY)));
        }
        mx = group8_max(mx);
        double sum = 0.0;
        for (int n = c0; n < nk32; n += 32) {
            const f32x4 v = *(const f32x4 *)(sr + n);
            const f32x4 e = {n < n_keys ? expf(v.x - mx) : 0.0f, n + 1 < n_keys ? expf(v.y - mx) : 0.0f,
                             n + 2 < n_keys ? expf(v.z - mx) : 0.0f, n + 3 < n_keys ? expf(v.w - mx) : 0.0f};
            *(f32x4 *)(sr + n) = e;
            sum += ((double)e.x + (double)e.y) + ((double)e.z + (double)e.w);
        }
        sum = group8_sum_d(sum);
        const float inv = (float)(1.0 / sum);
        for (int n = c0; n < nk32; n += 32) {
            const f32x4 e = *(const f32x4 *)(sr + n);
            *(f32x4 *)(sr + n) = f32x4{e.x * inv, e.y * inv, e.z * inv, e.w * inv};
        }
    }
    __syncthreads();

    // ---- phase 3
    const int ct = wv % CT, kw = wv / CT;
    split_acc d = {};
    // value column 32*ct + l32 of this lane; keys 16s + 8*hl .. +7
    const float * vb = vt + ((int64_t)kvh * HD + 32 * ct + l32) * v_ld;
    const int nsteps = 2 * ntiles;
    auto load_v = [&](f32x4 (&vf)[2], int s) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int n = 16 * s + 8 * hl + 4 * u;
            // n and v_ld are multiples of 4 and n_keys <= v_ld: a load at n < n_keys stays in
            // the row; past the sequence, key 0 is read and every key >= n_keys counts as 0
            const f32x4 v = *(const f32x4 *)(vb + (n < n_keys ? n : 0));
            vf[u] = f32x4{n < n_keys ? v.x : 0.0f, n + 1 < n_keys ? v.y : 0.0f, n + 2 < n_keys ? v.z : 0.0f,
                          n + 3 < n_keys ? v.w : 0.0f};
        }
    };
    constexpr int PV = 4;                           // value steps in flight
    f32x4 vq[PV][2];
#pragma unroll
    for (int u = 0; u < PV; u++) load_v(vq[u], kw + KW * u);
    for (int s0 = kw; s0 < nsteps; s0 += KW * PV) {
#pragma unroll
        for (int u = 0; u < PV; u++) {
            const int s = s0 + KW * u;
            if (s < nsteps) {
                const f32x4 v0 = vq[u][0], v1 = vq[u][1];
                load_v(vq[u], s + KW * PV);
                const float * pr = S + l32 * sstride + 16 * s + 8 * hl;
                const f32x4 p0 = *(const f32x4 *)pr, p1 = *(const f32x4 *)(pr + 4);
                mfma_split(split_bf16x8(p0, p1), split_bf16x8(v0, v1), d);
            }
        }
    }
    float16v o = split_sum(d);
    if constexpr (KW > 1) {
        float * part = S + ATTN_QT * sstride;      // [64 lanes][16] of the second key half
        __syncthreads();
        if (kw == 1) {
#pragma unroll
            for (int r = 0; r < 16; r += 4)
                *(f32x4 *)(part + (ct * 64 + lane) * 16 + r) = f32x4{o[r], o[r + 1], o[r + 2], o[r + 3]};
        }
        __syncthreads();
        if (kw == 1) return;
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
            const f32x4 w = *(const f32x4 *)(part + (ct * 64 + lane) * 16 + r);
            o[r] += w.x;
            o[r + 1] += w.y;
            o[r + 2] += w.z;
            o[r + 3] += w.w;
        }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int row = q0 + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (row < M) out[(int64_t)row * H * HD + (int64_t)h * HD + 32 * ct + l32] = o[r];
    }
}

// Exact form for any key count: the score rows are not kept (they need not fit the LDS);
// each 16-key score tile is recomputed in three passes over the keys, with the same
// products, sums and rounding as k_attn_mfma's phase 1, so every pass sees the same scores:
//   pass 1: row maxima;
//   pass 2: e = exp(s - max) (correctly rounded), sums in double, inv = (float)(1 / sum);
//   pass 3: per block of 64 keys, the four waves' probability tiles p = e * inv go through
//           LDS and each wave adds P V for its value columns on the f64 MFMA.
// One head and 16 query rows per workgroup (4 waves); wave w takes the score tile 4b + w of
// key block b.  Keys past n_keys score -inf (no weight) and read as zero values.
#define LONG_PSTR 68   // LDS floats per probability row of a 64-key block (16-byte aligned rows)
template <int HD>
__global__ void __launch_bounds__(256) k_attn_long(const float * __restrict__ q, const float * __restrict__ kc,
                                                   const float * __restrict__ vt, int64_t v_ld, int M, int n_keys,
                                                   int H, int Hkv, int q_tiles, int q_pos0, int window,
                                                   float * __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float P[16 * LONG_PSTR];
    __shared__ float red_f[4][16];
    __shared__ double red_d[4][16];
    constexpr int SS = HD / 16, CT = HD / 64;
    const int L = blockIdx.x, xcd = L & 7, j = L >> 3;
    const int h = 8 * (j / q_tiles) + xcd, qt = j % q_tiles;
    if (h >= H) return;
    const int kvh = h / (H / Hkv);
    const int q0 = qt * 16;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int64_t kvstride = (int64_t)Hkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int ntiles = (n_keys + 15) >> 4, nblocks = (ntiles + 3) >> 2;

    float4 qf[SS];
    {
        const int row = q0 + li;
        const float * qr = q + ((int64_t)min(row, M - 1) * H + h) * HD + 4 * lg;
#pragma unroll
        for (int s = 0; s < SS; s++) qf[s] = ld4_or0(qr + 16 * s, row < M);
    }
    const float * kbase = kc + (int64_t)kvh * HD + 4 * lg;
    // scores of tile t for rows lg + 4i, key 16t + li (-inf past the keys)
    auto scores = [&](int t, float (&sc)[4]) __attribute__((always_inline)) {
        const int n = 16 * t + li;
        const float * kr = kbase + (int64_t)min(n, n_keys - 1) * kvstride;
        float4 kf[SS];
#pragma unroll
        for (int s = 0; s < SS; s++) kf[s] = ld4_or0(kr + 16 * s, n < n_keys);
        double4v a[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int s = 0; s < SS; s++) {
            const float kb[4] = {kf[s].x, kf[s].y, kf[s].z, kf[s].w};
            const float qa[4] = {qf[s].x, qf[s].y, qf[s].z, qf[s].w};
#pragma unroll
            for (int c = 0; c < 4; c++) a[c] = mfma_f64((double)qa[c], (double)kb[c], a[c]);
        }
        const double4v acc = (a[0] + a[1]) + (a[2] + a[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const key_range kr = row_keys(q0 + lg + 4 * i, M, n_keys, q_pos0, window);
            sc[i] = n >= kr.lo && n <= kr.hi ? (float)acc[i] * scale : -INFINITY;
        }
    };

    // ---- pass 1: row maxima (lane: rows lg + 4i)
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int t = wv; t < ntiles; t += 4) {
        float sc[4];
        scores(t, sc);
#pragma unroll
        for (int i = 0; i < 4; i++) mx[i] = fmaxf(mx[i], sc[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        for (int o = 8; o > 0; o >>= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], o, WAVE));   // over li
        if (li == 0) red_f[wv][lg + 4 * i] = mx[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = lg + 4 * i;
        mx[i] = fmaxf(fmaxf(red_f[0][r], red_f[1][r]), fmaxf(red_f[2][r], red_f[3][r]));
    }

    // ---- pass 2: sums of e = exp(s - max) in double
    double sum[4] = {0.0, 0.0, 0.0, 0.0};
    for (int t = wv; t < ntiles; t += 4) {
        float sc[4];
        scores(t, sc);
#pragma unroll
        for (int i = 0; i < 4; i++) sum[i] += (double)(float)exp((double)(sc[i] - mx[i]));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        for (int o = 8; o > 0; o >>= 1) sum[i] += __shfl_xor(sum[i], o, WAVE);
        if (li == 0) red_d[wv][lg + 4 * i] = sum[i];
    }
    __syncthreads();
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = lg + 4 * i;
        inv[i] = (float)(1.0 / (((red_d[0][r] + red_d[1][r]) + red_d[2][r]) + red_d[3][r]));
    }

    // ---- pass 3: O = P V, one 64-key block at a time
    double4v o[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) o[ct][0] = o[ct][1] = 0.0;
    const float * vb = vt + ((int64_t)kvh * HD + 16 * wv + li) * v_ld;
    for (int b = 0; b < nblocks; b++) {
        const int t = 4 * b + wv;
        float sc[4];
        scores(min(t, ntiles - 1), sc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float e = (float)exp((double)(sc[i] - mx[i]));
            P[(lg + 4 * i) * LONG_PSTR + 16 * wv + li] = t < ntiles ? e * inv[i] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int n = 64 * b + 16 * s + 4 * lg;          // first of this lane's 4 keys
            const float4 pf = *(const float4 *)(P + li * LONG_PSTR + 16 * s + 4 * lg);
            const float pa[4] = {pf.x, pf.y, pf.z, pf.w};
            float4 vv[CT];
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                // in-row address (v_ld is a multiple of 16, so a row holds whole 16-key steps
                // of the cache); keys past the sequence read as zero
                const f32x4 v = *(const f32x4 *)(vb + (int64_t)64 * ct * v_ld + min(n, (int)v_ld - 4));
                vv[ct] = make_float4(n < n_keys ? v.x : 0.0f, n + 1 < n_keys ? v.y : 0.0f,
                                     n + 2 < n_keys ? v.z : 0.0f, n + 3 < n_keys ? v.w : 0.0f);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const double a = (double)pa[c];
#pragma unroll
                for (int ct = 0; ct < CT; ct++) {
                    const float vvv[4] = {vv[ct].x, vv[ct].y, vv[ct].z, vv[ct].w};
                    o[ct][c & 1] = mfma_f64(a, (double)vvv[c], o[ct][c & 1]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = q0 + lg + 4 * i;
        if (row >= M) continue;
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
            out[(int64_t)row * H * HD + (int64_t)h * HD + 16 * wv + 64 * ct + li] = (float)(o[ct][0][i] + o[ct][1][i]);
    }
}

// Few query rows (autoregressive decoding: one row per token): one workgroup of 4 waves per
// (row, head) instead of a 16-row tile per head.  Scores: 16 lanes per key, each adding the
// products of its HD/16 dimensions in f64 (f32 x f32 products are exact there), the 16 partial
// sums added by an xor butterfly, rounded to float and scaled; 16 keys per round.  Softmax as the
// oracle: max, e = (float)exp((double)(s - max)), sum in double, p = e * (float)(1 / sum).
// Output: HD dimensions x 256/HD key ranges per workgroup, each range summed in f64 in key order
// (16-byte loads of the transposed value cache), the ranges' f64 sums added in order, rounded to
// float once.  Only the f64 summation order differs from the oracle's (as in the matrix-core
// kernels): a float result differs where two orders straddle a rounding boundary.
// At most ROWS_MAX_KEYS visible keys per row.
#define ROWS_MAX_KEYS 1024
template <int HD>
__global__ void __launch_bounds__(256) k_attn_rows(const float * __restrict__ q, const float * __restrict__ kc,
                                                   const float * __restrict__ vt, int64_t v_ld, int M, int n_keys,
                                                   int H, int Hkv, int q_pos0, int window, float * __restrict__ out) {
#pragma clang fp contract(off)
    constexpr int DPL = HD / 16;            // dimensions per lane of a key's group
    constexpr int PARTS = 256 / HD;         // key ranges of the output sums
    __shared__ float sc[ROWS_MAX_KEYS];
    __shared__ float red[4];
    __shared__ double red_d[4];
    __shared__ double part[PARTS][HD];
    const int h = blockIdx.x % H, row = blockIdx.x / H;
    const int kvh = h / (H / Hkv);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const key_range kr = row_keys(row, M, n_keys, q_pos0, window);
    const int nk = kr.hi - kr.lo + 1;
    const float scale = 1.0f / sqrtf((float)HD);
    const int sub = lane & 15, grp = (tid >> 4);            // grp: key slot 0..15 of a round
    float qd[DPL];
    {
        const float * qr = q + ((int64_t)row * H + h) * HD + DPL * sub;
#pragma unroll
        for (int i = 0; i < DPL; i += 4) {
            const float4 v = *(const float4 *)(qr + i);
            qd[i] = v.x; qd[i + 1] = v.y; qd[i + 2] = v.z; qd[i + 3] = v.w;
        }
    }
    // output work of this thread (used after the softmax): dimension d, key range pt of PARTS
    // (range borders on multiples of 4 keys); the range's first PV x 4 values are requested now,
    // so that their latency passes during the scores and the softmax
    constexpr int PV = 8;
    const int d = tid % HD, pt = tid / HD;
    const int per = ((nk + PARTS - 1) / PARTS + 3) & ~3;
    const int ra = kr.lo + pt * per, rb = min(kr.lo + (pt + 1) * per, kr.hi + 1);
    const float * vr = vt + ((int64_t)kvh * HD + d) * v_ld;
    const int pa = (ra + 3) & ~3;                 // first 16-byte aligned key of the range
    float4 vpre[PV];
#pragma unroll
    for (int u = 0; u < PV; u++) vpre[u] = *(const float4 *)(vr + min(pa + 4 * u, (int)(v_ld - 4)));
    const int64_t kvstride = (int64_t)Hkv * HD;
    float mx = -INFINITY;
    // RK keys per lane group and round, all their loads issued before any arithmetic (a round
    // at a time would wait out one memory latency per 16 keys)
    constexpr int RK = 8;
    for (int j0 = 0; j0 < nk; j0 += 16 * RK) {
        float4 kv[RK][DPL / 4];
#pragma unroll
        for (int u = 0; u < RK; u++) {
            const int j = min(j0 + grp + 16 * u, nk - 1);
            const float * kp = kc + (int64_t)(kr.lo + j) * kvstride + (int64_t)kvh * HD + DPL * sub;
#pragma unroll
            for (int i = 0; i < DPL / 4; i++) kv[u][i] = *(const float4 *)(kp + 4 * i);
        }
#pragma unroll
        for (int u = 0; u < RK; u++) {
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < DPL / 4; i++) {
                acc = acc + (double)kv[u][i].x * (double)qd[4 * i];
                acc = acc + (double)kv[u][i].y * (double)qd[4 * i + 1];
                acc = acc + (double)kv[u][i].z * (double)qd[4 * i + 2];
                acc = acc + (double)kv[u][i].w * (double)qd[4 * i + 3];
            }
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
            const int j = j0 + grp + 16 * u;
            if (sub == 0 && j < nk) {
                const float sv = (float)acc * scale;
                sc[j] = sv;
                mx = fmaxf(mx, sv);
            }
        }
    }
    mx = wave_max(mx);
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    double sum = 0.0;
    for (int j = tid; j < nk; j += 256) {
        const float e = (float)exp((double)(sc[j] - mx));
        sc[j] = e;
        sum += (double)e;
    }
    sum = wave_sum_d(sum);
    if (lane == 0) red_d[wv] = sum;
    __syncthreads();
    const float inv = (float)(1.0 / (((red_d[0] + red_d[1]) + red_d[2]) + red_d[3]));
    for (int j = tid; j < nk; j += 256) sc[j] = sc[j] * inv;
    __syncthreads();
    {
        double acc = 0.0;
        int n = ra;
        for (; n < rb && (n & 3); n++) acc = acc + (double)vr[n] * (double)sc[n - kr.lo];
        // n == pa here (or the range is done): the prefetched 16-byte groups first
#pragma unroll
        for (int u = 0; u < PV; u++) {
            if (n + 4 <= rb) {
                const float * pp = sc + (n - kr.lo);
                acc = acc + (double)vpre[u].x * (double)pp[0];
                acc = acc + (double)vpre[u].y * (double)pp[1];
                acc = acc + (double)vpre[u].z * (double)pp[2];
                acc = acc + (double)vpre[u].w * (double)pp[3];
                n += 4;
            }
        }
        // 16 keys (four 16-byte loads) in flight per step
        for (; n + 16 <= rb; n += 16) {
            float4 v4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v4[u] = *(const float4 *)(vr + n + 4 * u);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float * pp = sc + (n + 4 * u - kr.lo);
                acc = acc + (double)v4[u].x * (double)pp[0];
                acc = acc + (double)v4[u].y * (double)pp[1];
                acc = acc + (double)v4[u].z * (double)pp[2];
                acc = acc + (double)v4[u].w * (double)pp[3];
            }
        }
        for (; n + 4 <= rb; n += 4) {
            const float4 v4 = *(const float4 *)(vr + n);
            const float * pp = sc + (n - kr.lo);
            acc = acc + (double)v4.x * (double)pp[0];
            acc = acc + (double)v4.y * (double)pp[1];
            acc = acc + (double)v4.z * (double)pp[2];
            acc = acc + (double)v4.w * (double)pp[3];
        }
        for (; n < rb; n++) acc = acc + (double)vr[n] * (double)sc[n - kr.lo];
        part[pt][d] = acc;
    }
    __syncthreads();
    if (tid < HD) {
        double acc = part[0][tid];
#pragma unroll
        for (int pt = 1; pt < PARTS; pt++) acc += part[pt][tid];
        out[(int64_t)row * H * HD + (int64_t)h * HD + tid] = (float)acc;
    }
}

extern "C" int dfx_rope_store(const float * qkv, const int32_t * pos, int64_t M, int H, int Hkv, int hd,
                              const float * tab, float * q_out, float * kc, float * vt, int64_t v_ld, void * stream) {
    if (M < 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || (hd & 1) || v_ld <= 0) {
        dfx_set_error("dfx_rope_store: bad shape M=%lld H=%d Hkv=%d hd=%d v_ld=%lld", (long long)M, H, Hkv, hd,
                      (long long)v_ld);
        return DFX_ERR_ARG;
    }
    if (M == 0) return DFX_OK;
    if (M > INT32_MAX - ROPE_RT || H + 2 * Hkv > 65535) {
        dfx_set_error("dfx_rope_store: shape too large M=%lld heads=%d hd=%d", (long long)M, H + 2 * Hkv, hd);
        return DFX_ERR_ARG;
    }
    const dim3 grid((unsigned)((M + ROPE_RT - 1) / ROPE_RT), (unsigned)(H + 2 * Hkv));
    if (hd == 128)
        hipLaunchKernelGGL(k_rope_store<128>, grid, dim3(256), 0, (hipStream_t)stream, qkv, pos, (int)M, H, Hkv, tab,
                           q_out, kc, vt, v_ld);
    else if (hd == 64)
        hipLaunchKernelGGL(k_rope_store<64>, grid, dim3(256), 0, (hipStream_t)stream, qkv, pos, (int)M, H, Hkv, tab,
                           q_out, kc, vt, v_ld);
    else {
        dfx_set_error("dfx_rope_store: head size %d (64 or 128 supported)", hd);
        return DFX_ERR_UNSUPPORTED;
    }
    DFX_CHECK_LAUNCH("dfx_rope_store");
    return DFX_OK;
}

// Compute units of the current device, read once per device.
static int attn_cu_count() {
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

// LDS a workgroup may use on the current device (160 KB on gfx950), read once per device
// (contexts on several host threads may ask at once).
static size_t attn_lds_limit() {
    static std::atomic<size_t> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    size_t v = cached[dev].load(std::memory_order_relaxed);
    if (!v) {
        int a = 0;
        if (hipDeviceGetAttribute(&a, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || a <= 0)
            a = 64 * 1024;
        v = (size_t)a;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Score-row stride of the matrix-core kernel: whole 16-key tiles, plus 4 floats so
// rows of a 16-row fragment start in different LDS banks.
static inline int attn_sstride(int64_t n_keys) { return (int)(((n_keys + 15) / 16) * 16 + 4); }

// Score-row stride of the split-bf16 kernel: whole 32-key tiles, plus 4 floats.
static inline int attn_split_sstride(int64_t n_keys) { return (int)(((n_keys + 31) / 32) * 32 + 4); }

#ifndef ATTN_NW
#define ATTN_NW 8   // waves per workgroup of the 128-wide exact kernel
#endif

// The exact (f64-summed) kernels: scores kept in LDS when a 16-row tile of them fits,
// else recomputed in three passes.  q_pos0 / window: the causal mask (q_pos0 < 0: none).
static int attn_exact(const float * q, const float * kc, const float * vt, int64_t v_ld, int M, int n_keys, int H,
                      int Hkv, int hd, int q_pos0, int window, float * out, hipStream_t st) {
    if (M <= 4 && n_keys <= ROWS_MAX_KEYS) {
        // decoding: one workgroup per (row, head) instead of a 16-row tile per head
        const dim3 grid((unsigned)(M * H));
        if (hd == 128)
            hipLaunchKernelGGL((k_attn_rows<128>), grid, dim3(256), 0, st, q, kc, vt, v_ld, M, n_keys, H, Hkv, q_pos0,
                               window, out);
        else
            hipLaunchKernelGGL((k_attn_rows<64>), grid, dim3(256), 0, st, q, kc, vt, v_ld, M, n_keys, H, Hkv, q_pos0,
                               window, out);
        DFX_CHECK_LAUNCH("dfx_attention (few rows)");
        return DFX_OK;
    }
    const int sstride = attn_sstride(n_keys);
    const size_t lds = (size_t)16 * sstride * sizeof(float);
    const int q_tiles = (M + 15) / 16;
    const dim3 grid((unsigned)(8 * ((H + 7) / 8) * q_tiles));
    // value columns split over two workgroups per query tile where twice the grid still gives
    // each CU at most one workgroup (LLaDA-8B at 50 rows, Dream-7B at 12-64 rows: 11-12 % less
    // attention time; slower on larger grids, where the second workgroup shares a CU)
    const int vs = 2 * (int)grid.x <= attn_cu_count() ? 2 : 1;
    const dim3 grid_vs((unsigned)(8 * ((H + 7) / 8) * q_tiles * vs));
    if (lds <= attn_lds_limit()) {
        // 128 dims: eight waves, a one-slot key ring (at most 128 VGPRs: four waves per SIMD);
        // 64 dims: four waves, three slots
        if (hd == 128 && ATTN_NW == 8)
            hipLaunchKernelGGL((k_attn_mfma<128, 1, 8>), grid_vs, dim3(512), lds, st, q, kc, vt, v_ld, M, n_keys, H, Hkv,
                               sstride, q_tiles, q_pos0, window, out, vs);
        else if (hd == 128)
            hipLaunchKernelGGL((k_attn_mfma<128, 2, 4>), grid_vs, dim3(256), lds, st, q, kc, vt, v_ld, M, n_keys, H, Hkv,
                               sstride, q_tiles, q_pos0, window, out, vs);
        else
            hipLaunchKernelGGL((k_attn_mfma<64, 3, 4>), grid_vs, dim3(256), lds, st, q, kc, vt, v_ld, M, n_keys, H, Hkv,
                               sstride, q_tiles, q_pos0, window, out, vs);
    } else if (hd == 128) {   // score rows longer than the LDS holds: recomputed in three passes
        hipLaunchKernelGGL((k_attn_long<128>), grid, dim3(256), 0, st, q, kc, vt, v_ld, M, n_keys, H, Hkv, q_tiles,
                           q_pos0, window, out);
    } else {
        hipLaunchKernelGGL((k_attn_long<64>), grid, dim3(256), 0, st, q, kc, vt, v_ld, M, n_keys, H, Hkv, q_tiles,
                           q_pos0, window, out);
    }
    DFX_CHECK_LAUNCH("dfx_attention");
    return DFX_OK;
}

extern "C" int dfx_attention(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M,
                             int64_t n_keys, int H, int Hkv, int hd, float * out, void * stream) {
    return dfx_attention_ex(q, kc, vt, v_ld, M, n_keys, H, Hkv, hd, out, DFX_ATTN_EXACT, stream);
}

extern "C" int dfx_attention_ex(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M,
                                int64_t n_keys, int H, int Hkv, int hd, float * out, int mode, void * stream) {
    if (mode != DFX_ATTN_SPLIT_BF16 && mode != DFX_ATTN_EXACT) {
        dfx_set_error("dfx_attention_ex: unknown mode %d", mode);
        return DFX_ERR_ARG;
    }
    if (M < 0 || n_keys <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128) || v_ld < n_keys ||
        (v_ld % 16) || M > INT32_MAX || n_keys > INT32_MAX) {
        dfx_set_error("dfx_attention: unsupported shape M=%lld keys=%lld H=%d Hkv=%d hd=%d v_ld=%lld "
                      "(v_ld must be a multiple of 16, >= keys)", (long long)M, (long long)n_keys, H, Hkv, hd,
                      (long long)v_ld);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    hipStream_t st = (hipStream_t)stream;
    if (mode == DFX_ATTN_SPLIT_BF16) {
        const int ss = attn_split_sstride(n_keys);
        const size_t lds = (size_t)ATTN_QT * ss * sizeof(float) + (hd == 64 ? 2 * 64 * 16 * sizeof(float) : 0);
        if (lds <= attn_lds_limit()) {
            const int q_tiles = (int)((M + ATTN_QT - 1) / ATTN_QT);
            const dim3 grid((unsigned)(8 * ((H + 7) / 8) * q_tiles));
            if (hd == 128)
                hipLaunchKernelGGL((k_attn_split<128>), grid, dim3(256), lds, st, q, kc, vt, v_ld, (int)M,
                                   (int)n_keys, H, Hkv, ss, q_tiles, out);
            else
                hipLaunchKernelGGL((k_attn_split<64>), grid, dim3(256), lds, st, q, kc, vt, v_ld, (int)M,
                                   (int)n_keys, H, Hkv, ss, q_tiles, out);
            DFX_CHECK_LAUNCH("dfx_attention");
            return DFX_OK;
        }
        // longer score rows: the exact forms below
    }
    return attn_exact(q, kc, vt, v_ld, (int)M, (int)n_keys, H, Hkv, hd, -1, 0, out, st);
}

extern "C" int dfx_attention_causal(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M,
                                    int64_t n_keys, int H, int Hkv, int hd, int64_t q_pos0, int window, float * out,
                                    void * stream) {
    if (M < 0 || n_keys <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128) || v_ld < n_keys ||
        (v_ld % 16) || M > INT32_MAX || n_keys > INT32_MAX || q_pos0 < 0 || q_pos0 + M > n_keys || window < 0) {
        dfx_set_error("dfx_attention_causal: unsupported shape M=%lld keys=%lld H=%d Hkv=%d hd=%d v_ld=%lld "
                      "q_pos0=%lld window=%d (queries must lie within the keys)", (long long)M, (long long)n_keys, H,
                      Hkv, hd, (long long)v_ld, (long long)q_pos0, window);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    return attn_exact(q, kc, vt, v_ld, (int)M, (int)n_keys, H, Hkv, hd, (int)q_pos0, window, out,
                      (hipStream_t)stream);
}
