// k_sampler.hip — per-row vocab statistics and remask selection.
//
// Row statistics restate the reference's per-masked-position scan
// (src/diffuse-sampler.cpp:34-57 compute_entropy, 241-252 top-1/top-2) as one
// workgroup reduction over a logits row, in a single read of the row:
//   argmax (strict >, lowest index on ties), top-2 (exact), and
//   S = sum of e = exp(x - max) and T = sum of e * (x - max), each thread keeping its sums
//   relative to its own running maximum m (when m grows to m', S and T are rescaled by
//   r = exp(m - m'): S' = r S, T' = r (T + (m - m') S)) until the row maximum is known;
//   entropy = -sum p log p = log S - T / S  (p = e / S, log p = (x - max) - log S).
// The reference drops terms with p <= 1e-10 (at most V * 2.3e-9 in all, far less for any
// real row) and adds 126464 float terms one after another, whose rounding walk is ~1e-5
// relative; here exp is the transcendental unit's 2^(x log2 e) (about 1 ulp), per-thread
// sums are float (T in base-2 units, one fma per element) and the sums across threads double.
#include "dfx_device.h"

#include <algorithm>

#define RS_THREADS 1024
#define RS_UNROLL 2

struct top2_t { float best; int idx; float second; };

__device__ __forceinline__ top2_t top2_merge(top2_t a, top2_t b) {
    // second = max over every element except the argmax
    if (b.best > a.best || (b.best == a.best && b.idx < a.idx)) {
        top2_t r = {b.best, b.idx, fmaxf(b.second, a.best)};
        return r;
    }
    top2_t r = {a.best, a.idx, fmaxf(a.second, b.best)};
    return r;
}

__device__ __forceinline__ top2_t top2_shfl(top2_t v, int off) {
    top2_t o;
    o.best = __shfl_xor(v.best, off, WAVE);
    o.idx = __shfl_xor(v.idx, off, WAVE);
    o.second = __shfl_xor(v.second, off, WAVE);
    return o;
}

#define LOG2E_F 1.44269504088896341f
#define LN2_D 0.69314718055994530942
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * LOG2E_F); }

// running top-2 of one element (elements arrive in increasing index order per thread)
__device__ __forceinline__ void top2_push(top2_t & t, float e, int i) {
    if (e > t.best) { t.second = fmaxf(t.second, t.best); t.best = e; t.idx = i; }
    else t.second = fmaxf(t.second, e);
}

__global__ void __launch_bounds__(RS_THREADS) k_row_stats(const float * __restrict__ logits, int64_t ld,
                                                          const int32_t * __restrict__ rows, int V,
                                                          dfx_row_stat * __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ top2_t red_t[RS_THREADS / 64];
    __shared__ double red_d[RS_THREADS / 64], red_d2[RS_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nw = RS_THREADS / 64;
    const float * x = logits + (int64_t)rows[blockIdx.x] * ld;
    const bool vec = ((V & 3) == 0) && ((((uintptr_t)x) & 15) == 0);

    // top-2, and S / T relative to this thread's running maximum m
    top2_t t = {-INFINITY, 0x7fffffff, -INFINITY};
    // T is kept in base-2 units while the row is scanned (tm = sum p * d2 with d2 = (x - m) log2 e
    // formed by one fma), and converted to natural units once at the end.
    float m = -INFINITY, m2 = -INFINITY, s = 0.0f, tm = 0.0f;   // m2 = m log2 e
    // one element e (at most the running m) into S and T; d2 is clamped where exp2(d2) is
    // already 0 in float, so that a -inf logit adds 0 * (-370), not 0 * -inf
    auto add = [&](float e) __attribute__((always_inline)) {
        const float d2 = fmaxf(fmaf(e, LOG2E_F, -m2), -370.0f);
        const float p = __builtin_amdgcn_exp2f(d2);
        s = s + p;
        tm = fmaf(p, d2, tm);
    };
    // raise the running maximum to m4 >= m, rescaling S and T
    auto raise = [&](float m4) __attribute__((always_inline)) {
        const float m42 = m4 * LOG2E_F;
        if (m == -INFINITY) {
            s = 0.0f;
            tm = 0.0f;
        } else {
            const float d2 = m2 - m42;
            const float r = __builtin_amdgcn_exp2f(d2);
            tm = r * fmaf(d2, s, tm);
            s = r * s;
        }
        m = m4;
        m2 = m42;
    };
    if (vec) {
        // RS_UNROLL float4 per thread and pass, the next pass's loads issued before this pass's
        // elements are used; clamped addresses (loads past the row's end re-read its last
        // float4, and such elements are skipped)
        constexpr int STEP = 4 * RS_UNROLL * RS_THREADS;
        float4 v[RS_UNROLL], nx[RS_UNROLL];
#pragma unroll
        for (int u = 0; u < RS_UNROLL; u++) v[u] = *(const float4 *)(x + min(4 * tid + 4 * u * RS_THREADS, V - 4));
        for (int i0 = 4 * tid; i0 < V; i0 += STEP) {
#pragma unroll
            for (int u = 0; u < RS_UNROLL; u++)
                nx[u] = *(const float4 *)(x + min(i0 + STEP + 4 * u * RS_THREADS, V - 4));
#pragma unroll
            for (int u = 0; u < RS_UNROLL; u++) {
                const int i = i0 + 4 * u * RS_THREADS;
                if (i >= V) continue;
                const float g = fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w));
                // elements <= the running second change neither the best nor the second
                if (g > t.second) {
                    top2_push(t, v[u].x, i);
                    top2_push(t, v[u].y, i + 1);
                    top2_push(t, v[u].z, i + 2);
                    top2_push(t, v[u].w, i + 3);
                }
                if (g > m) raise(g);
                if (m != -INFINITY) {
                    add(v[u].x);
                    add(v[u].y);
                    add(v[u].z);
                    add(v[u].w);
                }
            }
#pragma unroll
            for (int u = 0; u < RS_UNROLL; u++) v[u] = nx[u];
        }
    } else {
        for (int i = tid; i < V; i += RS_THREADS) {
            const float e = x[i];
            top2_push(t, e, i);
            if (e > m) raise(e);
            if (m != -INFINITY) add(e);
        }
    }
    for (int off = 32; off > 0; off >>= 1) t = top2_merge(t, top2_shfl(t, off));
    if (lane == 0) red_t[wv] = t;
    __syncthreads();
    t = red_t[0];
    for (int w = 1; w < nw; w++) t = top2_merge(t, red_t[w]);
    // no element above -inf: the reference's argmax stays at its start, index 0
    if (t.idx == 0x7fffffff) t.idx = 0;
    const float mx = t.best;
    // The reference's running second starts at -1e30 and is replaced by the old best
    // whenever a new best appears, so the sentinel survives only if index 0 is the argmax.
    float second = t.second;
    if (t.idx == 0) second = fmaxf(second, -1e30f);

    // this thread's S and T relative to the row maximum, summed over the row in double
    double sd = 0.0, td = 0.0;
    if (m != -INFINITY) {
        const double d = (double)m - (double)mx, r = (double)exp_fast(m - mx);
        sd = r * (double)s;
        td = r * ((double)tm * LN2_D + d * (double)s);   // tm back to natural units
    }
    sd = wave_sum_d(sd);
    td = wave_sum_d(td);
    if (lane == 0) {
        red_d[wv] = sd;
        red_d2[wv] = td;
    }
    __syncthreads();
    if (tid == 0) {
        double S = 0.0, T = 0.0;
        for (int w = 0; w < nw; w++) {
            S += red_d[w];
            T += red_d2[w];
        }
        dfx_row_stat r;
        r.token = t.idx;
        r.best = mx;
        r.second = second;
        r.entropy = S > 0.0 ? (float)(log(S) - T / S) : 0.0f;
        out[blockIdx.x] = r;
    }
}

extern "C" int dfx_row_stats(const float * logits, int64_t ld, const int32_t * rows, int64_t n_rows, int64_t V,
                             dfx_row_stat * out, void * stream) {
    if (n_rows < 0 || V <= 0 || V > INT32_MAX || ld < V) {
        dfx_set_error("dfx_row_stats: bad shape rows=%lld V=%lld ld=%lld", (long long)n_rows, (long long)V,
                      (long long)ld);
        return DFX_ERR_ARG;
    }
    if (n_rows == 0) return DFX_OK;
    hipLaunchKernelGGL(k_row_stats, dim3((unsigned)n_rows), dim3(RS_THREADS), 0, (hipStream_t)stream, logits, ld,
                       rows, (int)V, out);
    DFX_CHECK_LAUNCH("dfx_row_stats");
    return DFX_OK;
}

// Candidate records for the masked positions (src/diffuse-sampler.cpp:253-255):
// confidence = top-1 logit, or top1 - top2 for TOPK_MARGIN.
__global__ void k_make_candidates(const dfx_row_stat * __restrict__ st, const int32_t * __restrict__ pos, int n,
                                  int margin, dfx_candidate * __restrict__ out) {
#pragma clang fp contract(off)
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const dfx_row_stat s = st[i];
    dfx_candidate c;
    c.pos = pos[i];
    c.token = s.token;
    c.confidence = margin ? (s.best - s.second) : s.best;
    c.entropy = s.entropy;
    out[i] = c;
}

extern "C" int dfx_make_candidates(const dfx_row_stat * stats, const int32_t * pos, int n, int margin,
                                   dfx_candidate * out, void * stream) {
    if (n < 0 || (n > 0 && (!stats || !pos || !out))) {
        dfx_set_error("dfx_make_candidates: bad arguments (n=%d)", n);
        return DFX_ERR_ARG;
    }
    if (n == 0) return DFX_OK;
    hipLaunchKernelGGL(k_make_candidates, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, stats,
                       pos, n, margin, out);
    DFX_CHECK_LAUNCH("dfx_make_candidates");
    return DFX_OK;
}

// ---------------------------------------------------------------------------
// Selection: bitonic sort of candidate indices by the policy key in one workgroup.
// ---------------------------------------------------------------------------
#define SEL_MAX 2048
#define SEL_THREADS 1024

// true if candidate a goes before candidate b
__device__ __forceinline__ bool sel_before(const dfx_candidate & a, const dfx_candidate & b, bool by_entropy) {
    if (by_entropy) {
        if (a.entropy != b.entropy) return a.entropy < b.entropy;
    } else {
        if (a.confidence != b.confidence) return a.confidence > b.confidence;
    }
    return a.pos < b.pos;
}

__global__ void __launch_bounds__(SEL_THREADS) k_select(const dfx_candidate * __restrict__ cand, int n, int P,
                                                        int by_entropy, float tau, int n_sched,
                                                        int32_t * __restrict__ order, int32_t * __restrict__ n_unmask) {
    __shared__ dfx_candidate c[SEL_MAX];
    __shared__ int32_t ix[SEL_MAX];
    __shared__ int n_easy;
    const int tid = threadIdx.x;
    if (tid == 0) n_easy = 0;
    for (int i = tid; i < P; i += SEL_THREADS) {
        if (i < n) c[i] = cand[i];
        ix[i] = i;
    }
    __syncthreads();
    // padding indices (>= n) always sort last
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < P; i += SEL_THREADS) {
                const int l = i ^ j;
                if (l > i) {
                    const int a = ix[i], b = ix[l];
                    bool b_first;
                    if (a >= n) b_first = b < n || b < a;
                    else if (b >= n) b_first = false;
                    else b_first = sel_before(c[b], c[a], by_entropy != 0);
                    const bool up = (i & k) == 0;
                    if (up ? b_first : !b_first) { ix[i] = b; ix[l] = a; }
                }
            }
            __syncthreads();
        }
    }
    int cnt = 0;
    for (int i = tid; i < n; i += SEL_THREADS) {
        order[i] = ix[i];
        if (by_entropy && c[i].entropy < tau) cnt++;
    }
    if (cnt) atomicAdd(&n_easy, cnt);
    __syncthreads();
    if (tid == 0) {
        int u = by_entropy ? max(n_sched, n_easy) : n_sched;
        *n_unmask = min(u, n);
    }
}

// Candidates from the row statistics (as k_make_candidates) and their selection (as k_select)
// in one workgroup, for at most SEL_FUSED_MAX candidates: candidate i goes to place
// rank(i) = #{j : key j before key i} (sel_key below: the policy key, then the position), a
// strict total order, so this is k_select's order; the candidates are also written out (the
// unmask step reads them).
#define SEL_FUSED_MAX 1024
__device__ __forceinline__ uint64_t sel_key(const dfx_candidate & c, bool by_entropy);
__global__ void __launch_bounds__(SEL_FUSED_MAX) k_select_stats(const dfx_row_stat * __restrict__ st,
                                                                const int32_t * __restrict__ pos, int n, int margin,
                                                                int by_entropy, float tau, int n_sched,
                                                                dfx_candidate * __restrict__ cand,
                                                                int32_t * __restrict__ order,
                                                                int32_t * __restrict__ n_unmask) {
#pragma clang fp contract(off)
    __shared__ uint64_t key[SEL_FUSED_MAX];
    __shared__ int n_easy;
    const int tid = threadIdx.x;
    if (tid == 0) n_easy = 0;
    __syncthreads();
    uint64_t me = 0;
    if (tid < n) {
        const dfx_row_stat s = st[tid];
        dfx_candidate c;
        c.pos = pos[tid];
        c.token = s.token;
        c.confidence = margin ? (s.best - s.second) : s.best;
        c.entropy = s.entropy;
        cand[tid] = c;
        me = sel_key(c, by_entropy != 0);
        key[tid] = me;
        if (by_entropy && c.entropy < tau) atomicAdd(&n_easy, 1);
    }
    __syncthreads();
    if (tid < n) {
        int rank = 0;
        // equal keys (only if a caller repeats a position) keep the input order
        for (int j = 0; j < n; j++) rank += (key[j] < me || (key[j] == me && j < tid)) ? 1 : 0;
        order[rank] = tid;
    }
    if (tid == 0) *n_unmask = min(by_entropy ? max(n_sched, n_easy) : n_sched, n);
}

// More candidates than one workgroup sorts: the key order (ties by position) is a strict
// total order, so candidate i goes to place rank(i) = #{j : j before i}.  Each thread ranks
// one candidate against all of them, read in 1024-candidate tiles through LDS.
#define RANK_TILE 1024
// (key, position) as one unsigned 64-bit value whose order is sel_before's: the key
// (entropy, or -confidence) mapped to an unsigned int with the float order (-0 as +0,
// NaN last), then the position.  Unlike float comparisons this is a total order for every
// input, so the ranks are always a permutation.
__device__ __forceinline__ uint64_t sel_key(const dfx_candidate & c, bool by_entropy) {
    const float k = by_entropy ? c.entropy : -c.confidence;
    uint32_t u = __float_as_uint(k == 0.0f ? 0.0f : k);
    u = k != k ? 0xFFFFFFFFu : (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)c.pos;
}
__global__ void __launch_bounds__(256) k_select_rank(const dfx_candidate * __restrict__ cand, int n, int by_entropy,
                                                     int32_t * __restrict__ order) {
    __shared__ uint64_t t[RANK_TILE];
    const int i = blockIdx.x * 256 + threadIdx.x;
    const uint64_t me = sel_key(cand[min(i, n - 1)], by_entropy != 0);
    int rank = 0;
    for (int j0 = 0; j0 < n; j0 += RANK_TILE) {
        const int nt = min(RANK_TILE, n - j0);
        __syncthreads();
        for (int j = threadIdx.x; j < nt; j += 256) t[j] = sel_key(cand[j0 + j], by_entropy != 0);
        __syncthreads();
        // equal keys (only if a caller repeats a position) keep the input order
        for (int j = 0; j < nt; j++) rank += (t[j] < me || (t[j] == me && j0 + j < i)) ? 1 : 0;
    }
    if (i < n) order[rank] = i;
}

// n_unmask after k_select_rank: entropy_exit unmasks max(n_sched, the number of leading
// entries of the order with entropy < tau), the others n_sched; capped at n.
__global__ void __launch_bounds__(1024) k_select_count(const dfx_candidate * __restrict__ cand, int n, int by_entropy,
                                                       float tau, int n_sched, const int32_t * __restrict__ order,
                                                       int32_t * __restrict__ n_unmask) {
    __shared__ int first_hard;
    if (threadIdx.x == 0) first_hard = n;
    __syncthreads();
    if (by_entropy)
        for (int r = threadIdx.x; r < n; r += 1024)
            if (!(cand[order[r]].entropy < tau)) atomicMin(&first_hard, r);
    __syncthreads();
    if (threadIdx.x == 0) *n_unmask = min(by_entropy ? max(n_sched, first_hard) : n_sched, n);
}

extern "C" int dfx_select_from_stats(const dfx_row_stat * stats, const int32_t * pos, int n, int remasking,
                                     float tau, int n_sched, dfx_candidate * cand, int32_t * order,
                                     int32_t * n_unmask, void * stream) {
    if (n < 0 || remasking < 0 || remasking > 4 || remasking == 1 ||
        (n > 0 && (!stats || !pos || !cand || !order || !n_unmask))) {
        dfx_set_error("dfx_select_from_stats: unsupported n=%d or remasking=%d", n, remasking);
        return DFX_ERR_ARG;
    }
    const int margin = remasking == 4 ? 1 : 0;
    if (n > SEL_FUSED_MAX) {
        const int rc = dfx_make_candidates(stats, pos, n, margin, cand, stream);
        if (rc != DFX_OK) return rc;
        return dfx_select(cand, n, remasking, tau, n_sched, order, n_unmask, stream);
    }
    if (n == 0) {
        hipLaunchKernelGGL(k_select_stats, dim3(1), dim3(64), 0, (hipStream_t)stream, stats, pos, 0, margin,
                           remasking == 2 ? 1 : 0, tau, n_sched, cand, order, n_unmask);
    } else {
        hipLaunchKernelGGL(k_select_stats, dim3(1), dim3((unsigned)((n + 63) / 64 * 64)), 0, (hipStream_t)stream,
                           stats, pos, n, margin, remasking == 2 ? 1 : 0, tau, n_sched, cand, order, n_unmask);
    }
    DFX_CHECK_LAUNCH("dfx_select_from_stats");
    return DFX_OK;
}

extern "C" int dfx_select(const dfx_candidate * cand, int n, int remasking, float tau, int n_sched, int32_t * order,
                          int32_t * n_unmask, void * stream) {
    // remasking ids: include/diffuse.h:37-43 (LOW_CONFIDENCE, RANDOM, ENTROPY_EXIT, MASKGIT_PLUS, TOPK_MARGIN)
    if (n < 0 || remasking < 0 || remasking > 4 || remasking == 1) {
        dfx_set_error("dfx_select: unsupported n=%d or remasking=%d", n, remasking);
        return DFX_ERR_ARG;
    }
    if (n > SEL_MAX) {
        const int by_ent = remasking == 2 ? 1 : 0;
        hipLaunchKernelGGL(k_select_rank, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, cand, n,
                           by_ent, order);
        DFX_CHECK_LAUNCH("dfx_select rank");
        hipLaunchKernelGGL(k_select_count, dim3(1), dim3(1024), 0, (hipStream_t)stream, cand, n, by_ent, tau, n_sched,
                           order, n_unmask);
        DFX_CHECK_LAUNCH("dfx_select count");
        return DFX_OK;
    }
    int P = 1;
    while (P < n) P <<= 1;
    hipLaunchKernelGGL(k_select, dim3(1), dim3(SEL_THREADS), 0, (hipStream_t)stream, cand, n, P, remasking == 2 ? 1 : 0,
                       tau, n_sched, order, n_unmask);
    DFX_CHECK_LAUNCH("dfx_select");
    return DFX_OK;
}

// ---------------------------------------------------------------------------
// Autoregressive decoding (src/ar-sampler.cpp, src/ar-graph.cpp)
// ---------------------------------------------------------------------------
// Greedy sample_token (src/ar-sampler.cpp:99-117) on one logits row, in place:
// the repetition penalty over the recent tokens (src/ar-sampler.cpp:83-97; a token
// listed k times is penalised k times, in any order: each application maps x to x/p
// when x > 0 and to x*p otherwise, so only the count matters), then the first index
// of the maximum (strict >, from index 0).  A NaN in row[0], or a row with no value
// above -inf, gives token 0, as the reference's scan does.
// The decode state st lives on the device: [0] token of the next pass, [1] its
// position, [2] number of recent tokens n, [3] ring start, [4..4+R) ring of the last
// R (= repeat_last_n) tokens.  The chosen token becomes st[0], the position advances,
// the token enters the ring (the oldest leaves once R are held), and it is also
// written to tok_out.
#define GREEDY_RING_MAX 4096   // recent tokens the device sampler holds (longer windows: host sampler)
__global__ void __launch_bounds__(RS_THREADS) k_ar_greedy(float * __restrict__ row, int V, int32_t * __restrict__ st,
                                                          int R, float penalty, int32_t * __restrict__ tok_out) {
#pragma clang fp contract(off)
    __shared__ float red_v[RS_THREADS / 64];
    __shared__ int red_i[RS_THREADS / 64];
    __shared__ int ring[GREEDY_RING_MAX];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (penalty > 1.0f && R > 0) {
        // the ring's tokens in LDS; the first occurrence of each token applies the penalty
        // as many times as the token occurs, in one read-modify-write of the row
        const int n = st[2], start = st[3];
        for (int j = tid; j < n; j += RS_THREADS) ring[j] = st[4 + (start + j) % R];
        __syncthreads();
        for (int j = tid; j < n; j += RS_THREADS) {
            const int t = ring[j];
            bool first = true;
            int count = 0;
            for (int k = 0; k < n; k++) {
                first = first && !(k < j && ring[k] == t);
                count += ring[k] == t;
            }
            if (first && t >= 0 && t < V) {
                float v = row[t];
                for (int c = 0; c < count; c++) v = v > 0.0f ? v / penalty : v * penalty;
                row[t] = v;
            }
        }
    }
    __syncthreads();   // the penalised values are visible to the whole workgroup
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // eight loads in flight per thread; increasing i per thread, so the first maximum stays
    constexpr int U = 8;
    for (int i0 = tid; i0 < V; i0 += U * RS_THREADS) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * RS_THREADS;
            v[u] = i < V ? row[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v[u] > bv) { bv = v[u]; bi = i0 + u * RS_THREADS; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, WAVE);
        const int oi = __shfl_xor(bi, o, WAVE);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { red_v[wv] = bv; red_i[wv] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < RS_THREADS / 64; w++)
            if (red_v[w] > bv || (red_v[w] == bv && red_i[w] < bi)) { bv = red_v[w]; bi = red_i[w]; }
        const float r0 = row[0];
        const int tok = (r0 != r0 || bi == 0x7fffffff) ? 0 : bi;
        st[0] = tok;
        st[1] = st[1] + 1;
        if (R > 0) {
            const int n = st[2], start = st[3];
            if (n < R) {
                st[4 + (start + n) % R] = tok;
                st[2] = n + 1;
            } else {
                st[4 + start] = tok;
                st[3] = (start + 1) % R;
            }
        }
        tok_out[0] = tok;
    }
}

extern "C" int dfx_ar_greedy(float * row, int64_t V, int32_t * state, int repeat_last_n, float repeat_penalty,
                             int32_t * token_out, void * stream) {
    if (!row || !state || !token_out || V <= 0 || V > INT32_MAX || repeat_last_n > GREEDY_RING_MAX) {
        dfx_set_error("dfx_ar_greedy: bad arguments (V=%lld, repeat_last_n=%d, at most %d)", (long long)V,
                      repeat_last_n, GREEDY_RING_MAX);
        return DFX_ERR_ARG;
    }
    hipLaunchKernelGGL(k_ar_greedy, dim3(1), dim3(RS_THREADS), 0, (hipStream_t)stream, row, (int)V, state,
                       repeat_last_n > 0 ? repeat_last_n : 0, repeat_penalty, token_out);
    DFX_CHECK_LAUNCH("dfx_ar_greedy");
    return DFX_OK;
}

// Layer impact of ar_profile_layers (src/ar-graph.cpp:219-228): for each row m,
// out[m] = sum over i of (double)(d * d), d = x[m][i] - x_in[m][i] in float, added in
// increasing i (one thread per row, so the double sum has the scalar order).  The caller
// adds the rows in order in double and rounds to float, as ggml_sum does.
__global__ void __launch_bounds__(64) k_layer_impact(const float * __restrict__ x, const float * __restrict__ x_in,
                                                     int M, int64_t d, double * __restrict__ out) {
#pragma clang fp contract(off)
    const int m = blockIdx.x * 64 + threadIdx.x;
    if (m >= M) return;
    const float * a = x + (int64_t)m * d;
    const float * b = x_in + (int64_t)m * d;
    double s = 0.0;
    for (int64_t i = 0; i < d; i++) {
        const float df = a[i] - b[i];
        s += (double)(df * df);
    }
    out[m] = s;
}

extern "C" int dfx_layer_impact(const float * x, const float * x_in, int64_t M, int64_t d, double * out,
                                void * stream) {
    if (M < 0 || M > INT32_MAX || d <= 0) {
        dfx_set_error("dfx_layer_impact: bad shape M=%lld d=%lld", (long long)M, (long long)d);
        return DFX_ERR_ARG;
    }
    if (M == 0) return DFX_OK;
    hipLaunchKernelGGL(k_layer_impact, dim3((unsigned)((M + 63) / 64)), dim3(64), 0, (hipStream_t)stream, x, x_in,
                       (int)M, d, out);
    DFX_CHECK_LAUNCH("dfx_layer_impact");
    return DFX_OK;
}

// ---------------------------------------------------------------------------
// Device-resident denoising step bookkeeping
// ---------------------------------------------------------------------------
// The sequence state lives on the device: seq[N] (token ids), prev[N] (seq as it was
// right after the last forward, src/diffuse-sampler.cpp:154, 171, 194), masked[N] (0 / 1)
// and lastc[N] (step at which a change was last seen, -1 never).

// Exclusive prefix of a per-thread flag over a workgroup of SCAN_T threads, and the total.
#define SCAN_T 1024
__device__ __forceinline__ int block_scan(bool flag, int * red, int & total) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const unsigned long long b = __ballot(flag);
    const int in_wave = __popcll(b & ((1ull << lane) - 1ull));
    if (lane == 0) red[wv] = __popcll(b);
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < SCAN_T / 64; w++) {
        const int c = red[w];
        if (w < wv) before += c;
        total += c;
    }
    __syncthreads();
    return before + in_wave;
}

// compute_active_set (src/diffuse-cache.h:79-116) and the row lists of one step.
//   active: full step, or changed (seq != prev, which also records lastc = step), still
//   masked, or changed within `keep` steps; a cached step whose active set is empty or
//   everything becomes full.
//   pass rows a = 0..M-1 in position order: tok[a] = seq[act[a]], act[a] = position;
//   head rows: pass rows whose logits the sampler reads (masked positions, or their left
//   neighbours when shift; every pass row when head_all), hrows[k] = pass row,
//   hmap[k] = position;
//   sampler rows: every masked position i in order, srows[k] = i (or max(i-1, 0) when
//   shift), spos[k] = i.
// counts = {M, n_head, n_cand, full}.  One workgroup.
__global__ void __launch_bounds__(SCAN_T) k_step_prepare(int N, int step, int full, int keep, int shift, int head_all,
                                                         const int32_t * __restrict__ seq,
                                                         const int32_t * __restrict__ prev,
                                                         const int32_t * __restrict__ masked, int32_t * lastc,
                                                         int32_t * tok, int32_t * act, int32_t * hrows, int32_t * hmap,
                                                         int32_t * srows, int32_t * spos, int32_t * counts) {
    __shared__ int red[SCAN_T / 64];
    const int tid = threadIdx.x;
    int M = 0;
    if (!full) {
        for (int t0 = 0; t0 < N; t0 += SCAN_T) {
            const int i = t0 + tid;
            bool on = false;
            if (i < N) {
                const bool changed = seq[i] != prev[i];
                int lc = lastc[i];
                if (changed) {
                    lc = step;
                    lastc[i] = step;
                }
                const bool recent = keep > 0 && lc >= 0 && step - lc <= keep;
                on = changed || masked[i] != 0 || recent;
            }
            int tot;
            const int idx = block_scan(on, red, tot);
            if (on) act[M + idx] = i;
            M += tot;
        }
        if (M >= N || M == 0) full = 1;
    }
    if (full) {
        for (int i = tid; i < N; i += SCAN_T) act[i] = i;
        M = N;
    }
    __syncthreads();
    // pass tokens and head rows (act is in position order)
    int nh = 0;
    for (int a0 = 0; a0 < M; a0 += SCAN_T) {
        const int a = a0 + tid;
        bool need = false;
        int p = 0;
        if (a < M) {
            p = act[a];
            tok[a] = seq[p];
            need = head_all || (shift ? ((p + 1 < N && masked[p + 1] != 0) || (p == 0 && masked[0] != 0))
                                      : masked[p] != 0);
        }
        int tot;
        const int idx = block_scan(need, red, tot);
        if (need) {
            hrows[nh + idx] = a;
            hmap[nh + idx] = p;
        }
        nh += tot;
    }
    // sampler rows
    int nc = 0;
    for (int t0 = 0; t0 < N; t0 += SCAN_T) {
        const int i = t0 + tid;
        const bool m = i < N && masked[i] != 0;
        int tot;
        const int idx = block_scan(m, red, tot);
        if (m) {
            srows[nc + idx] = shift ? max(i - 1, 0) : i;
            spos[nc + idx] = i;
        }
        nc += tot;
    }
    if (tid == 0) {
        counts[0] = M;
        counts[1] = nh;
        counts[2] = nc;
        counts[3] = full;
    }
}

// update_seq then unmask (src/diffuse-sampler.cpp:154, 316-323): prev = seq (when the cache
// is on), then the first n_unmask selected candidates write their token and clear their
// mask; ustep[pos] = step when given; hist[step] = n_unmask, or -1 if the selection named
// a candidate or position out of range (nothing is written for it).  One workgroup.
__global__ void __launch_bounds__(SCAN_T) k_step_unmask(int N, int use_cache, int step, int32_t * seq,
                                                        int32_t * prev, int32_t * masked,
                                                        const dfx_candidate * __restrict__ cand,
                                                        const int32_t * __restrict__ order,
                                                        const int32_t * __restrict__ n_unmask, int n_cand,
                                                        int32_t * ustep, int32_t * hist) {
    __shared__ int bad;
    const int tid = threadIdx.x;
    if (tid == 0) bad = 0;
    if (use_cache)
        for (int i = tid; i < N; i += SCAN_T) prev[i] = seq[i];
    __syncthreads();
    const int n = min(*n_unmask, n_cand);
    for (int j = tid; j < n; j += SCAN_T) {
        const int o = order[j];
        const dfx_candidate c = cand[o >= 0 && o < n_cand ? o : 0];
        if (o < 0 || o >= n_cand || c.pos < 0 || c.pos >= N) {   // never written out of range
            bad = 1;
            continue;
        }
        seq[c.pos] = c.token;
        masked[c.pos] = 0;
        if (ustep) ustep[c.pos] = step;
    }
    __syncthreads();
    if (tid == 0) hist[step] = bad ? -1 : n;   // -1: the selection named a bad candidate
}

extern "C" int dfx_step_prepare(int N, int step, int full, int keep, int shift, int head_all, const int32_t * seq,
                                const int32_t * prev, const int32_t * masked, int32_t * lastc, int32_t * tok,
                                int32_t * act, int32_t * hrows, int32_t * hmap, int32_t * srows, int32_t * spos,
                                int32_t * counts, void * stream) {
    if (N <= 0 || !seq || !prev || !masked || !lastc || !tok || !act || !hrows || !hmap || !srows || !spos || !counts) {
        dfx_set_error("dfx_step_prepare: bad arguments (N=%d)", N);
        return DFX_ERR_ARG;
    }
    hipLaunchKernelGGL(k_step_prepare, dim3(1), dim3(SCAN_T), 0, (hipStream_t)stream, N, step, full, keep, shift,
                       head_all, seq, prev, masked, lastc, tok, act, hrows, hmap, srows, spos, counts);
    DFX_CHECK_LAUNCH("dfx_step_prepare");
    return DFX_OK;
}

extern "C" int dfx_step_unmask(int N, int use_cache, int step, int32_t * seq, int32_t * prev, int32_t * masked,
                               const dfx_candidate * cand, const int32_t * order, const int32_t * n_unmask, int n_cand,
                               int32_t * ustep, int32_t * hist, void * stream) {
    if (N <= 0 || n_cand < 0 || !seq || !prev || !masked || !n_unmask || !hist || (n_cand && (!cand || !order))) {
        dfx_set_error("dfx_step_unmask: bad arguments (N=%d, n_cand=%d)", N, n_cand);
        return DFX_ERR_ARG;
    }
    hipLaunchKernelGGL(k_step_unmask, dim3(1), dim3(SCAN_T), 0, (hipStream_t)stream, N, use_cache, step, seq, prev,
                       masked, cand, order, n_unmask, n_cand, ustep, hist);
    DFX_CHECK_LAUNCH("dfx_step_unmask");
    return DFX_OK;
}
