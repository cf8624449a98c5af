// engine.cpp — forward pass and denoising loop on one gfx950 GPU.
//
// Forward (src/diffuse-graph.cpp:11-160 full, 395-593 cached): one HIP stream,
// per layer
//   rmsnorm+convert -> Q|K|V GEMM (+bias) -> RoPE + cache store -> attention over
//   the cache -> convert -> O GEMM (+residual) -> rmsnorm+convert -> gate|up GEMM
//   -> SwiGLU+convert -> down GEMM (+residual)
// then the final norm and the vocab head for the rows whose logits are read.
// The cached step runs the same sequence on the active rows only: their K/V are
// scattered into the HBM-resident cache before attention, which then reads all
// positions (src/diffuse-cache.h:124-140 update_kv + the [cached ‖ active] concat).
//
// Denoising loop (src/diffuse-sampler.cpp:60-370): host bookkeeping of seq /
// is_masked / the active set, device row statistics + selection, and only the
// per-candidate records come back to the host each step.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>

#include "engine.h"

namespace {

#define TRY(x)                         \
    do {                               \
        const int rc_ = (x);           \
        if (rc_ != DFX_OK) return rc_; \
    } while (0)

int hip_ok(hipError_t e, const char * what) {
    if (e == hipSuccess) return DFX_OK;
    dfx_set_error("%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? DFX_ERR_OOM : DFX_ERR_HIP;
}

struct dims {
    int64_t d, F, V, L, H, Hkv, hd, dkv, nqkv;
    explicit dims(const diffuse_hparams & hp) {
        d = hp.n_embd; F = hp.n_ff; V = hp.n_vocab; L = hp.n_layer; H = hp.n_head; Hkv = hp.n_head_kv;
        hd = d / H; dkv = hd * Hkv; nqkv = d + 2 * dkv;
    }
};

void drop_graphs(diffuse_context * c) {
    for (auto & g : c->graphs) (void)hipGraphExecDestroy(g.exec);
    c->graphs.clear();
}

void free_buffers(diffuse_context * c) {
    drop_graphs(c);
    void * bufs[] = {c->x, c->act, c->qkv, c->qr, c->att, c->gu, c->logits, c->kc, c->vc, c->rope_tab,
                     c->d_ints, c->ws, c->d_stats, c->d_out, c->x_prev, c->d_imp, c->d_ar, c->d_state,
                     c->d_counts, c->d_hist, c->tile_cnt};
    for (void * p : bufs)
        if (p) (void)hipFree(p);
    if (c->h_pin) (void)hipHostFree(c->h_pin);
    if (c->h_out) (void)hipHostFree(c->h_out);
    if (c->h_row) (void)hipHostFree(c->h_row);
    if (c->h_hist) (void)hipHostFree(c->h_hist);
    c->d_state = c->d_counts = c->d_hist = c->h_hist = nullptr;
    c->steps_cap = 0;
    c->x_prev = nullptr;
    c->d_imp = nullptr;
    c->d_ar = nullptr;
    c->ar_ring = 0;
    c->h_row = nullptr;
    c->ar_past = 0;
    c->x = c->qkv = c->qr = c->att = c->gu = c->logits = c->kc = c->vc = c->rope_tab = nullptr;
    c->act = nullptr;
    c->d_ints = c->d_tok = c->d_pos = c->d_hrows = c->d_hmap = c->d_srows = c->d_spos = c->d_order = c->d_nun = nullptr;
    c->ws = c->d_out = c->h_out = nullptr;
    c->tile_cnt = nullptr;
    c->out_bytes = 0;
    c->d_stats = nullptr;
    c->d_cand = nullptr;
    c->h_pin = nullptr;
    c->cap = 0;
    c->kv_valid = 0;
}

// NEOX rope angles, as GGML's rope cache: theta_0 = p, theta_{i+1} = theta_i *
// powf(base, -2/n_dims); cos/sin by cosf/sinf (freq_scale 1, ext_factor 0,
// attn_factor 1 as passed at src/diffuse-graph.cpp:76-79).
void rope_table(int n_pos, int hd, float base, std::vector<float> & tab) {
    const int half = hd / 2;
    tab.resize((size_t)n_pos * half * 2);
    const float theta_scale = powf(base, -2.0f / (float)hd);
    for (int p = 0; p < n_pos; p++) {
        float theta = (float)p;
        for (int i = 0; i < half; i++) {
            tab[((size_t)p * half + i) * 2 + 0] = cosf(theta);
            tab[((size_t)p * half + i) * 2 + 1] = sinf(theta);
            theta *= theta_scale;
        }
    }
}

int ensure_capacity(diffuse_context * c, int N) {
    if (N <= c->cap) return DFX_OK;
    N = (N + 15) & ~15;     // the transposed value cache rows are read 4 keys at a time
    free_buffers(c);
    const dims D(c->model->hparams);
    const int64_t n = N;
    auto A = [&](void ** p, size_t bytes) { return hip_ok(hipMalloc(p, bytes ? bytes : 1), "context hipMalloc"); };
    TRY(A((void **)&c->x, n * D.d * 4));
    const int64_t kmax = std::max(D.d, D.F);
    // passes of at most 4 rows also keep an int8 plane (matrix-vector kernels)
    TRY(A((void **)&c->act, std::max({dfx_act_bytes(DFX_TYPE_Q4_K, n, kmax),
                                      dfx_act_bytes(DFX_TYPE_Q4_K, std::min<int64_t>(n, 4), kmax),
                                      dfx_act_bytes(DFX_TYPE_Q8_0, n, kmax), dfx_act_bytes(DFX_TYPE_F16, n, kmax),
                                      dfx_act_bytes(DFX_TYPE_F32, n, kmax)})));
    TRY(A((void **)&c->qkv, n * D.nqkv * 4));
    TRY(A((void **)&c->qr, n * D.d * 4));
    TRY(A((void **)&c->att, n * D.d * 4));
    TRY(A((void **)&c->gu, n * 2 * D.F * 4));
    TRY(A((void **)&c->logits, n * D.V * 4));
    TRY(A((void **)&c->kc, D.L * n * D.dkv * 4));
    TRY(A((void **)&c->vc, D.L * n * D.dkv * 4));
    TRY(A((void **)&c->rope_tab, n * D.hd * 4));
    TRY(A((void **)&c->d_ints, 6 * n * 4));
    c->d_tok = c->d_ints;
    c->d_pos = c->d_ints + n;
    c->d_hrows = c->d_ints + 2 * n;
    c->d_hmap = c->d_ints + 3 * n;
    c->d_srows = c->d_ints + 4 * n;
    c->d_spos = c->d_ints + 5 * n;
    // split-K workspace for the GEMMs with few output tiles (Q|K|V, O, down) and the chunk
    // totals of half tiles (Q|K|V, gate|up); their completion counters start (and stay) zero
    c->ws_bytes = std::max({dfx_gemm_ws_bytes(n, D.nqkv, D.d), dfx_gemm_ws_bytes(n, D.d, D.d),
                            dfx_gemm_ws_bytes(n, D.d, D.F), dfx_gemm_ws_bytes(n, 2 * D.F, D.d)});
    TRY(A(&c->ws, c->ws_bytes));
    const size_t cnt_bytes = std::max(dfx_gemm_tile_cnt_bytes(n, D.nqkv), dfx_gemm_tile_cnt_bytes(n, 2 * D.F));
    TRY(A((void **)&c->tile_cnt, cnt_bytes));
    TRY(hip_ok(hipMemsetAsync(c->tile_cnt, 0, cnt_bytes, c->stream), "counter clear"));
    TRY(A((void **)&c->d_stats, n * sizeof(dfx_row_stat)));
    TRY(A((void **)&c->d_state, 5 * n * 4));
    c->out_bytes = n * sizeof(dfx_candidate) + n * 4 + 16;
    TRY(A(&c->d_out, c->out_bytes));
    c->d_cand = (dfx_candidate *)c->d_out;
    c->d_order = (int32_t *)(c->d_cand + n);
    c->d_nun = c->d_order + n;
    TRY(hip_ok(hipHostMalloc((void **)&c->h_pin, n * 8 * 4, hipHostMallocDefault), "hipHostMalloc"));
    TRY(hip_ok(hipHostMalloc(&c->h_out, c->out_bytes, hipHostMallocDefault), "hipHostMalloc"));
    // caches start at zero like diffuse_step_cache::init (src/diffuse-cache.h:43-49)
    TRY(hip_ok(hipMemsetAsync(c->kc, 0, D.L * n * D.dkv * 4, c->stream), "memset"));
    TRY(hip_ok(hipMemsetAsync(c->vc, 0, D.L * n * D.dkv * 4, c->stream), "memset"));
    std::vector<float> tab;
    rope_table(N, (int)D.hd, c->model->hparams.rope_theta, tab);
    TRY(hip_ok(hipMemcpyAsync(c->rope_tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, c->stream),
               "rope table upload"));
    TRY(hip_ok(hipStreamSynchronize(c->stream), "rope table upload"));
    c->cap = N;
    return DFX_OK;
}

hipEvent_t take_event(diffuse_context * c) {
    if (!c->prof_pool.empty()) {
        hipEvent_t e = c->prof_pool.back();
        c->prof_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Device -> host copy on the context's stream, waited for.  The engine never touches the
// legacy stream: another host thread may be capturing its own context's stream meanwhile.
static int d2h_sync(diffuse_context * c, void * dst, const void * src, size_t bytes) {
    TRY(hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "D2H"));
    return hip_ok(hipStreamSynchronize(c->stream), "D2H");
}

// The half-tile GEMMs raise tile_cnt[1] when the two halves of a tile ran on different XCDs
// (their chunk-total handover assumes one L2; see k_q4k_w): checked after every pass that
// reads results back, so such a pass fails instead of returning possibly stale sums.
int check_tiles(diffuse_context * c) {
    if (!c->tile_cnt) return DFX_OK;
    int32_t flag = 0;
    TRY(d2h_sync(c, &flag, c->tile_cnt + 1, sizeof(flag)));
    if (flag) {
        TRY(hip_ok(hipMemsetAsync(c->tile_cnt + 1, 0, sizeof(int32_t), c->stream), "counter clear"));
        dfx_set_error("GEMM half tiles ran on different XCDs (workgroup-to-XCD mapping not round-robin): "
                      "results of this pass are invalid");
        return DFX_ERR_HIP;
    }
    return DFX_OK;
}

// Every GEMM of the forward goes through here; with profiling on, a pair of events
// brackets the launch on the context stream (read back by prof_collect).
// With n_partials, a split-K GEMM may leave its chunk sums in c->ws (see dfx_gemm_ex)
// for the next RMSNorm to add.
int gemm(diffuse_context * c, const dev_matrix & w, int64_t N, int64_t K, int64_t M, const float * bias,
         const float * res, float * y, int64_t ldy, const int32_t * ymap, bool split_ok, int * n_partials = nullptr,
         const dfx_epi * epi = nullptr) {
    void * ws = split_ok ? c->ws : nullptr;
    const size_t wsb = split_ok ? c->ws_bytes : 0;
    if (n_partials) *n_partials = 0;
    if (!c->prof || M == 0)
        return dfx_gemm_ex(w.type, w.data, N, K, c->act, M, bias, res, y, ldy, ymap, ws, wsb, c->stream, n_partials,
                           epi);
    diffuse_context::gemm_rec r;
    r.a = take_event(c);
    r.b = take_event(c);
    r.type = w.type;
    r.M = M;
    r.flops = 2.0 * (double)M * N * K;
    r.bytes = (double)dfx_device_row_bytes(w.type, K) * N + (double)M * K * 2 +
              (double)M * N * (epi && epi->kind == DFX_EPI_SWIGLU ? 2 : 4);
    if (!r.a || !r.b) return hip_ok(hipErrorOutOfMemory, "hipEventCreate");
    TRY(hip_ok(hipEventRecord(r.a, c->stream), "event"));
    TRY(dfx_gemm_ex(w.type, w.data, N, K, c->act, M, bias, res, y, ldy, ymap, ws, wsb, c->stream, n_partials, epi));
    TRY(hip_ok(hipEventRecord(r.b, c->stream), "event"));
    c->prof_pending.push_back(r);
    return DFX_OK;
}

// After a stream sync: fold the pending GEMM timings into the per-type totals.
void prof_collect(diffuse_context * c) {
    for (auto & r : c->prof_pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess && r.type >= 0 && r.type < 32)
            for (int cls : {0, r.M > 96 ? 1 : 2, r.M >= 288 ? 3 : -1}) {
                if (cls < 0) continue;
                auto & t = c->prof_tot[cls][r.type];
                t.launches++;
                t.ms += ms;
                t.flops += r.flops;
                t.bytes += r.bytes;
            }
        c->prof_pool.push_back(r.a);
        c->prof_pool.push_back(r.b);
    }
    c->prof_pending.clear();
}

// GEMMs of a projection group into out[M][g.n_out]; input rows already in x.
// RMSNorm of x + conversion, then the group's GEMM(s).  `pending` split-K partial sums of
// the GEMM that produced x (left in c->ws) are added to x by the first RMSNorm.
int run_group(diffuse_context * c, const proj_group & g, const float * norm, int64_t M, int64_t K, float * out,
              int & pending, const dfx_epi * rope = nullptr) {
    const float eps = c->model->hparams.rms_norm_eps;
    auto norm_convert = [&](int type) -> int {
        if (pending == 0) return dfx_rmsnorm_convert_ex(type, c->x, nullptr, norm, M, K, eps, c->act, c->stream);
        const int np = pending;
        pending = 0;
        return dfx_rmsnorm_convert_add(type, c->x, nullptr, (const float *)c->ws, np, M, norm, M, K, eps, c->act,
                                       c->stream);
    };
    if (g.swiglu) {   // out[M][n_out / 2] = silu(gate) * up
        TRY(norm_convert(g.all.type));
        dfx_epi e{};
        e.kind = DFX_EPI_SWIGLU;
        e.tile_cnt = c->tile_cnt;
        return gemm(c, g.all, g.n_out, K, M, nullptr, nullptr, out, g.n_out / 2, nullptr, true, nullptr, &e);
    }
    if (rope) {       // Q|K|V rotated and stored by the GEMM's epilogue (rows permuted at load)
        TRY(norm_convert(g.all.type));
        return gemm(c, g.all, g.n_out, K, M, g.bias, nullptr, nullptr, g.n_out, nullptr, true, nullptr, rope);
    }
    if (g.fused) {
        TRY(norm_convert(g.all.type));
        return gemm(c, g.all, g.n_out, K, M, g.bias, nullptr, out, g.n_out, nullptr, true);
    }
    for (size_t i = 0; i < g.parts.size(); i++) {
        const dev_matrix & p = g.parts[i];
        TRY(norm_convert(p.type));
        TRY(gemm(c, p, p.rows, K, M, g.bias ? g.bias + g.col_off[i] : nullptr, nullptr, out + g.col_off[i], g.n_out,
                 nullptr, true));
    }
    return DFX_OK;
}

// Enqueue the layers of one forward over the M rows in d_tok/d_pos, attending over keys
// 0..n_keys-1 of the cache.  o: the autoregressive graph's options (causal mask, skipped
// layers, impact profile).  pending: split-K partial sums of the last down projection still
// to be added to x (by the head's RMSNorm).
int forward_layers(diffuse_context * c, int M, int n_keys, const pass_opts & o, int & pending) {
    const diffuse_model & m = *c->model;
    const dims D(m.hparams);
    const int32_t * tok = o.tok ? o.tok : c->d_tok;
    const int32_t * pos = o.pos ? o.pos : c->d_pos;
    TRY(dfx_embed(m.tok_embd.type, m.tok_embd.data, D.d, tok, M, c->x, c->stream));
    // split-K partial sums of the last O / down projection, still to be added to x (by
    // the RMSNorm that reads x next); profiling needs x whole after every layer
    pending = 0;
    int * defer = o.impact_rows ? nullptr : &pending;
    for (int64_t il = 0; il < D.L; il++) {
        if (o.skip && o.skip[il]) continue;   // src/ar-graph.cpp:98-102
        const dev_layer & L = m.layers[il];
        float * kc = c->kc + il * (int64_t)c->cap * D.dkv;
        float * vc = c->vc + il * (int64_t)c->cap * D.dkv;
        if (o.impact_rows)
            TRY(hip_ok(hipMemcpyAsync(c->x_prev, c->x, (size_t)M * D.d * 4, hipMemcpyDeviceToDevice, c->stream),
                       "layer input copy"));
        if (L.qkv.rope) {
            dfx_epi e{};
            e.kind = DFX_EPI_ROPE;
            e.H = (int)D.H;
            e.Hkv = (int)D.Hkv;
            e.hd = (int)D.hd;
            e.pos = pos;
            e.tab = c->rope_tab;
            e.q_out = c->qr;
            e.kc = kc;
            e.vt = vc;
            e.v_ld = c->cap;
            e.tile_cnt = c->tile_cnt;
            TRY(run_group(c, L.qkv, L.attn_norm, M, D.d, nullptr, pending, &e));
        } else {
            TRY(run_group(c, L.qkv, L.attn_norm, M, D.d, c->qkv, pending));
            TRY(dfx_rope_store(c->qkv, pos, M, (int)D.H, (int)D.Hkv, (int)D.hd, c->rope_tab, c->qr, kc, vc, c->cap,
                               c->stream));
        }
        if (o.q_pos0 >= 0)
            TRY(dfx_attention_causal(c->qr, kc, vc, c->cap, M, n_keys, (int)D.H, (int)D.Hkv, (int)D.hd, o.q_pos0,
                                     o.window, c->att, c->stream));
        else
            TRY(dfx_attention_ex(c->qr, kc, vc, c->cap, M, n_keys, (int)D.H, (int)D.Hkv, (int)D.hd, c->att,
                                 c->attn_mode, c->stream));
        TRY(dfx_act_convert(L.o.type, c->att, M, D.d, c->act, c->stream));
        TRY(gemm(c, L.o, D.d, D.d, M, nullptr, c->x, c->x, D.d, nullptr, true, defer));
        TRY(run_group(c, L.gu, L.ffn_norm, M, D.d, c->gu, pending));
        if (L.gu.swiglu)
            TRY(dfx_act_convert(L.down.type, c->gu, M, D.F, c->act, c->stream));
        else
            TRY(dfx_swiglu_convert(L.down.type, c->gu, M, D.F, c->act, c->stream));
        TRY(gemm(c, L.down, D.d, D.F, M, nullptr, c->x, c->x, D.d, nullptr, true, defer));
        if (o.impact_rows) TRY(dfx_layer_impact(c->x, c->x_prev, M, D.d, o.impact_rows + il * M, c->stream));
    }
    return DFX_OK;
}

// Final norm + vocab head for the n_head pass rows hrows[] (of M), logits to rows hmap[].
int forward_head(diffuse_context * c, int M, int n_head, const int32_t * hrows, const int32_t * hmap, int pending) {
    if (n_head <= 0) return DFX_OK;
    const diffuse_model & m = *c->model;
    const dims D(m.hparams);
    const float eps = m.hparams.rms_norm_eps;
    // rows without logits never need the last layer's x
    if (pending)
        TRY(dfx_rmsnorm_convert_add(m.output.type, c->x, hrows, (const float *)c->ws, pending, M, m.output_norm,
                                    n_head, D.d, eps, c->act, c->stream));
    else
        TRY(dfx_rmsnorm_convert_ex(m.output.type, c->x, hrows, m.output_norm, n_head, D.d, eps, c->act, c->stream));
    return gemm(c, m.output, D.V, D.d, n_head, nullptr, nullptr, c->logits, D.V, hmap, false);
}

// One whole forward: layers, then logits for the n_head rows d_hrows go to logits[d_hmap].
int forward_pass(diffuse_context * c, int M, int n_keys, int n_head, const pass_opts & o = pass_opts()) {
    int pending = 0;
    TRY(forward_layers(c, M, n_keys, o, pending));
    return forward_head(c, M, n_head, o.hrows ? o.hrows : c->d_hrows, o.hmap ? o.hmap : c->d_hmap, pending);
}

int upload_i32(diffuse_context * c, int32_t * dst, const int32_t * src, int n, int slot) {
    if (n <= 0) return DFX_OK;
    int32_t * stage = c->h_pin + (size_t)slot * c->cap;
    memcpy(stage, src, (size_t)n * 4);
    return hip_ok(hipMemcpyAsync(dst, stage, (size_t)n * 4, hipMemcpyHostToDevice, c->stream), "H2D");
}

// Stage n values into slot `slot` of h_pin; upload_slots sends slots 0..n_slots-1 to d_ints.
void stage_i32(diffuse_context * c, const int32_t * src, int n, int slot) {
    if (n > 0) memcpy(c->h_pin + (size_t)slot * c->cap, src, (size_t)n * 4);
}
int upload_slots(diffuse_context * c, int n_slots) {
    return hip_ok(hipMemcpyAsync(c->d_ints, c->h_pin, (size_t)n_slots * c->cap * 4, hipMemcpyHostToDevice, c->stream),
                  "H2D");
}

// src/diffuse-sampler.cpp:12-31 (t * M_PI is a double product narrowed for cosf)
int tokens_to_unmask(int step, int total_steps, int total_masked, int schedule) {
    const float t0 = (float)step / total_steps;
    const float t1 = (float)(step + 1) / total_steps;
    float frac;
    if (schedule == 0) {
        const float cos0 = cosf(t0 * M_PI * 0.5f);
        const float cos1 = cosf(t1 * M_PI * 0.5f);
        frac = (cos0 - cos1) / cos0;
    } else {
        frac = 1.0f / (total_steps - step);
    }
    int n = (int)roundf(frac * total_masked);
    if (n < 1 && total_masked > 0) n = 1;
    return std::min(n, total_masked);
}

const char * remask_name(int r) {
    return r == 2 ? "entropy_exit" : r == 0 ? "low_confidence" : r == 3 ? "maskgit_plus" : r == 4 ? "topk_margin"
                                                                                               : "random";
}


// forward_layers over M rows and n_keys keys from a captured graph (captured on first use).
int layers_graphed(diffuse_context * c, int M, int n_keys, int & pending) {
    for (auto & g : c->graphs)
        if (g.M == M && g.n_keys == n_keys && g.mode == c->attn_mode) {
            pending = g.pending;
            return hip_ok(hipGraphLaunch(g.exec, c->stream), "hipGraphLaunch");
        }
    if (c->graphs.size() >= 64) drop_graphs(c);
    hipGraph_t graph = nullptr;
    TRY(hip_ok(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"));
    const int rc = forward_layers(c, M, n_keys, pass_opts(), pending);
    const hipError_t e = hipStreamEndCapture(c->stream, &graph);
    if (rc != DFX_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc != DFX_OK ? rc : hip_ok(e, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    TRY(hip_ok(ei, "hipGraphInstantiate"));
    c->graphs.push_back({M, n_keys, c->attn_mode, pending, exec});
    return hip_ok(hipGraphLaunch(exec, c->stream), "hipGraphLaunch");
}

// Per-step device records and events of the device-resident loop, for up to n steps.
int ensure_steps(diffuse_context * c, int n) {
    if (n > c->steps_cap) {
        if (c->d_counts) (void)hipFree(c->d_counts);
        if (c->d_hist) (void)hipFree(c->d_hist);
        if (c->h_hist) (void)hipHostFree(c->h_hist);
        c->d_counts = c->d_hist = c->h_hist = nullptr;
        c->steps_cap = 0;
        TRY(hip_ok(hipMalloc((void **)&c->d_counts, (size_t)n * 4 * 4), "hipMalloc"));
        TRY(hip_ok(hipMalloc((void **)&c->d_hist, (size_t)n * 4), "hipMalloc"));
        TRY(hip_ok(hipHostMalloc((void **)&c->h_hist, (size_t)n * 4, hipHostMallocDefault), "hipHostMalloc"));
        c->steps_cap = n;
    }
    for (auto * v : {&c->ev_unmask, &c->ev_fwd0, &c->ev_fwd1})
        while ((int)v->size() < n) {
            hipEvent_t e = nullptr;
            TRY(hip_ok(hipEventCreate(&e), "hipEventCreate"));
            v->push_back(e);
        }
    return DFX_OK;
}

// The denoising loop with its bookkeeping on the device (temperature 0, every remasking
// policy but RANDOM): seq / prev / masked / lastc stay in HBM; each step is
//   k_step_prepare (active set, pass / head / sampler rows) -> layers -> head -> row
//   statistics -> candidates -> selection -> k_step_unmask (update_seq + unmask)
// and no step waits for its own selection.  The host needs a step's row count before
// enqueueing its layers and its masked count before the head and sampler; both follow from
// unmask counts of earlier steps (for a cached step: the positions masked when the previous
// step began, plus, with keep_active, those unmasked in the steps before that whose change
// was seen within the window), so the host enqueues step s's layers once step s-2 has
// ended and its head once step s-1 has: the GPU always has the next step's layers queued.
// A step enqueued speculatively after a step that unmasked everything left is dropped
// after its layers.  The prepare kernel's own counts are checked against the host's at
// the end.
int generate_device(diffuse_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                    const dfx_sampler_params & p, int32_t * out, dfx_gen_stats * stats,
                    const diffuse_step_callback * callback, int32_t * unmask_step) {
    using clk = std::chrono::steady_clock;
    const diffuse_model & md = *c->model;
    const int V = (int)md.hparams.n_vocab;
    const int mask_id = (int)md.hparams.mask_token_id;
    const bool shift = md.is_dream;
    const int N = n_prompt + n_generate;
    const int S = std::max(p.n_steps, 1);
    const bool use_cache = p.use_cache != 0;
    const int keep = std::max(p.cache_keep_active, 0);
    TRY(ensure_steps(c, S));
    int32_t * d_seq = c->d_state, * d_prev = d_seq + c->cap, * d_msk = d_prev + c->cap;
    int32_t * d_lastc = d_msk + c->cap, * d_ustep = d_lastc + c->cap;
    {
        int32_t * h = c->h_pin;   // 8 * cap int32
        for (int i = 0; i < N; i++) {
            h[i] = i < n_prompt ? prompt[i] : mask_id;
            h[c->cap + i] = -1;
            h[2 * c->cap + i] = i < n_prompt ? 0 : 1;
            h[3 * c->cap + i] = -1;
            h[4 * c->cap + i] = -1;
        }
        TRY(hip_ok(hipMemcpyAsync(d_seq, h, (size_t)5 * c->cap * 4, hipMemcpyHostToDevice, c->stream), "H2D"));
    }
    std::vector<int> rows(S, 0), nun(S, 0), full_v(S, 0), det(S, 0), masked_start(S + 1, 0);
    masked_start[0] = n_generate;
    bool cache_init = false;
    int actual_steps = 0;
    const auto gen_start = clk::now();
    auto step_unmasked = [&](int t) -> int {   // unmask count of an enqueued step (waits for it)
        TRY(hip_ok(hipEventSynchronize(c->ev_unmask[t]), "step"));
        const int n = c->h_hist[t];
        if (n < 0) {
            dfx_set_error("diffuse_generate: the selection of step %d named a candidate out of range", t);
            return DFX_ERR_HIP;
        }
        nun[t] = n;
        masked_start[t + 1] = masked_start[t] - n;
        return DFX_OK;
    };
    for (int s = 0; s < p.n_steps; s++) {
        if (s >= 2) TRY(step_unmasked(s - 2));
        // ---- row count of the step (compute_active_set, src/diffuse-cache.h:79-116, by counts)
        const bool force_full = !use_cache || !cache_init || (p.cache_refresh > 0 && s > 0 && s % p.cache_refresh == 0);
        int M = N;
        bool full = force_full;
        if (!force_full) {
            // positions masked when step s-1 began (still masked, or unmasked by step s-1)
            M = masked_start[s - 1];
            // plus those unmasked by step t <= s-2 whose change step t+1 saw, within the window
            if (keep > 0)
                for (int t = std::max(0, s - keep - 1); t <= s - 2; t++)
                    if (det[t + 1]) M += nun[t];
            if (M >= N || M == 0) full = true;
        }
        if (full) M = N;
        det[s] = !force_full;
        rows[s] = M;
        full_v[s] = full;
        TRY(dfx_step_prepare(N, s, force_full ? 1 : 0, keep, shift ? 1 : 0, shift ? 1 : 0, d_seq, d_prev, d_msk,
                             d_lastc, c->d_tok, c->d_pos, c->d_hrows, c->d_hmap, c->d_srows, c->d_spos,
                             c->d_counts + 4 * s, c->stream));
        TRY(hip_ok(hipEventRecord(c->ev_fwd0[s], c->stream), "event"));
        int pending = 0;
        if (c->use_graphs && !c->prof)
            TRY(layers_graphed(c, M, N, pending));
        else
            TRY(forward_layers(c, M, N, pass_opts(), pending));
        TRY(hip_ok(hipEventRecord(c->ev_fwd1[s], c->stream), "event"));
        if (use_cache) cache_init = true;
        // ---- the head and the sampler need the masked count when step s begins
        if (s >= 1) TRY(step_unmasked(s - 1));
        const int n_masked = masked_start[s];
        if (n_masked <= 0) break;   // the previous step unmasked everything: this one's layers are dropped
        actual_steps = s + 1;
        const int n_head = shift ? M : n_masked;
        TRY(forward_head(c, M, n_head, c->d_hrows, c->d_hmap, pending));
        const int n_sched = tokens_to_unmask(s, p.n_steps, n_masked, p.schedule);
        TRY(dfx_row_stats(c->logits, V, c->d_srows, n_masked, V, c->d_stats, c->stream));
        TRY(dfx_select_from_stats(c->d_stats, c->d_spos, n_masked, p.remasking, p.entropy_threshold, n_sched,
                                  c->d_cand, c->d_order, c->d_nun, c->stream));
        TRY(dfx_step_unmask(N, use_cache ? 1 : 0, s, d_seq, d_prev, d_msk, c->d_cand, c->d_order, c->d_nun, n_masked,
                            unmask_step ? d_ustep : nullptr, c->d_hist, c->stream));
        TRY(hip_ok(hipMemcpyAsync(c->h_hist + s, c->d_hist + s, 4, hipMemcpyDeviceToHost, c->stream), "D2H"));
        TRY(hip_ok(hipEventRecord(c->ev_unmask[s], c->stream), "event"));
        if (callback && *callback) {
            TRY(step_unmasked(s));
            std::vector<int32_t> seq(N);
            TRY(d2h_sync(c, seq.data(), d_seq, (size_t)N * 4));
            (*callback)(s + 1, p.n_steps, seq);
        }
    }
    TRY(hip_ok(hipStreamSynchronize(c->stream), "generate"));
    TRY(check_tiles(c));
    for (int t = 0; t < actual_steps; t++) TRY(step_unmasked(t));
    const double gen_ms = std::chrono::duration<double, std::milli>(clk::now() - gen_start).count();
    // the device's own row counts must be the ones the host launched with
    std::vector<int32_t> counts((size_t)4 * S);
    TRY(d2h_sync(c, counts.data(), c->d_counts, (size_t)4 * S * 4));
    for (int t = 0; t < actual_steps; t++)
        if (counts[4 * t] != rows[t] || counts[4 * t + 3] != full_v[t] ||
            counts[4 * t + 2] != masked_start[t] || (!shift && counts[4 * t + 1] != masked_start[t])) {
            dfx_set_error("diffuse_generate: step %d ran %d rows (full %d) but the active set has %d (full %d)", t,
                          rows[t], full_v[t], counts[4 * t], counts[4 * t + 3]);
            return DFX_ERR_HIP;
        }
    std::vector<int32_t> seq(N);
    TRY(d2h_sync(c, seq.data(), d_seq, (size_t)N * 4));
    memcpy(out, seq.data() + n_prompt, (size_t)n_generate * 4);
    if (unmask_step) {
        std::vector<int32_t> us(N);
        TRY(d2h_sync(c, us.data(), d_ustep, (size_t)N * 4));
        memcpy(unmask_step, us.data() + n_prompt, (size_t)n_generate * 4);
    }
    double total_fwd = 0;
    for (int t = 0; t < actual_steps; t++) {
        float ms = 0.0f;
        TRY(hip_ok(hipEventElapsedTime(&ms, c->ev_fwd0[t], c->ev_fwd1[t]), "event"));
        total_fwd += ms;
        DIFFUSE_LOG("  step %d/%d: unmasked %d tokens, %d remaining (fwd=%.1fms, active=%d/%d%s)", t + 1, p.n_steps,
                    nun[t], masked_start[t + 1], ms, rows[t], N,
                    !full_v[t] ? " CACHED" : (det[t] == 0 && t > 0 && use_cache) ? " REFRESH" : "");
        if (stats && t < 256) {
            stats->rows_per_step[t] = rows[t];
            stats->unmasked_per_step[t] = nun[t];
            stats->step_ms[t] = ms;
        }
    }
    const int as = std::max(actual_steps, 1);
    DIFFUSE_LOG("=== TIMING BREAKDOWN (%d steps, cache=%s, device loop) ===", actual_steps, use_cache ? "ON" : "OFF");
    DIFFUSE_LOG("  forward:   %8.1f ms  (%5.1f%%)  avg=%.1f ms/step", total_fwd, 100.0 * total_fwd / gen_ms,
                total_fwd / as);
    DIFFUSE_LOG("  TOTAL:     %8.1f ms  (%.2f tok/s)", gen_ms, 1000.0 * n_generate / gen_ms);
    if (stats) {
        stats->actual_steps = actual_steps;
        stats->total_ms = gen_ms;
        stats->forward_ms = total_fwd;
        stats->sample_ms = gen_ms - total_fwd;
    }
    prof_collect(c);
    return DFX_OK;
}

}  // namespace

int engine_context_new(const diffuse_model * m, int n_ctx, int n_threads, diffuse_context ** out) {
    diffuse_context * c = new diffuse_context();
    c->model = m;
    c->n_ctx = n_ctx;
    c->n_threads = n_threads;
    // non-blocking: no implicit ordering with the legacy stream, so a synchronous copy made by
    // another context (host thread) never has to wait for, or join, this stream while it is
    // being captured into a graph; every host read of this stream's results waits for it first
    int rc = hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc == DFX_OK) rc = hip_ok(hipEventCreate(&c->ev0), "hipEventCreate");
    if (rc == DFX_OK) rc = hip_ok(hipEventCreate(&c->ev1), "hipEventCreate");
    if (rc == DFX_OK) rc = hip_ok(hipEventCreate(&c->ev2), "hipEventCreate");
    if (rc == DFX_OK) rc = ensure_capacity(c, std::max(n_ctx, 1));
    if (rc != DFX_OK) {
        engine_context_free(c);
        return rc;
    }
    *out = c;
    return DFX_OK;
}

void engine_context_free(diffuse_context * c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    prof_collect(c);
    free_buffers(c);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->ev2) (void)hipEventDestroy(c->ev2);
    for (hipEvent_t e : c->prof_pool) (void)hipEventDestroy(e);
    for (auto * v : {&c->ev_unmask, &c->ev_fwd0, &c->ev_fwd1})
        for (hipEvent_t e : *v) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int engine_profile(diffuse_context * c, bool enable) {
    if (c->stream) TRY(hip_ok(hipStreamSynchronize(c->stream), "profile"));
    prof_collect(c);
    c->prof = enable;
    for (auto & cls : c->prof_tot)
        for (auto & t : cls) t = diffuse_context::prof_total();
    return DFX_OK;
}

int engine_profile_read(diffuse_context * c, int wtype, int rows_class, int64_t * launches, double * ms,
                        double * flops, double * bytes) {
    if (wtype < 0 || wtype >= 32 || rows_class < 0 || rows_class > 3) return DFX_ERR_ARG;
    TRY(hip_ok(hipStreamSynchronize(c->stream), "profile"));
    prof_collect(c);
    const auto & t = c->prof_tot[rows_class][wtype];
    if (launches) *launches = t.launches;
    if (ms) *ms = t.ms;
    if (flops) *flops = t.flops;
    if (bytes) *bytes = t.bytes;
    return DFX_OK;
}

int engine_forward(diffuse_context * c, const int32_t * tokens, int n, float * logits_out) {
    if (n <= 0 || !tokens || !logits_out) {
        dfx_set_error("diffuse_forward: bad arguments");
        return DFX_ERR_ARG;
    }
    const dims D(c->model->hparams);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->model->tok_embd.rows) {
            dfx_set_error("diffuse_forward: token %d out of range", tokens[i]);
            return DFX_ERR_ARG;
        }
    TRY(ensure_capacity(c, n));
    std::vector<int32_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0);
    TRY(upload_i32(c, c->d_tok, tokens, n, 0));
    TRY(upload_i32(c, c->d_pos, idx.data(), n, 1));
    TRY(upload_i32(c, c->d_hrows, idx.data(), n, 2));
    TRY(upload_i32(c, c->d_hmap, idx.data(), n, 3));
    c->kv_valid = 0;
    c->ar_past = 0;
    TRY(forward_pass(c, n, n, n));
    TRY(hip_ok(hipMemcpyAsync(logits_out, c->logits, (size_t)n * D.V * 4, hipMemcpyDeviceToHost, c->stream), "D2H"));
    TRY(hip_ok(hipStreamSynchronize(c->stream), "forward"));
    TRY(check_tiles(c));
    c->kv_valid = n;   // the K/V of positions 0..n-1 are in the cache
    prof_collect(c);
    return DFX_OK;
}

int engine_forward_cached(diffuse_context * c, const int32_t * active_tokens, const int32_t * active_pos, int n_active,
                          int n_total, float * logits_out) {
    if (n_active <= 0 || !active_tokens || !active_pos || !logits_out || n_active > n_total) {
        dfx_set_error("diffuse_forward_cached: bad arguments");
        return DFX_ERR_ARG;
    }
    if (c->kv_valid != n_total) {
        dfx_set_error("diffuse_forward_cached: the cache holds %d positions, not %d (run a full forward first)",
                      c->kv_valid, n_total);
        return DFX_ERR_ARG;
    }
    const dims D(c->model->hparams);
    std::vector<char> seen(n_total, 0);
    for (int a = 0; a < n_active; a++) {
        if (active_tokens[a] < 0 || active_tokens[a] >= c->model->tok_embd.rows) {
            dfx_set_error("diffuse_forward_cached: token %d out of range", active_tokens[a]);
            return DFX_ERR_ARG;
        }
        if (active_pos[a] < 0 || active_pos[a] >= n_total || seen[active_pos[a]]) {
            dfx_set_error("diffuse_forward_cached: position %d out of range or repeated", active_pos[a]);
            return DFX_ERR_ARG;
        }
        seen[active_pos[a]] = 1;
    }
    std::vector<int32_t> idx(n_active);
    std::iota(idx.begin(), idx.end(), 0);
    TRY(upload_i32(c, c->d_tok, active_tokens, n_active, 0));
    TRY(upload_i32(c, c->d_pos, active_pos, n_active, 1));
    TRY(upload_i32(c, c->d_hrows, idx.data(), n_active, 2));
    TRY(upload_i32(c, c->d_hmap, idx.data(), n_active, 3));
    // the active rows' K/V are written into the cache before attention reads all
    // n_total positions (update_kv + the [cached | active] concat of the reference)
    TRY(forward_pass(c, n_active, n_total, n_active));
    TRY(hip_ok(hipMemcpyAsync(logits_out, c->logits, (size_t)n_active * D.V * 4, hipMemcpyDeviceToHost, c->stream),
               "D2H"));
    TRY(hip_ok(hipStreamSynchronize(c->stream), "forward"));
    TRY(check_tiles(c));
    prof_collect(c);
    return DFX_OK;
}

int engine_generate(diffuse_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                    const dfx_sampler_params & p, int32_t * out, dfx_gen_stats * stats,
                    const diffuse_step_callback * callback, int32_t * unmask_step) {
    using clk = std::chrono::steady_clock;
    const diffuse_model & md = *c->model;
    const int V = (int)md.hparams.n_vocab;
    const int mask_id = (int)md.hparams.mask_token_id;
    const bool shift = md.is_dream;   // Dream reads logits of position max(i-1, 0)
    const int N = n_prompt + n_generate;
    if (n_prompt < 0 || n_generate < 0 || N <= 0 || p.n_steps < 0) {
        dfx_set_error("diffuse_generate: bad arguments");
        return DFX_ERR_ARG;
    }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= md.tok_embd.rows) {
            dfx_set_error("diffuse_generate: prompt token %d out of range", prompt[i]);
            return DFX_ERR_ARG;
        }
    if (mask_id < 0 || mask_id >= md.tok_embd.rows) {
        dfx_set_error("diffuse_generate: mask token %d outside the embedding table", mask_id);
        return DFX_ERR_FORMAT;
    }
    TRY(ensure_capacity(c, N));
    c->kv_valid = 0;   // the generation leaves the cache partly stale
    c->ar_past = 0;

    std::vector<int32_t> seq(prompt, prompt + n_prompt);
    seq.resize(N, mask_id);
    std::vector<char> is_masked(N, 0);
    for (int i = n_prompt; i < N; i++) is_masked[i] = 1;
    int n_masked = n_generate;
    std::mt19937 rng(p.seed);

    const bool use_cache = p.use_cache != 0;
    std::vector<int32_t> prev_seq(N, -1);
    std::vector<int> last_changed(N, -1);
    bool cache_init = false;
    if (stats) memset(stats, 0, sizeof(*stats));
    if (unmask_step)
        for (int i = 0; i < n_generate; i++) unmask_step[i] = -1;

    DIFFUSE_LOG("diffusion: %d steps, %d tokens to generate, scheduler=%s, cache=%s, refresh=%d, keep_active=%d",
                p.n_steps, n_generate, remask_name(p.remasking), use_cache ? "ON" : "OFF", p.cache_refresh,
                p.cache_keep_active);

    if (c->device_loop && p.temperature <= 0.0f && p.remasking != 1 && n_generate > 0)
        return generate_device(c, prompt, n_prompt, n_generate, p, out, stats, callback, unmask_step);

    double total_fwd = 0, total_sample = 0, total_sort = 0, total_unmask = 0;
    int actual_steps = 0;
    const auto gen_start = clk::now();
    std::vector<int32_t> act, tok, hrows, hmap, srows, spos, order;
    std::vector<dfx_candidate> cand;
    std::vector<char> need(N);

    for (int step = 0; step < p.n_steps && n_masked > 0; step++) {
        actual_steps++;
        const auto t0 = clk::now();
        const bool force_full = !use_cache || !cache_init ||
                                (p.cache_refresh > 0 && step > 0 && step % p.cache_refresh == 0);
        bool full = force_full;
        act.clear();
        if (!force_full) {
            // compute_active_set (src/diffuse-cache.h:79-116)
            for (int i = 0; i < N; i++) {
                const bool changed = seq[i] != prev_seq[i];
                if (changed) last_changed[i] = step;
                const bool recent = p.cache_keep_active > 0 && last_changed[i] >= 0 &&
                                    (step - last_changed[i]) <= p.cache_keep_active;
                if (changed || is_masked[i] || recent) act.push_back(i);
            }
            if ((int)act.size() >= N || act.empty()) full = true;
        }
        if (full) {
            act.resize(N);
            std::iota(act.begin(), act.end(), 0);
        }
        const int M = (int)act.size();
        // rows whose logits the sampler reads this step (only masked positions, or
        // their left neighbour for Dream); other rows skip the vocab head.
        std::fill(need.begin(), need.end(), 0);
        for (int i = 0; i < N; i++)
            if (is_masked[i]) need[shift ? std::max(i - 1, 0) : i] = 1;
        tok.resize(M);
        hrows.clear();
        hmap.clear();
        for (int a = 0; a < M; a++) {
            tok[a] = seq[act[a]];
            if (need[act[a]]) {
                hrows.push_back(a);
                hmap.push_back(act[a]);
            }
        }
        // rows the sampler scans: every masked position (its left neighbour's row for Dream)
        srows.clear();
        spos.clear();
        for (int i = 0; i < N; i++)
            if (is_masked[i]) {
                srows.push_back(shift ? std::max(i - 1, 0) : i);
                spos.push_back(i);
            }
        const int n_cand = (int)spos.size();
        // The step's six index arrays go up in one copy; the forward, the row statistics,
        // candidates and selection are queued behind it, and the host waits once, for the
        // copy of the selection back.
        stage_i32(c, tok.data(), M, 0);
        stage_i32(c, act.data(), M, 1);
        stage_i32(c, hrows.data(), (int)hrows.size(), 2);
        stage_i32(c, hmap.data(), (int)hmap.size(), 3);
        stage_i32(c, srows.data(), n_cand, 4);
        stage_i32(c, spos.data(), n_cand, 5);
        const double prep_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
        TRY(upload_slots(c, 6));
        TRY(hip_ok(hipEventRecord(c->ev0, c->stream), "event"));
        TRY(forward_pass(c, M, N, (int)hrows.size()));
        TRY(hip_ok(hipEventRecord(c->ev1, c->stream), "event"));
        if (use_cache) {   // update_seq right after the forward (src/diffuse-sampler.cpp:154, 171, 194)
            prev_seq = seq;
            cache_init = true;
        }

        // ---- candidates (src/diffuse-sampler.cpp:222-270) ----
        TRY(dfx_row_stats(c->logits, V, c->d_srows, n_cand, V, c->d_stats, c->stream));
        const int n_sched = tokens_to_unmask(step, p.n_steps, n_masked, p.schedule);
        int n_unmask = n_sched;
        cand.resize(n_cand);
        order.resize(n_cand);
        const bool greedy = p.temperature <= 0.0f;
        if (greedy) {
            TRY(dfx_make_candidates(c->d_stats, c->d_spos, n_cand, p.remasking == 4 ? 1 : 0, c->d_cand, c->stream));
            if (p.remasking != 1)
                TRY(dfx_select(c->d_cand, n_cand, p.remasking, p.entropy_threshold, n_sched, c->d_order, c->d_nun,
                               c->stream));
            TRY(hip_ok(hipEventRecord(c->ev2, c->stream), "event"));
            TRY(hip_ok(hipMemcpyAsync(c->h_out, c->d_out, c->out_bytes, hipMemcpyDeviceToHost, c->stream), "D2H"));
        } else {
            TRY(hip_ok(hipEventRecord(c->ev2, c->stream), "event"));
        }
        TRY(hip_ok(hipStreamSynchronize(c->stream), "step"));
        const auto t2 = clk::now();
        float gpu_fwd_ms = 0.0f, gpu_smp_ms = 0.0f;
        TRY(hip_ok(hipEventElapsedTime(&gpu_fwd_ms, c->ev0, c->ev1), "event"));
        TRY(hip_ok(hipEventElapsedTime(&gpu_smp_ms, c->ev1, c->ev2), "event"));
        const double fwd_ms = prep_ms + gpu_fwd_ms;
        total_fwd += fwd_ms;
        total_sample += gpu_smp_ms;
        if (greedy) {
            const auto * hc = (const dfx_candidate *)c->h_out;
            std::copy(hc, hc + n_cand, cand.begin());
            if (p.remasking != 1) {
                const auto * ho = (const int32_t *)(hc + c->cap);
                std::copy(ho, ho + n_cand, order.begin());
                n_unmask = ho[c->cap];
                for (int j = 0; j < n_cand; j++)
                    if (order[j] < 0 || order[j] >= n_cand) {
                        dfx_set_error("diffuse_generate: selection returned index %d of %d", order[j], n_cand);
                        return DFX_ERR_HIP;
                    }
            }
        } else {
            // Stochastic path stays on the host like the reference (src/diffuse-sampler.cpp:256-269).
            std::vector<dfx_row_stat> st(n_cand);
            std::vector<float> rowbuf((size_t)V);
            TRY(d2h_sync(c, st.data(), c->d_stats, (size_t)n_cand * sizeof(dfx_row_stat)));
            std::vector<float> probs((size_t)V);
            for (int j = 0; j < n_cand; j++) {
                TRY(d2h_sync(c, rowbuf.data(), c->logits + (size_t)srows[j] * V, (size_t)V * 4));
                const float mx = *std::max_element(rowbuf.begin(), rowbuf.end());
                float sum = 0.0f;
                for (int v = 0; v < V; v++) {
                    probs[v] = expf((rowbuf[v] - mx) / p.temperature);
                    sum += probs[v];
                }
                for (int v = 0; v < V; v++) probs[v] /= sum;
                std::discrete_distribution<int> dist(probs.begin(), probs.end());
                const int s = dist(rng);
                cand[j] = dfx_candidate{spos[j], s, probs[s], st[j].entropy};
            }
        }
        const auto t3 = clk::now();
        total_sample += std::chrono::duration<double, std::milli>(t3 - t2).count();   // host part

        // ---- ordering (src/diffuse-sampler.cpp:277-308) ----
        const auto t4 = clk::now();
        std::vector<dfx_candidate> sorted(n_cand);
        if (p.remasking == 1) {
            std::shuffle(cand.begin(), cand.end(), rng);
            sorted = cand;
        } else if (p.temperature <= 0.0f) {
            for (int j = 0; j < n_cand; j++) sorted[j] = cand[order[j]];
        } else {
            const bool by_ent = p.remasking == 2;
            sorted = cand;
            std::sort(sorted.begin(), sorted.end(), [by_ent](const dfx_candidate & a, const dfx_candidate & b) {
                if (by_ent) {
                    if (a.entropy != b.entropy) return a.entropy < b.entropy;
                } else if (a.confidence != b.confidence) {
                    return a.confidence > b.confidence;
                }
                return a.pos < b.pos;
            });
            if (by_ent) {
                int n_easy = 0;
                for (const auto & x : sorted) {
                    if (x.entropy < p.entropy_threshold) n_easy++;
                    else break;
                }
                n_unmask = std::min(std::max(n_sched, n_easy), n_cand);
            }
        }
        const auto t5 = clk::now();
        total_sort += std::chrono::duration<double, std::milli>(t5 - t4).count();

        // ---- unmask (src/diffuse-sampler.cpp:316-323) ----
        const auto t6 = clk::now();
        int done = 0;
        for (int j = 0; j < n_unmask && j < n_cand; j++) {
            seq[sorted[j].pos] = sorted[j].token;
            is_masked[sorted[j].pos] = 0;
            if (unmask_step) unmask_step[sorted[j].pos - n_prompt] = step;
            n_masked--;
            done++;
        }
        const auto t7 = clk::now();
        total_unmask += std::chrono::duration<double, std::milli>(t7 - t6).count();

        DIFFUSE_LOG("  step %d/%d: unmasked %d tokens, %d remaining (fwd=%.1fms, active=%d/%d%s)", step + 1, p.n_steps,
                    done, n_masked, fwd_ms, full ? N : M, N, !full ? " CACHED" : (force_full && step > 0) ? " REFRESH" : "");
        if (stats && step < 256) {
            stats->rows_per_step[step] = M;
            stats->unmasked_per_step[step] = done;
            stats->step_ms[step] = (float)fwd_ms;
        }
        prof_collect(c);   // the stream was synchronised by the sampler
        if (callback && *callback) (*callback)(step + 1, p.n_steps, seq);
    }

    const double gen_ms = std::chrono::duration<double, std::milli>(clk::now() - gen_start).count();
    const double overhead = gen_ms - total_fwd - total_sample - total_sort - total_unmask;
    const int as = std::max(actual_steps, 1);
    DIFFUSE_LOG("=== TIMING BREAKDOWN (%d steps, cache=%s) ===", actual_steps, use_cache ? "ON" : "OFF");
    DIFFUSE_LOG("  forward:   %8.1f ms  (%5.1f%%)  avg=%.1f ms/step", total_fwd, 100.0 * total_fwd / gen_ms, total_fwd / as);
    DIFFUSE_LOG("  sampling:  %8.1f ms  (%5.1f%%)  avg=%.1f ms/step", total_sample, 100.0 * total_sample / gen_ms,
                total_sample / as);
    DIFFUSE_LOG("  sorting:   %8.1f ms  (%5.1f%%)", total_sort, 100.0 * total_sort / gen_ms);
    DIFFUSE_LOG("  unmask:    %8.1f ms  (%5.1f%%)", total_unmask, 100.0 * total_unmask / gen_ms);
    DIFFUSE_LOG("  overhead:  %8.1f ms  (%5.1f%%)", overhead, 100.0 * overhead / gen_ms);
    DIFFUSE_LOG("  TOTAL:     %8.1f ms  (%.2f tok/s)", gen_ms, 1000.0 * n_generate / gen_ms);
    if (stats) {
        stats->actual_steps = actual_steps;
        stats->total_ms = gen_ms;
        stats->forward_ms = total_fwd;
        stats->sample_ms = total_sample + total_sort + total_unmask;
    }
    TRY(check_tiles(c));
    memcpy(out, seq.data() + n_prompt, (size_t)n_generate * 4);
    return DFX_OK;
}

int engine_hip_ok(hipError_t e, const char * what) { return hip_ok(e, what); }
int engine_check_tiles(diffuse_context * c) { return check_tiles(c); }
int engine_reserve(diffuse_context * c, int N) { return ensure_capacity(c, N); }
int engine_pass(diffuse_context * c, int M, int n_keys, int n_head, const pass_opts & o) {
    return forward_pass(c, M, n_keys, n_head, o);
}
void engine_prof_collect(diffuse_context * c) { prof_collect(c); }
