// ar.cpp — the autoregressive API on one gfx950 GPU (src/ar-graph.cpp, src/ar-cache.h,
// src/ar-sampler.cpp).
//
// The append-only cache is the context's key / value cache: a pass over n_new tokens at
// positions n_past.. stores their keys and values at those positions (dfx_rope_store)
// and attends causally over positions 0..n_past+n_new-1 (dfx_attention_causal), so the
// reference's concat of cached and new K/V (src/ar-graph.cpp:146-172) is the cache read
// itself.  Skipped layers write nothing, as in the reference.
//
// Sampling: temperature <= 0 is the greedy path, done on the device (dfx_ar_greedy keeps
// the next token, its position and the repeat-penalty ring in device memory, so a decode
// pass needs no upload); otherwise the row comes back to the host and sample_token runs
// with the reference's own std:: algorithms (nth_element, sort, discrete_distribution
// over a std::mt19937), as the reference does, token for token.
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

int check_tokens(const diffuse_context * c, const int32_t * t, int n, const char * what) {
    for (int i = 0; i < n; i++)
        if (t[i] < 0 || t[i] >= c->model->tok_embd.rows) {
            dfx_set_error("%s: token %d out of range", what, t[i]);
            return DFX_ERR_ARG;
        }
    return DFX_OK;
}

// Device buffers of the AR path beyond the context's own (made on first use, freed with
// the context's buffers): the profile's layer-input copy and row sums, the decode state,
// the pinned logits row.
int ar_buffers(diffuse_context * c, bool profile, int ring, bool host_row) {
    const int64_t d = c->model->hparams.n_embd, L = c->model->hparams.n_layer, V = c->model->hparams.n_vocab;
    if (profile && !c->x_prev) {
        TRY(engine_hip_ok(hipMalloc((void **)&c->x_prev, (size_t)c->cap * d * 4), "hipMalloc"));
        TRY(engine_hip_ok(hipMalloc((void **)&c->d_imp, (size_t)L * c->cap * 8), "hipMalloc"));
    }
    ring = std::max(ring, 0);
    if (!c->d_ar || c->ar_ring < ring) {
        if (c->d_ar) (void)hipFree(c->d_ar);
        c->d_ar = nullptr;
        TRY(engine_hip_ok(hipMalloc((void **)&c->d_ar, (size_t)(8 + ring) * 4), "hipMalloc"));
        c->ar_ring = ring;
        TRY(engine_hip_ok(hipMemsetAsync(c->d_ar, 0, 16, c->stream), "memset"));
    }
    if (host_row && !c->h_row)
        TRY(engine_hip_ok(hipHostMalloc((void **)&c->h_row, (size_t)V * 4, hipHostMallocDefault), "hipHostMalloc"));
    return DFX_OK;
}

// One causal pass over n_new tokens at positions ar_past.. (ar_forward_impl,
// src/ar-graph.cpp:262-399).  Logits: every row (all_rows) or the last row into logits
// row 0.  profile: every layer runs and the per-layer impacts come back in impact[L].
int ar_pass(diffuse_context * c, const int32_t * tokens, int n_new, int window, bool all_rows, bool profile,
            float * impact) {
    const int n_past = c->ar_past;
    if (n_new <= 0 || n_past + n_new > c->cap) {
        dfx_set_error("ar_forward: %d tokens after %d exceed the context's %d positions", n_new, n_past, c->cap);
        return DFX_ERR_ARG;
    }
    if (window < 0) {
        dfx_set_error("ar_forward: negative sliding window %d", window);
        return DFX_ERR_ARG;
    }
    TRY(check_tokens(c, tokens, n_new, "ar_forward"));
    const int64_t L = c->model->hparams.n_layer;
    int32_t * st = c->h_pin;
    const int64_t cap = c->cap;
    for (int i = 0; i < n_new; i++) {
        st[i] = tokens[i];
        st[cap + i] = n_past + i;
        st[2 * cap + i] = all_rows ? i : n_new - 1;
        st[3 * cap + i] = all_rows ? i : 0;
    }
    TRY(engine_hip_ok(hipMemcpyAsync(c->d_ints, st, (size_t)4 * cap * 4, hipMemcpyHostToDevice, c->stream), "H2D"));
    pass_opts o;
    o.q_pos0 = n_past;
    o.window = window;
    o.skip = (!profile && !c->ar_skip.empty()) ? c->ar_skip.data() : nullptr;
    o.impact_rows = profile ? c->d_imp : nullptr;
    c->kv_valid = 0;
    TRY(engine_pass(c, n_new, n_past + n_new, all_rows ? n_new : 1, o));
    c->ar_past = n_past + n_new;
    if (profile) {
        // rows added in order in double, then rounded (ggml_sum over the rows)
        std::vector<double> rows((size_t)L * n_new);
        TRY(engine_hip_ok(hipMemcpyAsync(rows.data(), c->d_imp, rows.size() * 8, hipMemcpyDeviceToHost, c->stream),
                          "D2H"));
        TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "profile"));
        for (int64_t il = 0; il < L; il++) {
            double tot = 0.0;
            for (int m = 0; m < n_new; m++) tot += rows[il * n_new + m];
            impact[il] = (float)tot;
        }
    }
    return DFX_OK;
}

// ar_profile_layers' choice (src/ar-graph.cpp:474-503): rank (impact, layer) ascending,
// skip the first n_skip outside layers 0, 1, L-2, L-1.
int choose_skip(const std::vector<float> & impact, int n_skip, std::vector<uint8_t> & skip) {
    const int L = (int)impact.size();
    skip.assign(L, 0);
    if (n_skip <= 0) return 0;
    std::vector<std::pair<float, int>> ranked;
    for (int il = 0; il < L; il++) ranked.push_back({impact[il], il});
    std::sort(ranked.begin(), ranked.end());
    DIFFUSE_LOG("  lowest impact layers:");
    for (int i = 0; i < std::min(n_skip + 4, L); i++)
        DIFFUSE_LOG("    layer %2d: impact = %.6e%s", ranked[i].second, ranked[i].first,
                    (ranked[i].second < 2 || ranked[i].second >= L - 2) ? " [PROTECTED]" : "");
    int skipped = 0;
    for (auto & r : ranked) {
        if (skipped >= n_skip) break;
        if (r.second < 2 || r.second >= L - 2) continue;
        skip[r.second] = 1;
        skipped++;
    }
    DIFFUSE_LOG("  layer-skip: %d/%d layers skipped during decode", skipped, L);
    return skipped;
}

// ---- sample_token for temperature > 0 (src/ar-sampler.cpp:11-140), on the host

void top_k_filter(float * lg, int V, int top_k) {
    if (top_k <= 0 || top_k >= V) return;
    std::vector<float> tmp(lg, lg + V);
    std::nth_element(tmp.begin(), tmp.begin() + top_k, tmp.end(), std::greater<float>());
    const float threshold = tmp[top_k - 1];
    for (int i = 0; i < V; i++)
        if (lg[i] < threshold) lg[i] = -INFINITY;
}

void top_p_filter(float * lg, int V, float top_p) {
    if (top_p >= 1.0f) return;
    const float mx = *std::max_element(lg, lg + V);
    float sum = 0.0f;
    for (int i = 0; i < V; i++) {
        lg[i] = expf(lg[i] - mx);
        sum += lg[i];
    }
    for (int i = 0; i < V; i++) lg[i] /= sum;
    std::vector<int> idx(V);
    std::iota(idx.begin(), idx.end(), 0);
    std::sort(idx.begin(), idx.end(), [&](int a, int b) { return lg[a] > lg[b]; });
    float cum = 0.0f;
    int cutoff = V;
    for (int i = 0; i < V; i++) {
        cum += lg[idx[i]];
        if (cum >= top_p) {
            cutoff = i + 1;
            break;
        }
    }
    for (int i = cutoff; i < V; i++) lg[idx[i]] = 0.0f;
    for (int i = 0; i < V; i++) lg[i] = lg[i] > 0.0f ? logf(lg[i]) : -INFINITY;
}

int32_t sample_host(float * lg, int V, const dfx_ar_params & p, const std::vector<int32_t> & recent,
                    std::mt19937 & rng) {
    if (p.repeat_penalty > 1.0f)
        for (int32_t t : recent)
            if (t >= 0 && t < V) lg[t] = lg[t] > 0.0f ? lg[t] / p.repeat_penalty : lg[t] * p.repeat_penalty;
    if (p.temperature <= 0.0f) {
        int best = 0;
        float bv = lg[0];
        for (int i = 1; i < V; i++)
            if (lg[i] > bv) {
                bv = lg[i];
                best = i;
            }
        return best;
    }
    for (int i = 0; i < V; i++) lg[i] /= p.temperature;
    top_k_filter(lg, V, p.top_k);
    top_p_filter(lg, V, p.top_p);
    const float mx = *std::max_element(lg, lg + V);
    float sum = 0.0f;
    std::vector<float> probs(V);
    for (int i = 0; i < V; i++) {
        probs[i] = expf(lg[i] - mx);
        sum += probs[i];
    }
    for (int i = 0; i < V; i++) probs[i] /= sum;
    std::discrete_distribution<int> dist(probs.begin(), probs.end());
    return dist(rng);
}

}  // namespace

int engine_ar_forward(diffuse_context * c, const int32_t * tokens, int n_new, bool reset, int window,
                      float * logits_out) {
    if (!tokens || n_new <= 0) {
        dfx_set_error("ar_forward: bad arguments");
        return DFX_ERR_ARG;
    }
    if (reset) {
        TRY(engine_reserve(c, n_new));
        c->ar_past = 0;
    }
    TRY(ar_pass(c, tokens, n_new, window, true, false, nullptr));
    const int64_t V = c->model->hparams.n_vocab;
    if (logits_out)
        TRY(engine_hip_ok(hipMemcpyAsync(logits_out, c->logits, (size_t)n_new * V * 4, hipMemcpyDeviceToHost,
                                         c->stream), "D2H"));
    TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "ar_forward"));
    TRY(engine_check_tiles(c));
    engine_prof_collect(c);
    return DFX_OK;
}

int engine_ar_profile(diffuse_context * c, const int32_t * tokens, int n, int window, int n_skip, float * logits_out,
                      float * impact_out, uint8_t * skip_out) {
    if (!tokens || n <= 0) {
        dfx_set_error("ar_profile_layers: bad arguments");
        return DFX_ERR_ARG;
    }
    const int L = (int)c->model->hparams.n_layer;
    TRY(engine_reserve(c, n));
    TRY(ar_buffers(c, true, 0, false));
    c->ar_skip.clear();
    c->ar_past = 0;
    DIFFUSE_LOG("ar_profile_layers: %d tokens, target skip=%d/%d layers", n, n_skip, L);
    std::vector<float> impact(L, 0.0f);
    TRY(ar_pass(c, tokens, n, window, true, true, impact.data()));
    std::vector<uint8_t> skip;
    choose_skip(impact, n_skip, skip);
    c->ar_skip = skip;
    const int64_t V = c->model->hparams.n_vocab;
    if (logits_out)
        TRY(engine_hip_ok(hipMemcpyAsync(logits_out, c->logits, (size_t)n * V * 4, hipMemcpyDeviceToHost, c->stream),
                          "D2H"));
    TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "ar_profile_layers"));
    TRY(engine_check_tiles(c));
    if (impact_out) memcpy(impact_out, impact.data(), (size_t)L * 4);
    if (skip_out) memcpy(skip_out, skip.data(), (size_t)L);
    engine_prof_collect(c);
    return DFX_OK;
}

int engine_ar_generate(diffuse_context * c, const int32_t * prompt, int n_prompt, int max_tokens,
                       const dfx_ar_params & p, std::vector<int32_t> & out, dfx_ar_stats * stats,
                       const std::function<bool(int32_t, int)> * cb) {
    using clk = std::chrono::steady_clock;
    out.clear();
    if (stats) memset(stats, 0, sizeof(*stats));
    if (!prompt || n_prompt <= 0 || max_tokens < 0 || p.sliding_window < 0) {
        dfx_set_error("ar_generate: bad arguments");
        return DFX_ERR_ARG;
    }
    TRY(check_tokens(c, prompt, n_prompt, "ar_generate"));
    const diffuse_hparams & hp = c->model->hparams;
    const int V = (int)hp.n_vocab, L = (int)hp.n_layer;
    const int total_ctx = n_prompt + std::max(max_tokens, 1);
    DIFFUSE_LOG("ar_generate: prompt=%d tokens, max_generate=%d, ctx=%d", n_prompt, max_tokens, total_ctx);
    // greedy sampling runs on the device for rings up to 4096 recent tokens (the same
    // result as the host sampler, which takes longer windows)
    const bool greedy = p.temperature <= 0.0f && std::min(std::max(p.repeat_last_n, 0), total_ctx) <= 4096;
    // the recent list never holds more than total_ctx tokens, so a ring of that size
    // never evicts where the reference's list would not
    const int ring = std::min(std::max(p.repeat_last_n, 0), total_ctx);
    TRY(engine_reserve(c, total_ctx));
    TRY(ar_buffers(c, p.layer_skip > 0, ring, !greedy));
    c->ar_past = 0;
    c->ar_skip.clear();
    std::mt19937 rng(p.seed);

    const auto gen_start = clk::now();
    // ---- prefill (the last row's logits are the only ones read)
    std::vector<float> impact(L, 0.0f);
    if (p.layer_skip > 0) {
        DIFFUSE_LOG("ar_profile_layers: %d tokens, target skip=%d/%d layers", n_prompt, p.layer_skip, L);
        TRY(ar_pass(c, prompt, n_prompt, p.sliding_window, false, true, impact.data()));
        std::vector<uint8_t> skip;
        const int skipped = choose_skip(impact, p.layer_skip, skip);
        c->ar_skip = skip;
        if (stats) stats->n_skipped_layers = skipped;
    } else {
        TRY(ar_pass(c, prompt, n_prompt, p.sliding_window, false, false, nullptr));
    }
    TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "ar_generate prefill"));
    TRY(engine_check_tiles(c));
    const double prefill_ms = std::chrono::duration<double, std::milli>(clk::now() - gen_start).count();
    DIFFUSE_LOG("  prefill: %d tokens in %.1f ms (%.1f tok/s)", n_prompt, prefill_ms, 1000.0 * n_prompt / prefill_ms);

    // recent tokens for the repeat penalty: the prompt's tail (src/ar-sampler.cpp:221-228)
    std::vector<int32_t> recent;
    for (int i = std::max(0, n_prompt - p.repeat_last_n); i < n_prompt; i++) recent.push_back(prompt[i]);

    // decode state of the greedy path: zeros, then [token, position, n, start, ring...];
    // the position starts one before the first generated token's (the sampler advances it)
    int32_t * tok_host = c->h_pin;
    if (greedy) {
        int32_t * st = c->h_pin;
        memset(st, 0, (size_t)(8 + ring) * 4);
        st[4 + 1] = n_prompt - 1;
        st[4 + 2] = (int)recent.size();
        for (size_t j = 0; j < recent.size(); j++) st[8 + j] = recent[j];
        TRY(engine_hip_ok(hipMemcpyAsync(c->d_ar, st, (size_t)(8 + ring) * 4, hipMemcpyHostToDevice, c->stream),
                          "H2D"));
        tok_host = c->h_pin + 8 + ring;
    }
    int32_t * d_zero = c->d_ar, * d_state = c->d_ar + 4;
    int32_t * d_tokout = c->d_ints;   // slot 0 of the index arrays is free during decoding

    auto sample = [&](int32_t & tok) -> int {
        if (greedy) {
            TRY(dfx_ar_greedy(c->logits, V, d_state, ring, p.repeat_penalty, d_tokout, c->stream));
            TRY(engine_hip_ok(hipMemcpyAsync(tok_host, d_tokout, 4, hipMemcpyDeviceToHost, c->stream), "D2H"));
            TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "ar_generate"));
            tok = *tok_host;
        } else {
            TRY(engine_hip_ok(hipMemcpyAsync(c->h_row, c->logits, (size_t)V * 4, hipMemcpyDeviceToHost, c->stream),
                              "D2H"));
            TRY(engine_hip_ok(hipStreamSynchronize(c->stream), "ar_generate"));
            tok = sample_host(c->h_row, V, p, recent, rng);
        }
        recent.push_back(tok);
        if ((int)recent.size() > p.repeat_last_n) recent.erase(recent.begin());
        out.push_back(tok);
        return DFX_OK;
    };

    int32_t tok = 0;
    TRY(sample(tok));
    bool stop = cb && *cb && !(*cb)(tok, n_prompt);
    int n_decoded = 0;
    const auto dec_start = clk::now();
    pass_opts o;
    o.window = p.sliding_window;
    o.hrows = d_zero;
    o.hmap = d_zero;
    for (int i = 1; i < max_tokens && !stop; i++) {
        const int32_t last = out.back();
        if (last == 151643 || last == 151645 || last == 151644) {   // src/ar-sampler.cpp:253-260
            DIFFUSE_LOG("  EOS token %d at position %d", last, n_prompt + i - 1);
            break;
        }
        if (c->ar_past + 1 > c->cap) {
            dfx_set_error("ar_generate: context full");
            return DFX_ERR_ARG;
        }
        if (greedy) {
            o.tok = d_state;        // the token and position the sampler left on the device
            o.pos = d_state + 1;
        } else {
            int32_t * st = c->h_pin;
            st[0] = last;
            st[1] = c->ar_past;
            TRY(engine_hip_ok(hipMemcpyAsync(c->d_ints, st, 4, hipMemcpyHostToDevice, c->stream), "H2D"));
            TRY(engine_hip_ok(hipMemcpyAsync(c->d_pos, st + 1, 4, hipMemcpyHostToDevice, c->stream), "H2D"));
            o.tok = c->d_ints;
            o.pos = c->d_pos;
        }
        o.q_pos0 = c->ar_past;
        o.skip = c->ar_skip.empty() ? nullptr : c->ar_skip.data();
        TRY(engine_pass(c, 1, c->ar_past + 1, 1, o));
        c->ar_past += 1;
        TRY(sample(tok));
        n_decoded++;
        if (cb && *cb && !(*cb)(tok, n_prompt + i)) break;
    }
    const auto gen_end = clk::now();
    const double decode_ms = std::chrono::duration<double, std::milli>(gen_end - dec_start).count();
    const double total_ms = std::chrono::duration<double, std::milli>(gen_end - gen_start).count();
    DIFFUSE_LOG("=== AR GENERATION COMPLETE ===");
    DIFFUSE_LOG("  prefill:  %6.1f ms  (%d tokens, %.1f tok/s)", prefill_ms, n_prompt,
                1000.0 * n_prompt / std::max(prefill_ms, 0.1));
    DIFFUSE_LOG("  decode:   %6.1f ms  (%d tokens, %.2f tok/s)", decode_ms, n_decoded,
                n_decoded > 0 ? 1000.0 * n_decoded / decode_ms : 0.0);
    DIFFUSE_LOG("  total:    %6.1f ms  (%d generated)", total_ms, (int)out.size());
    DIFFUSE_LOG("  KV cache: %d / %d positions used", c->ar_past, total_ctx);
    if (stats) {
        stats->prefill_ms = prefill_ms;
        stats->decode_ms = decode_ms;
        stats->total_ms = total_ms;
        stats->n_prompt = n_prompt;
        stats->n_decoded = n_decoded;
        stats->n_generated = (int)out.size();
    }
    engine_prof_collect(c);
    return DFX_OK;
}
