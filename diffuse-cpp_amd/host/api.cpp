// api.cpp — the C form (dfx.h) and the C++ form (diffuse.h) of the public API.
//
// C++ entry points keep the reference's error behaviour: load failures are fatal
// (DIFFUSE_DIE, src/diffuse-common.h:17-21 and src/diffuse-model.cpp:4-10, 74-80,
// 92-95), diffuse_forward returns false after logging (src/diffuse-graph.cpp:331-345),
// and a failed forward inside diffuse_generate is fatal (src/diffuse-sampler.cpp:152,
// 169, 192).
#include <cstdlib>
#include <cstring>

#include "engine.h"

#define DIFFUSE_DIE(fmt, ...)                                              \
    do {                                                                   \
        fprintf(stderr, "[diffuse] FATAL: " fmt "\n", ##__VA_ARGS__);      \
        exit(1);                                                           \
    } while (0)

// ---- C ABI ----
extern "C" int dfx_model_load(const char * path, dfx_model ** out) {
    if (!path || !out) {
        dfx_set_error("dfx_model_load: null argument");
        return DFX_ERR_ARG;
    }
    return engine_model_load(path, out);
}

extern "C" void dfx_model_free(dfx_model * m) { engine_model_free(m); }

extern "C" int dfx_model_hparams(const dfx_model * m, dfx_hparams * o) {
    if (!m || !o) return DFX_ERR_ARG;
    const diffuse_hparams & h = m->hparams;
    o->n_vocab = h.n_vocab;
    o->n_embd = h.n_embd;
    o->n_head = h.n_head;
    o->n_head_kv = h.n_head_kv;
    o->n_layer = h.n_layer;
    o->n_ff = h.n_ff;
    o->n_ctx_max = h.n_ctx_max;
    o->rope_theta = h.rope_theta;
    o->rms_norm_eps = h.rms_norm_eps;
    o->mask_token_id = h.mask_token_id;
    o->is_dream = m->is_dream ? 1 : 0;
    return DFX_OK;
}

extern "C" int dfx_context_new(const dfx_model * m, int n_ctx, dfx_context ** out) {
    if (!m || !out || n_ctx < 0) {
        dfx_set_error("dfx_context_new: bad argument");
        return DFX_ERR_ARG;
    }
    return engine_context_new(m, n_ctx, 1, out);
}

extern "C" void dfx_context_free(dfx_context * c) { engine_context_free(c); }

extern "C" int dfx_forward(dfx_context * c, const int32_t * tokens, int n, float * logits_out) {
    if (!c) return DFX_ERR_ARG;
    return engine_forward(c, tokens, n, logits_out);
}

extern "C" int dfx_forward_cached(dfx_context * c, const int32_t * active_tokens, const int32_t * active_pos,
                                  int n_active, int n_total, float * logits_out) {
    if (!c) return DFX_ERR_ARG;
    return engine_forward_cached(c, active_tokens, active_pos, n_active, n_total, logits_out);
}

extern "C" int dfx_generate(dfx_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                            const dfx_sampler_params * p, int32_t * out, dfx_gen_stats * stats) {
    if (!c || !p || (!prompt && n_prompt) || (!out && n_generate)) {
        dfx_set_error("dfx_generate: null argument");
        return DFX_ERR_ARG;
    }
    return engine_generate(c, prompt, n_prompt, n_generate, *p, out, stats, nullptr);
}

extern "C" int dfx_generate_trace(dfx_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                                  const dfx_sampler_params * p, int32_t * out, dfx_gen_stats * stats,
                                  int32_t * unmask_step) {
    if (!c || !p || (!prompt && n_prompt) || (!out && n_generate)) {
        dfx_set_error("dfx_generate_trace: null argument");
        return DFX_ERR_ARG;
    }
    return engine_generate(c, prompt, n_prompt, n_generate, *p, out, stats, nullptr, unmask_step);
}

extern "C" int dfx_context_set_attention(dfx_context * c, int mode) {
    if (!c || (mode != DFX_ATTN_SPLIT_BF16 && mode != DFX_ATTN_EXACT)) {
        dfx_set_error("dfx_context_set_attention: bad context or mode %d", mode);
        return DFX_ERR_ARG;
    }
    c->attn_mode = mode;
    return DFX_OK;
}

extern "C" int dfx_context_set_device_loop(dfx_context * c, int enable) {
    if (!c || enable < 0 || enable > 2) return DFX_ERR_ARG;
    c->device_loop = enable != 0;
    c->use_graphs = enable == 1;
    return DFX_OK;
}

extern "C" int dfx_context_profile(dfx_context * c, int enable) {
    if (!c) return DFX_ERR_ARG;
    return engine_profile(c, enable != 0);
}

extern "C" int dfx_context_profile_read(dfx_context * c, int wtype, int64_t * launches, double * ms, double * flops,
                                        double * bytes) {
    if (!c) return DFX_ERR_ARG;
    return engine_profile_read(c, wtype, 0, launches, ms, flops, bytes);
}

extern "C" int dfx_context_profile_read_rows(dfx_context * c, int wtype, int rows_class, int64_t * launches,
                                             double * ms, double * flops, double * bytes) {
    if (!c) return DFX_ERR_ARG;
    return engine_profile_read(c, wtype, rows_class, launches, ms, flops, bytes);
}

extern "C" int dfx_ar_forward(dfx_context * c, const int32_t * tokens, int n_new, int reset, int sliding_window,
                              float * logits_out) {
    if (!c) return DFX_ERR_ARG;
    return engine_ar_forward(c, tokens, n_new, reset != 0, sliding_window, logits_out);
}

extern "C" int dfx_ar_profile_layers(dfx_context * c, const int32_t * tokens, int n_tokens, int sliding_window,
                                     int n_skip, float * logits_out, float * impact_out, uint8_t * skip_out) {
    if (!c) return DFX_ERR_ARG;
    return engine_ar_profile(c, tokens, n_tokens, sliding_window, n_skip, logits_out, impact_out, skip_out);
}

extern "C" int dfx_ar_generate(dfx_context * c, const int32_t * prompt, int n_prompt, int max_tokens,
                               const dfx_ar_params * p, int32_t * out, int * n_out, dfx_ar_stats * stats,
                               dfx_ar_token_fn cb, void * user) {
    if (!c || !p || !out || !n_out) {
        dfx_set_error("dfx_ar_generate: null argument");
        return DFX_ERR_ARG;
    }
    *n_out = 0;
    std::vector<int32_t> toks;
    std::function<bool(int32_t, int)> f;
    if (cb) f = [cb, user](int32_t t, int pos) { return cb(t, pos, user) != 0; };
    const int rc = engine_ar_generate(c, prompt, n_prompt, max_tokens, *p, toks, stats, cb ? &f : nullptr);
    memcpy(out, toks.data(), toks.size() * 4);
    *n_out = (int)toks.size();
    return rc;
}

// ---- C++ API (include/diffuse.h) ----
diffuse_model * diffuse_model_load(const std::string & path, int /*n_threads*/) {
    diffuse_model * m = nullptr;
    if (engine_model_load(path, &m) != DFX_OK) DIFFUSE_DIE("%s", dfx_last_error());
    return m;
}

void diffuse_model_free(diffuse_model * model) { engine_model_free(model); }

const diffuse_hparams & diffuse_model_hparams(const diffuse_model * model) { return model->hparams; }

diffuse_context * diffuse_context_new(const diffuse_model * model, int n_ctx, int n_threads) {
    diffuse_context * c = nullptr;
    if (engine_context_new(model, n_ctx, n_threads, &c) != DFX_OK)
        DIFFUSE_DIE("failed to create context: %s", dfx_last_error());
    return c;
}

void diffuse_context_free(diffuse_context * ctx) { engine_context_free(ctx); }

bool diffuse_forward(diffuse_context * ctx, const int32_t * tokens, int n_tokens, float * logits_out) {
    if (engine_forward(ctx, tokens, n_tokens, logits_out) != DFX_OK) {
        DIFFUSE_LOG("forward failed: %s", dfx_last_error());
        return false;
    }
    return true;
}

std::vector<int32_t> diffuse_generate(diffuse_context * ctx, const std::vector<int32_t> & prompt_tokens,
                                      int n_generate, const diffuse_sampler_params & params,
                                      diffuse_step_callback callback) {
    dfx_sampler_params p;
    p.n_steps = params.n_steps;
    p.temperature = params.temperature;
    p.schedule = (int)params.schedule;
    p.remasking = (int)params.remasking;
    p.seed = params.seed;
    p.entropy_threshold = params.entropy_threshold;
    p.use_cache = params.use_cache ? 1 : 0;
    p.cache_refresh = params.cache_refresh;
    p.cache_keep_active = params.cache_keep_active;
    std::vector<int32_t> out((size_t)std::max(n_generate, 0));
    const int rc = engine_generate(ctx, prompt_tokens.data(), (int)prompt_tokens.size(), n_generate, p, out.data(),
                                   nullptr, callback ? &callback : nullptr);
    if (rc != DFX_OK) DIFFUSE_DIE("generation failed: %s", dfx_last_error());
    return out;
}

// ar_generate (src/ar-sampler.cpp:143-314); a failed forward ends the generation with
// what was generated so far, as the reference's decode loop does (src/ar-sampler.cpp:262-265),
// and a failed prefill is fatal (src/ar-sampler.cpp:199-209).
std::vector<int32_t> ar_generate(diffuse_context * ctx, const std::vector<int32_t> & prompt_tokens, int max_tokens,
                                 const ar_sampler_params & params, ar_token_callback callback) {
    dfx_ar_params p;
    p.temperature = params.temperature;
    p.top_p = params.top_p;
    p.top_k = params.top_k;
    p.repeat_penalty = params.repeat_penalty;
    p.repeat_last_n = params.repeat_last_n;
    p.seed = params.seed;
    p.layer_skip = params.layer_skip;
    p.sliding_window = params.sliding_window;
    std::vector<int32_t> out;
    const std::function<bool(int32_t, int)> cb = callback;
    const int rc = engine_ar_generate(ctx, prompt_tokens.data(), (int)prompt_tokens.size(), max_tokens, p, out,
                                      nullptr, cb ? &cb : nullptr);
    if (rc != DFX_OK) {
        if (out.empty()) DIFFUSE_DIE("ar_generate: prefill failed: %s", dfx_last_error());
        DIFFUSE_LOG("ar_generate: decode failed: %s", dfx_last_error());
    }
    return out;
}

// Speculative decoding (src/ar-speculative.cpp) is not built; the symbol exists so programs
// written against diffuse.h link.
std::vector<int32_t> ar_speculative_generate(diffuse_context *, diffuse_context *, const std::vector<int32_t> &, int,
                                             const ar_spec_params &, ar_token_callback, ar_spec_stats *) {
    DIFFUSE_LOG("ar_speculative_generate: the autoregressive path is not available in this build");
    return {};
}
