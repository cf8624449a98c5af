#pragma once
// diffuse.h — public C++ API of the MI355X denoising engine.
//
// Declaration-compatible with diffuse-cpp's include/diffuse.h (lines 1-159): the
// same names, member order, defaults and enum order, so the reference's callers
// (tools/main-cli.cpp, tools/main-bench.cpp, tools/dump-logits.cpp,
// tests/test-forward.cpp) compile and link against this library unchanged.
// The implementation runs the forward pass and the sampler on one gfx950 GPU;
// the C ABI underneath is in dfx.h.

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

struct diffuse_model;
struct diffuse_context;

// Model shape, filled from GGUF metadata by diffuse_model_load.
struct diffuse_hparams {
    uint32_t n_vocab      = 0;
    uint32_t n_embd       = 0;
    uint32_t n_head       = 0;
    uint32_t n_head_kv    = 0;         // equals n_head without GQA
    uint32_t n_layer      = 0;
    uint32_t n_ff         = 0;
    uint32_t n_ctx_max    = 0;
    float    rope_theta   = 500000.0f;
    float    rms_norm_eps = 1e-5f;
    uint32_t mask_token_id = 0;

    uint32_t n_embd_head() const { return n_head > 0 ? n_embd / n_head : 0; }
};

// Unmasking schedule: how many masked positions to reveal per step.
enum class diffuse_schedule {
    COSINE,
    LINEAR,
};

// Which masked positions to reveal first.
enum class diffuse_remasking {
    LOW_CONFIDENCE,   // highest top-1 logit first
    RANDOM,           // shuffled with the sampler seed
    ENTROPY_EXIT,     // lowest entropy first; also reveals every position below the threshold
    MASKGIT_PLUS,     // highest top-1 logit first
    TOPK_MARGIN,      // largest top1 - top2 logit margin first
};

struct diffuse_sampler_params {
    int      n_steps     = 32;
    float    temperature = 0.0f;          // 0 = argmax
    diffuse_schedule   schedule   = diffuse_schedule::COSINE;
    diffuse_remasking  remasking  = diffuse_remasking::LOW_CONFIDENCE;
    uint32_t seed       = 42;
    float    entropy_threshold = 1.5f;    // ENTROPY_EXIT threshold (nats)
    bool     use_cache   = true;          // inter-step KV cache
    int      cache_refresh    = 0;        // full forward every N steps (0 = never)
    int      cache_keep_active = 0;       // keep changed positions active N more steps
};

struct diffuse_params {
    std::string model_path;
    std::string prompt;
    int         n_generate  = 128;
    int         n_threads   = 4;
    diffuse_sampler_params sampler;
};

// Called after every denoising step with the whole (prompt + generated) sequence.
using diffuse_step_callback = std::function<void(
    int step, int total_steps, const std::vector<int32_t> & tokens)>;

// ---- model ----
diffuse_model * diffuse_model_load(const std::string & path, int n_threads);
void            diffuse_model_free(diffuse_model * model);
const diffuse_hparams & diffuse_model_hparams(const diffuse_model * model);

// ---- context: device activations, KV cache and logits for one sequence ----
diffuse_context * diffuse_context_new(const diffuse_model * model, int n_ctx, int n_threads);
void              diffuse_context_free(diffuse_context * ctx);

// ---- one forward pass: tokens[n_tokens] -> logits_out[n_tokens * n_vocab] ----
bool diffuse_forward(diffuse_context * ctx,
                     const int32_t * tokens, int n_tokens,
                     float * logits_out);

// ---- full denoising loop; returns the n_generate generated ids ----
std::vector<int32_t> diffuse_generate(
    diffuse_context * ctx,
    const std::vector<int32_t> & prompt_tokens,
    int n_generate,
    const diffuse_sampler_params & params,
    diffuse_step_callback callback = nullptr);

// ---- autoregressive API (declared for link compatibility; not on the GPU path) ----
struct ar_sampler_params {
    float    temperature    = 0.0f;
    float    top_p          = 0.9f;
    int      top_k          = 40;
    float    repeat_penalty = 1.1f;
    int      repeat_last_n  = 64;
    uint32_t seed           = 42;
    int      layer_skip     = 0;
    int      sliding_window = 0;
};

using ar_token_callback = std::function<bool(int32_t token, int pos)>;

std::vector<int32_t> ar_generate(
    diffuse_context * ctx,
    const std::vector<int32_t> & prompt_tokens,
    int max_tokens,
    const ar_sampler_params & params,
    ar_token_callback callback = nullptr);

struct ar_spec_params {
    int K = 5;
    int layer_skip = 0;
    int sliding_window = 0;
};

struct ar_spec_stats {
    int total_draft_tokens  = 0;
    int total_accepted      = 0;
    int total_generated     = 0;
    int total_target_batches = 0;
    int total_target_decodes = 0;
    int total_fast_rejects   = 0;
    double prefill_ms = 0;
    double decode_ms  = 0;

    float acceptance_rate() const {
        return total_draft_tokens > 0 ? (float)total_accepted / total_draft_tokens : 0.0f;
    }
    float tokens_per_target_call() const {
        int calls = total_target_batches + total_target_decodes;
        return calls > 0 ? (float)total_generated / calls : 1.0f;
    }
};

std::vector<int32_t> ar_speculative_generate(
    diffuse_context * target_ctx,
    diffuse_context * draft_ctx,
    const std::vector<int32_t> & prompt_tokens,
    int max_tokens,
    const ar_spec_params & params,
    ar_token_callback callback = nullptr,
    ar_spec_stats * stats_out = nullptr);
