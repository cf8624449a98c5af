/*
 * oracle.h — CPU restatement of diffuse-cpp's denoising forward pass and sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP path
 * and the timed CPU baseline; nothing in the product links, loads or calls it.
 *
 * What it restates (reference file:line, under diffuse-cpp):
 *   - forward graph, full and cached:   src/diffuse-graph.cpp:11-160, 395-593
 *   - inter-step cache bookkeeping:     src/diffuse-cache.h:79-146
 *   - schedule, entropy, sampler loop:  src/diffuse-sampler.cpp:12-370
 *   - hparams / sampler defaults:       include/diffuse.h:15-55
 *   - GGML CPU op semantics the graph relies on (GGML is an empty submodule in the
 *     reference, see .gitmodules:1-3; the semantics below are restated from
 *     GGML's published source, README.md:7 pins "GGML v0.9.8"):
 *       block codecs Q8_0 / Q4_K / Q6_K / F16, activation quantisation to the
 *       weight's vec_dot_type (Q8_K for K-quants, Q8_0 for Q8_0, F16 for F16),
 *       integer block dot products, rms_norm (double sum), NEOX rope (theta by
 *       repeated multiplication), soft_max (double sum), silu = x/(1+exp(-x)).
 *
 * Parity status per function is recorded in the header comment of oracle.cpp.
 */
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (ggml.h enum ggml_type). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
};

/* ---- codecs ---- */
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
void     orc_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n);
void     orc_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n);
int64_t  orc_block_size(int type);             /* elements per block */
int64_t  orc_type_size(int type);              /* bytes per block    */
int64_t  orc_row_size(int type, int64_t n);    /* bytes for n elements, -1 if n not a block multiple */
int      orc_dequant_row(int type, const void * x, float * y, int64_t n);
void     orc_quantize_row_q8_K(const float * x, void * y, int64_t n);   /* activation side */
void     orc_quantize_row_q8_0(const float * x, void * y, int64_t n);   /* activation side */
/* One vec_dot: weight row (type) against an activation row already converted to
 * the weight's vec_dot_type.  Returns 0 on success. */
int      orc_vec_dot(int wtype, int64_t n, const void * w_row, const void * a_row, float * out);

/* ---- ops (row-major: X[M][K], Y[M][N]) ---- */
/* Y[m][n] = sum_k W[n][k] * X[m][k] with GGML mul_mat semantics (X converted to
 * the vec_dot_type of W first). W rows are ne0=K contiguous blocks. */
int  orc_mul_mat(int wtype, const void * W, int64_t N, int64_t K,
                 const float * X, int64_t M, float * Y, int n_threads);
void orc_rms_norm_mul(const float * x, const float * w, int64_t M, int64_t K, float eps, float * y);
/* cos/sin table for NEOX rope: tab[(p*half + i)*2 + {0,1}] for positions 0..n_pos-1 */
void orc_rope_table(int n_pos, int head_dim, float theta_base, float * tab);
void orc_rope_neox(float * x, int64_t M, int n_heads, int head_dim, const int32_t * pos,
                   const float * tab);
float orc_silu(float x);
/* Bidirectional attention, q [M][H][hd], k/v [n_keys][H][hd] (heads already expanded), out [M][H*hd]. */
void  orc_attention(const float * q, const float * k, const float * v, int M, int n_keys, int H, int hd,
                    float * out, int n_threads);

/* ---- model ---- */
typedef struct {
    int         type;        /* ORC_TYPE_* */
    int64_t     ne0, ne1;    /* ne0 = input dim (contiguous), ne1 = rows */
    const void * data;       /* NULL = absent (optional biases) */
} orc_tensor;

typedef struct {
    orc_tensor attn_norm, wq, wk, wv, wo, bq, bk, bv, ffn_norm, ffn_gate, ffn_up, ffn_down;
} orc_layer;

typedef struct {
    uint32_t n_vocab, n_embd, n_head, n_head_kv, n_layer, n_ff;
    float    rope_theta, rms_norm_eps;
    uint32_t mask_token_id;
    int      is_dream;       /* model_type == "dream": shifted logits in the sampler */
    orc_tensor tok_embd, output_norm, output;
    const orc_layer * layers;  /* n_layer entries */
} orc_model;

/* Per-layer K/V cache, reference layout (src/diffuse-cache.h:12-26):
 * k[layer][pos][n_head][head_dim] fp32 after RoPE and GQA expansion. */
typedef struct {
    int     n_tokens;
    float * k;               /* n_layer * n_tokens * n_head * head_dim */
    float * v;
} orc_kv;

/* Full forward over n_tokens positions 0..n-1 (src/diffuse-graph.cpp:11-160,
 * 309-379). logits: [n][n_vocab]. If kv != NULL its K/V are filled. */
int orc_forward_full(const orc_model * m, const int32_t * tokens, int n, float * logits,
                     orc_kv * kv, int n_threads);

/* Cached forward (src/diffuse-graph.cpp:395-673): active rows only; keys are
 * [cached ‖ active] in that order; active K/V written back into kv afterwards. */
int orc_forward_cached(const orc_model * m, const int32_t * active_tokens,
                       const int32_t * active_pos, int n_active, int n_total,
                       orc_kv * kv, const int32_t * cached_pos, float * logits, int n_threads);

/* ---- sampler ---- */
enum { ORC_SCHED_COSINE = 0, ORC_SCHED_LINEAR = 1 };
enum { ORC_REMASK_LOW_CONFIDENCE = 0, ORC_REMASK_RANDOM = 1, ORC_REMASK_ENTROPY_EXIT = 2,
       ORC_REMASK_MASKGIT_PLUS = 3, ORC_REMASK_TOPK_MARGIN = 4 };

typedef struct {
    int      n_steps;
    float    temperature;
    int      schedule;
    int      remasking;
    uint32_t seed;
    float    entropy_threshold;
    int      use_cache;
    int      cache_refresh;
    int      cache_keep_active;
} orc_sampler_params;

int   orc_tokens_to_unmask(int step, int total_steps, int total_masked, int schedule);
float orc_entropy(const float * row, int n_vocab);
/* argmax (strict >, lowest index on ties) + second-best as in the reference loop */
void  orc_top2(const float * row, int n_vocab, int * best, float * best_val, float * second_val);

typedef struct { int32_t pos, token; float confidence, entropy; } orc_candidate;
/* Orders candidates in place as the remasking policy does (ENTROPY_EXIT: entropy
 * ascending; LOW_CONFIDENCE / MASKGIT_PLUS / TOPK_MARGIN: confidence descending).
 * Ties are broken by position ascending (std::sort leaves them unspecified).
 * Returns the number to unmask for ENTROPY_EXIT given n_sched, else n_sched capped. */
int   orc_order_candidates(orc_candidate * c, int n, int remasking, float entropy_threshold,
                           int n_sched);

typedef struct {
    int    actual_steps;
    int    rows_per_step[256];   /* active rows of each step's forward */
    int    unmasked_per_step[256];
} orc_gen_stats;

/* diffuse_sample restated (src/diffuse-sampler.cpp:60-370). out: n_generate ids. */
int orc_generate(const orc_model * m, const int32_t * prompt, int n_prompt, int n_generate,
                 const orc_sampler_params * p, int32_t * out, orc_gen_stats * stats, int n_threads);

/* ---- autoregressive path (src/ar-graph.cpp, src/ar-cache.h, src/ar-sampler.cpp) ---- */
/* Causal attention: key n visible to query m when kpos[n] <= qpos[m] and, with window > 0,
 * qpos[m] - kpos[n] < window (src/ar-graph.cpp:70-88). */
void orc_attention_causal(const float * q, const float * k, const float * v, int M, int n_keys, int H, int hd,
                          const int32_t * qpos, const int32_t * kpos, int window, float * out, int n_threads);

/* Append-only cache, k/v [n_layer][n_ctx_max][n_head*head_dim] after RoPE and GQA
 * expansion; positions 0..n_past-1 valid. */
typedef struct {
    int       n_ctx_max, n_past, sliding_window;
    float *   k;
    float *   v;
    uint8_t * skip;     /* [n_layer] layers left out of non-profiling passes */
    float *   impact;   /* [n_layer] filled by a profiling pass */
} orc_ar_cache;

/* ar_sampler_params (include/diffuse.h:96-107). */
typedef struct {
    float    temperature, top_p;
    int      top_k;
    float    repeat_penalty;
    int      repeat_last_n;
    uint32_t seed;
    int      layer_skip, sliding_window;
} orc_ar_params;

/* ar_forward_impl (src/ar-graph.cpp:262-399): n_new tokens at positions n_past..; logits
 * [n_new][V], or the last row's only; profile = the layer-impact pass of
 * ar_profile_layers (every layer runs, impacts written). */
int orc_ar_forward(const orc_model * m, const int32_t * tokens, int n_new, orc_ar_cache * c, float * logits,
                   int last_only, int profile, int n_threads);
int orc_ar_choose_skip(const float * impact, int n_layer, int n_skip, uint8_t * skip);

typedef struct orc_rng orc_rng;   /* std::mt19937 */
orc_rng * orc_rng_new(uint32_t seed);
void      orc_rng_free(orc_rng * r);
/* sample_token (src/ar-sampler.cpp:99-140) on a copy of row. */
int orc_ar_sample(const float * row, int V, const orc_ar_params * p, const int32_t * recent, int n_recent,
                  orc_rng * rng);
/* ar_generate (src/ar-sampler.cpp:143-314): out gets up to max(max_tokens, 1) ids, *n_out how many;
 * skip_out (n_layer bytes, optional) the skipped-layer mask chosen by profiling. */
int orc_ar_generate(const orc_model * m, const int32_t * prompt, int n_prompt, int max_tokens,
                    const orc_ar_params * p, int32_t * out, int * n_out, uint8_t * skip_out, int n_threads);

#ifdef __cplusplus
}
#endif
