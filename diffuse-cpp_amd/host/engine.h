// engine.h — internal structures of the gfx950 engine behind diffuse.h / dfx.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdio>
#include <functional>
#include <string>
#include <vector>

#include "dfx.h"
#include "dfx_epi.h"
#include "diffuse.h"

#define DIFFUSE_LOG(fmt, ...) fprintf(stderr, "[diffuse] " fmt "\n", ##__VA_ARGS__)

// Internal kernel entry points with row maps (k_gemm.hip, k_quant.hip, k_sampler.hip).
// epi: null (plain), DFX_EPI_SWIGLU (gate|up rows interleaved in blocks of 16: y[m][f] =
// silu(gate) * up with row stride ldy >= N / 2; no bias, residual or row map) or DFX_EPI_ROPE
// (Q|K|V columns rotated and stored into q_out and the caches; bias allowed, no residual, row
// map or y).
int dfx_gemm_ex(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, const float * bias,
                const float * residual, float * y, int64_t ldy, const int32_t * ymap, void * ws, size_t ws_bytes,
                void * stream, int * n_partials, const dfx_epi * epi = nullptr);
int dfx_rmsnorm_convert_ex(int wtype, const float * x, const int32_t * xmap, const float * w, int64_t M, int64_t K,
                           float eps, void * act, void * stream);
// RMSNorm + conversion of x after adding a deferred split-K result: row r (= xmap[m] or m)
// becomes x[r] = (sum over s < n_part of part[s][r]) + x[r] (written back), then is
// normalised and converted like dfx_rmsnorm_convert_ex.  part rows are K floats, slices
// part_rows rows apart.
int dfx_rmsnorm_convert_add(int wtype, float * x, const int32_t * xmap, const float * part, int n_part,
                            int64_t part_rows, const float * w, int64_t M, int64_t K, float eps, void * act,
                            void * stream);
extern "C" void dfx_set_error(const char * fmt, ...);

// A weight matrix in the device layout of dfx.h: rows x cols, rows of super-blocks.
struct dev_matrix {
    int       type = -1;          // storage type (DFX_TYPE_*)
    int64_t   rows = 0, cols = 0;
    uint8_t * data = nullptr;
};

// Matrices that read the same activations (Q|K|V, gate|up), stacked by rows in
// one allocation.  When every part has the same type one GEMM covers them all.
struct proj_group {
    std::vector<dev_matrix> parts;
    std::vector<int64_t>    col_off;    // output column of each part
    int64_t                 n_out = 0;
    bool                    fused = false;
    dev_matrix              all;        // valid when fused
    float *                 bias = nullptr;   // [n_out] f32 or null
    // gate|up fused with rows interleaved in blocks of 16 (16 gate rows, then the 16 up rows
    // of the same F-indices): its GEMM applies SwiGLU in the epilogue (DFX_EPI_SWIGLU)
    bool                    swiglu = false;
    // Q|K|V fused with the rows of every Q and K head permuted in blocks of 32 (16 dims of the
    // first half, then the 16 dims hd/2 later that they rotate with): its GEMM applies RoPE and
    // stores Q and the K/V cache in the epilogue (DFX_EPI_ROPE)
    bool                    rope = false;
};

struct dev_layer {
    float *    attn_norm = nullptr;   // f32 [n_embd]
    float *    ffn_norm = nullptr;
    proj_group qkv;                   // output [q | k | v]
    dev_matrix o;
    proj_group gu;                    // output [gate | up]
    dev_matrix down;
};

struct diffuse_model {
    diffuse_hparams hparams;
    std::string     model_type;
    bool            is_dream = false;
    dev_matrix      tok_embd;        // gather table (F32 tables stay F32)
    dev_matrix      output;          // vocab head in GEMM layout
    float *         output_norm = nullptr;
    std::vector<dev_layer> layers;
    std::vector<void *>    allocs;
    size_t          device_bytes = 0;
};

struct diffuse_context {
    const diffuse_model * model = nullptr;
    int          n_ctx = 0;
    int          n_threads = 1;
    hipStream_t  stream = nullptr;
    int          cap = 0;            // rows the device buffers hold

    float *      x = nullptr;        // [cap][d]       residual stream
    uint8_t *    act = nullptr;      // converted GEMM input for up to cap rows of max(d, F)
    float *      qkv = nullptr;      // [cap][d + 2 dkv]
    float *      qr = nullptr;       // [cap][d]       roped queries
    float *      att = nullptr;      // [cap][d]
    float *      gu = nullptr;       // [cap][2F]
    float *      logits = nullptr;   // [cap][V]       per position
    float *      kc = nullptr;       // [L][cap][dkv]        inter-step key cache
    float *      vc = nullptr;       // [L][Hkv][hd][cap]    inter-step value cache, transposed
    float *      rope_tab = nullptr; // [cap][hd/2][2]
    // The six index arrays of a step are slots 0..5 of one allocation d_ints [6][cap],
    // staged in the same order in h_pin, so one copy uploads them all.
    int32_t *    d_ints = nullptr;
    int32_t *    d_tok = nullptr;    // slot 0: tokens of this pass
    int32_t *    d_pos = nullptr;    // slot 1: positions of this pass
    int32_t *    d_hrows = nullptr;  // slot 2: pass rows that need logits
    int32_t *    d_hmap = nullptr;   // slot 3: logits row of each of them
    int32_t *    d_srows = nullptr;  // slot 4: logits rows scanned by the sampler
    int32_t *    d_spos = nullptr;   // slot 5: masked position of each scanned row
    void *       ws = nullptr;       // split-K workspace (also the half tiles' chunk totals)
    size_t       ws_bytes = 0;
    int32_t *    tile_cnt = nullptr; // completion counters of half-tile GEMM launches (kept zero)
    dfx_row_stat *  d_stats = nullptr;
    // Sampler results, one allocation d_out = [cand: cap][order: cap][n_unmask], read back
    // with one copy into the pinned h_out.
    void *       d_out = nullptr;
    dfx_candidate * d_cand = nullptr;
    int32_t *    d_order = nullptr;
    int32_t *    d_nun = nullptr;
    void *       h_out = nullptr;
    size_t       out_bytes = 0;
    int32_t *    h_pin = nullptr;    // pinned staging, 8 * cap int32
    hipEvent_t   ev0 = nullptr, ev1 = nullptr, ev2 = nullptr;
    int          attn_mode = DFX_ATTN_EXACT;   // dfx_attention_ex mode of the forward passes
    int          kv_valid = 0;       // positions 0..kv_valid-1 of the cache hold a full forward's K/V

    // Device-resident denoising loop (temperature 0, every policy but RANDOM): the sequence
    // state lives in d_state [5][cap] = seq | prev | masked | lastc | ustep; per step, the
    // prepare kernel's counts d_counts [steps][4] and the unmask count d_hist [steps],
    // copied to the pinned h_hist as each step ends (event ev_unmask[step]).
    bool         device_loop = true;
    // The layer stack of a step captured once per (rows, keys, attention mode) as a HIP graph
    // and replayed (kernels only: no memset or copy nodes); dropped with the buffers.
    struct layers_graph { int M, n_keys, mode, pending; hipGraphExec_t exec; };
    bool         use_graphs = true;
    std::vector<layers_graph> graphs;
    int32_t *    d_state = nullptr;
    int32_t *    d_counts = nullptr;
    int32_t *    d_hist = nullptr;
    int32_t *    h_hist = nullptr;
    int          steps_cap = 0;
    std::vector<hipEvent_t> ev_unmask, ev_fwd0, ev_fwd1;

    // Autoregressive state (src/ar-cache.h): positions 0..ar_past-1 of kc / vc hold the keys
    // and values of the tokens passed so far (layers in ar_skip keep stale rows).
    int          ar_past = 0;
    std::vector<uint8_t> ar_skip;    // [L] layers left out of non-profiling passes
    float *      x_prev = nullptr;   // [cap][d] layer input, kept while profiling
    double *     d_imp = nullptr;    // [L][cap] per-row layer impact sums
    int32_t *    d_ar = nullptr;     // [4] zeros (head row / map of a one-row pass), then the
                                     // greedy decode state of dfx_ar_greedy [4 + ar_ring]
    int          ar_ring = 0;        // ring capacity of d_ar
    float *      h_row = nullptr;    // pinned [V]: one logits row for the host sampler

    // Optional per-GEMM timing: a pair of events around every GEMM launch on `stream`.
    struct gemm_rec { hipEvent_t a, b; int type; int64_t M; double flops, bytes; };
    bool                  prof = false;
    std::vector<gemm_rec> prof_pending;      // launched, not yet read
    std::vector<hipEvent_t> prof_pool;       // reusable events
    struct prof_total { long launches = 0; double ms = 0, flops = 0, bytes = 0; };
    // by row class (0 every launch, 1 M > 96, 2 M <= 96, 3 M >= 288) and weight type id
    prof_total            prof_tot[4][32];
};

// Options of one forward pass (the autoregressive graph of src/ar-graph.cpp:27-260):
// causal attention, skipped layers, layer-impact profiling and index arrays other than
// the context's d_tok / d_pos / d_hrows / d_hmap.
struct pass_opts {
    int64_t         q_pos0 = -1;         // >= 0: causal, query row m at position q_pos0 + m
    int             window = 0;          // causal: keys within this many positions (0 = all)
    const uint8_t * skip = nullptr;      // [L] host: nonzero = layer left out
    double *        impact_rows = nullptr;   // device [L][M]: per-row impact sums (no split-K deferral)
    const int32_t * tok = nullptr;       // device index arrays replacing the context's
    const int32_t * pos = nullptr;
    const int32_t * hrows = nullptr;
    const int32_t * hmap = nullptr;
};

// engine.cpp internals shared with ar.cpp
int  engine_hip_ok(hipError_t e, const char * what);
int  engine_reserve(diffuse_context * c, int N);
int  engine_pass(diffuse_context * c, int M, int n_keys, int n_head, const pass_opts & o);
int  engine_check_tiles(diffuse_context * c);   // after a synchronised pass: half-tile XCD check
void engine_prof_collect(diffuse_context * c);

// ar.cpp (src/ar-graph.cpp, src/ar-sampler.cpp)
int  engine_ar_forward(diffuse_context * c, const int32_t * tokens, int n_new, bool reset, int window,
                       float * logits_out);
int  engine_ar_profile(diffuse_context * c, const int32_t * tokens, int n, int window, int n_skip, float * logits_out,
                       float * impact_out, uint8_t * skip_out);
int  engine_ar_generate(diffuse_context * c, const int32_t * prompt, int n_prompt, int max_tokens,
                        const dfx_ar_params & p, std::vector<int32_t> & out, dfx_ar_stats * stats,
                        const std::function<bool(int32_t, int)> * cb);

// model.cpp
int  engine_model_load(const std::string & path, diffuse_model ** out);
void engine_model_free(diffuse_model * m);

// engine.cpp
int  engine_context_new(const diffuse_model * m, int n_ctx, int n_threads, diffuse_context ** out);
void engine_context_free(diffuse_context * c);
int  engine_forward(diffuse_context * c, const int32_t * tokens, int n, float * logits_out);
int  engine_forward_cached(diffuse_context * c, const int32_t * active_tokens, const int32_t * active_pos, int n_active,
                           int n_total, float * logits_out);
int  engine_profile(diffuse_context * c, bool enable);
int  engine_profile_read(diffuse_context * c, int wtype, int rows_class, int64_t * launches, double * ms,
                         double * flops, double * bytes);
int  engine_generate(diffuse_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                     const dfx_sampler_params & p, int32_t * out, dfx_gen_stats * stats,
                     const diffuse_step_callback * callback, int32_t * unmask_step = nullptr);
