/*
 * dfx.h — C ABI of the MI355X (gfx950) denoising path.
 *
 * Plain C types only: device pointers, sizes, an opaque stream handle
 * (hipStream_t passed as void*, NULL = the library's default stream).
 * Every entry point returns 0 on success or a negative DFX_ERR_* code;
 * dfx_last_error() gives the message of the most recent failure on the
 * calling thread.  No entry point allocates device memory except the ones
 * named *_alloc / *_new / *_load.
 *
 * Two levels:
 *   1. Kernel entry points (dfx_dequant ... dfx_select): one HIP kernel (or a
 *      fixed short sequence) on caller-owned device buffers.  Each replaces a
 *      GGML CPU op of the reference graph, cited per function.
 *   2. Model / context entry points (dfx_model_load ... dfx_generate): the
 *      C form of diffuse-cpp's public API (include/diffuse.h:71-91), for FFI
 *      callers that cannot bind C++ (std::string / std::vector / std::function).
 *      The C++ API in diffuse.h is implemented on top of these.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ---- */
#define DFX_OK               0
#define DFX_ERR_ARG         -1   /* bad argument / shape */
#define DFX_ERR_UNSUPPORTED -2   /* tensor type or shape the kernels do not handle */
#define DFX_ERR_HIP         -3   /* HIP runtime error */
#define DFX_ERR_IO          -4   /* file could not be opened / read */
#define DFX_ERR_FORMAT      -5   /* malformed GGUF or missing key / tensor */
#define DFX_ERR_OOM         -6   /* device allocation failed */

/* ---- tensor types: GGML ids, as stored in GGUF ---- */
enum {
    DFX_TYPE_F32  = 0,
    DFX_TYPE_F16  = 1,
    DFX_TYPE_Q8_0 = 8,
    DFX_TYPE_Q4_K = 12,
    DFX_TYPE_Q6_K = 14,
    DFX_TYPE_Q8_K = 15,
};

const char * dfx_last_error(void);

/* ---- device plumbing (lets FFI callers run kernels without another runtime) ---- */
int dfx_device_count(int * n);
int dfx_malloc(void ** ptr, size_t bytes);
int dfx_free(void * ptr);
int dfx_memcpy_h2d(void * dst, const void * src, size_t bytes, void * stream);
int dfx_memcpy_d2h(void * dst, const void * src, size_t bytes, void * stream);
int dfx_memcpy_d2d(void * dst, const void * src, size_t bytes, void * stream);
int dfx_memset(void * dst, int value, size_t bytes, void * stream);
int dfx_stream_create(void ** stream);
int dfx_stream_destroy(void * stream);
int dfx_stream_sync(void * stream);
/* Elapsed ms between two points on a stream: start records, stop records + waits. */
int dfx_timer_start(void ** timer, void * stream);
int dfx_timer_stop(void * timer, void * stream, float * ms);

/* ---- device weight layout ----
 * Weights live in HBM as rows of 256-element super-blocks, each 16-byte aligned:
 *   Q4_K  144 B  GGML block_q4_K as is                      {d, dmin, scales[12], qs[128]}
 *   Q6_K  224 B  GGML block_q6_K (210 B) + 14 zero bytes    {ql[128], qh[64], scales[16], d, pad}
 *   Q8_0  272 B  eight GGML block_q8_0 regrouped            {d[8], qs[8][32]}
 *   F16   512 B  256 halves
 *   F32  1024 B  256 floats
 * dfx_repack_rows converts GGUF bytes (n_rows x n_cols, GGML layout) into this
 * layout on the host.  n_cols must be a multiple of 256.
 */
int64_t dfx_device_row_bytes(int type, int64_t n_cols);   /* -1 if unsupported */
int     dfx_device_type(int gguf_type);                   /* storage type used for a GGUF type */
int dfx_repack_rows(int gguf_type, const void * src, int64_t n_rows, int64_t n_cols, void * dst);

/* ---- kernel entry points ---- */

/* Dequantise n_rows x n_cols of a device-layout weight to f32 (bit-exact with
 * GGML dequantize_row_*; used by get_rows at src/diffuse-graph.cpp:43). */
int dfx_dequant(int type, const void * w, int64_t n_rows, int64_t n_cols, float * out, void * stream);

/* Embedding gather: x[m][:] = dequant(table row tokens[m]) as f32
 * (ggml_get_rows, src/diffuse-graph.cpp:43, 197, 433). */
int dfx_embed(int type, const void * table, int64_t n_embd, const int32_t * tokens, int64_t M,
              float * x, void * stream);

/* Activation conversion to the weight's vec_dot_type, the way GGML's mul_mat
 * converts src1 before its dot products (Q8_K blocks of 256 for Q4_K/Q6_K, Q8_0
 * blocks of 32 for Q8_0, F16 for F16, F32 kept for F32).  The result goes to an
 * activation buffer of dfx_act_bytes(wtype, M, K) bytes:
 *   q   f16 [M][K]      int8 quants as exact f16 integers (F16: the f16 values;
 *                       F32 weights: the f32 values themselves, f32 [M][K])
 *   d   f32 [M][K/blk]  block scales (Q8_K: blk 256; Q8_0: blk 32, the f16 scale)
 *   bs  f16 [M][K/16]   Q8_K only: sums of q over 16 elements
 * each part starting at a 256-byte boundary, in this order.  For Q4_K and Q6_K
 * weights q holds ceil(M/32)*32 rows in the GEMM's matrix-core operand order: each
 * 128-element K step of a 32-row tile is 8 KB of consecutive memory (the order is
 * spelled out next to act_frag_off in the library's device header). */
size_t dfx_act_bytes(int wtype, int64_t M, int64_t K);
int dfx_act_convert(int wtype, const float * x, int64_t M, int64_t K, void * act, void * stream);

/* y = rms_norm(x) * w, then converted as dfx_act_convert (src/diffuse-graph.cpp:51-58,
 * 127-134, 146-153). */
int dfx_rmsnorm_convert(int wtype, const float * x, const float * w, int64_t M, int64_t K, float eps,
                        void * act, void * stream);

/* s = silu(g) * u converted for the down projection (src/diffuse-graph.cpp:136-139).
 * gu is the [M][2F] output of the fused gate|up GEMM: row m holds gate then up. */
int dfx_swiglu_convert(int wtype, const float * gu, int64_t M, int64_t F, void * act, void * stream);

/* GEMM (src/diffuse-graph.cpp:61-63, 122, 136-140, 154):
 *   y[m][n] = sum_k x[m][k] * W[n][k]  (+ bias[n])  (+ residual[m][n])
 * on the matrix cores, or for one or two rows of Q4_K / Q6_K weights (and up to four rows of a
 * matrix of at most 4096 x 4096) on integer dot products over the int8 copy that the conversions
 * keep for up to four rows.
 * act: the converted activations of x (dfx_*_convert with the same wtype and the same M: the
 * layout depends on M);
 * W: device-layout [N][K]; y f32 [M][N].  For Q4_K / Q6_K / Q8_0 the result
 * equals GGML's integer block dot products scaled and summed in a fixed K order
 * (chunks of 2048 elements, chunk sums added in order), i.e. the CPU mul_mat value
 * for value.  residual may alias y (in-place residual add).
 * ws: split-K workspace of dfx_gemm_ws_bytes(M, N, K) bytes, or NULL (no split). */
size_t dfx_gemm_ws_bytes(int64_t M, int64_t N, int64_t K);
int dfx_gemm(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
             const float * bias, const float * residual, float * y, void * ws, void * stream);

/* dfx_gemm on Q4_K weights whose column tiles may each split their K range (two 2048-element
 * chunks) over two workgroups of one launch, the later of which adds the two chunk totals in
 * chunk order and applies the epilogue: the same bits as dfx_gemm, with the workgroups spread
 * more evenly over the CUs where a whole-tile grid would leave some with one workgroup and
 * others with two (a scheduling form of the same mul_mat; no counterpart in the reference).
 * Other weight types, shapes and row counts run as dfx_gemm.  ws: dfx_gemm_ws_bytes(M, N, K)
 * bytes (2*M*N floats used).  tile_cnt: dfx_gemm_tile_cnt_bytes(M, N) bytes, all zero before
 * the first call; every call leaves them zero except tile_cnt[1], which a call sets to 1 when
 * the two halves of a tile ran on different XCDs (the handover of their chunk totals assumes
 * one L2, i.e. the round-robin workgroup-to-XCD dispatch): the results of such a call are
 * invalid.  Callers check tile_cnt[1] after the call and clear it.  Calls sharing tile_cnt or
 * ws must not overlap. */
size_t dfx_gemm_tile_cnt_bytes(int64_t M, int64_t N);
int dfx_gemm_counted(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                     const float * bias, const float * residual, float * y, void * ws, int32_t * tile_cnt,
                     void * stream);

/* GEMM of a fused gate|up matrix with the SwiGLU of the FFN (src/diffuse-graph.cpp:136-139:
 * silu(gate) * up of two ggml_mul_mat results) applied to the accumulators before they are
 * stored.  W: device-layout [N][K] whose rows are gate and up interleaved in blocks of 16
 * (rows 32j..32j+15 = gate rows 16j..16j+15, rows 32j+16..32j+31 = the up rows of the same
 * indices), N = 2F a multiple of 32.  y[m][f] (row stride ldy >= F) = silu(g) * u with g, u
 * the dfx_gemm values of gate row f and up row f (same K order, same split-K choice) and
 * silu(x) = x / (1 + exp(-x)) as GGML's f32 silu: the same bits as dfx_gemm followed by
 * dfx_swiglu_convert's products, without writing or reading the [M][2F] gate|up block.
 * ws: as in dfx_gemm. */
int dfx_gemm_swiglu(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y,
                    int64_t ldy, void * ws, void * stream);

/* GEMM of a fused Q|K|V matrix with the NEOX RoPE and the cache store of dfx_rope_store
 * (src/diffuse-graph.cpp:61-79, 466-469: the Q/K/V projections, their biases and
 * ggml_rope_ext) applied to the accumulators: no [M][(H + 2 Hkv) hd] block is written.
 * W: device-layout [N][K], a slice of the Q|K|V layout starting at column col0 (a multiple of
 * 32), in which the rows of every Q and K head are permuted in blocks of 32: rows 32j..32j+15
 * of a head are its dims 16j..16j+15 and rows 32j+16..32j+31 the dims hd/2 + 16j.. they rotate
 * with (hd a multiple of 32); V rows are in order.  bias (or NULL) follows W's rows.  The
 * rotated rows are stored as dfx_rope_store stores them: q_out [M][H][hd], kc[pos][Hkv][hd],
 * vt[Hkv][hd][v_ld] at column pos[m]; the same bits as dfx_gemm (+bias) followed by
 * dfx_rope_store on the unpermuted rows.  ws: as in dfx_gemm. */
int dfx_gemm_rope(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M, const float * bias,
                  int col0, const int32_t * pos, int H, int Hkv, int hd, const float * tab, float * q_out,
                  float * kc, float * vt, int64_t v_ld, void * ws, void * stream);

/* Force the tile and split-K choice of the Q4_K or Q6_K GEMM for every later call in the
 * process (tuning and tests; every choice gives the same bits): "<TM>x<TN>[x<D>]" picks a
 * register tile, "s" splits K where possible, "n" never splits, "w" / "w1" / "w3" pick the
 * Q4_K LDS-DMA kernel (w3: 96 rows per tile), "v1" / "v2" a Q4_K 32-row register tile in
 * workgroups of one or two waves, "k" / "k2" / "k4" the Q4_K super-block-parallel kernel over
 * 1, 2 or 4 column tiles per workgroup ("ks": K split at chunk borders); NULL or "" restores
 * the built-in choice.
 * DFX_Q4K_TILE and DFX_Q6K_TILE in the environment are read once, before the first call.
 * No counterpart in the reference (GGML has no tile choice). */
int dfx_gemm_force_tile(int wtype, const char * spec);

/* dfx_gemm without a workspace argument and without any allocation: the split-K partial
 * sums go to a library-held device array of 32 MiB per GPU (held from the library's load to
 * process end).  Quantised weights whose split would need more (M * N * ceil(K / 2048) * 4
 * bytes) keep K whole, which gives the same bits; an F16 split that would not fit is refused
 * with DFX_ERR_ARG (the split rule needs at most 16 MiB).  Same kernels and the same bits as
 * dfx_gemm with a workspace.  The first call on a device may be made under stream capture
 * (it looks the array's address up with the thread's capture mode relaxed).  Calls on one GPU
 * share that array: calls that overlap in time on one GPU (several streams or host threads)
 * race; serialise them.  No counterpart in the reference: for callers that cannot allocate
 * device memory (code under stream capture, serving loops that forbid hipMalloc). */
int dfx_gemm_noalloc(int wtype, const void * w, int64_t N, int64_t K, const void * act, int64_t M,
                     const float * bias, const float * residual, float * y, void * stream);

/* NEOX RoPE + cache store (src/diffuse-graph.cpp:71-79, 466-469; cache contents of
 * src/diffuse-cache.h:23-26 but at n_head_kv width — the GQA repeat of 84-95 is
 * index math in the attention kernel).  qkv: [M][(H + 2*Hkv)*hd] f32 (Q | K | V);
 * pos[M] absolute positions (< v_ld); tab: [n_pos][hd/2][cos, sin] f32.
 * Writes q_out [M][H][hd], kc[pos][Hkv][hd] and the transposed value cache
 * vt[Hkv][hd][v_ld] (v_ld = cache capacity in positions). */
int dfx_rope_store(const float * qkv, const int32_t * pos, int64_t M, int H, int Hkv, int hd,
                   const float * tab, float * q_out, float * kc, float * vt, int64_t v_ld, void * stream);

/* Bidirectional attention, no mask (src/diffuse-graph.cpp:97-119 / 528-553):
 * out[m][h*hd + j] = sum_n softmax_n(q_m . k_n / sqrt(hd)) * v_n[j], keys 0..n_keys-1
 * of the cache (kc[n][Hkv][hd], vt[Hkv][hd][v_ld], n_keys <= v_ld, v_ld a multiple of
 * 16), query head h reads KV head h / (H/Hkv).  Any number of keys: score rows that do not
 * fit the LDS are recomputed instead of stored. */
int dfx_attention(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M, int64_t n_keys,
                  int H, int Hkv, int hd, float * out, void * stream);   /* mode DFX_ATTN_EXACT */

/* Attention arithmetic (same contract as dfx_attention; softmax as the reference:
 * max, exp(s - max), sum in double, p = e * (float)(1/sum)):
 *   DFX_ATTN_SPLIT_BF16 - scores and P.V on the bf16 MFMA with every f32 operand split
 *     into three bf16 parts (x = hi + mid + lo) and each product taken as its six terms
 *     down to 2^-16 of it (error < 2^-25 of the product, as f32), f32 accumulation,
 *     f32 exp.
 *   DFX_ATTN_EXACT - products exact in f64, sums in f64 rounded once, correctly rounded
 *     exp: the float result does not depend on the summation order (the oracle's
 *     arithmetic, bit for bit); the default of dfx_attention and of every context. */
#define DFX_ATTN_SPLIT_BF16 0
#define DFX_ATTN_EXACT      1
int dfx_attention_ex(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M, int64_t n_keys,
                     int H, int Hkv, int hd, float * out, int mode, void * stream);

/* Causal attention of the autoregressive graph (src/ar-graph.cpp:70-88 mask, 176-196
 * ggml_flash_attn_ext): query row m sits at position q_pos0 + m and attends to the
 * keys q_pos0 + m - window + 1 .. q_pos0 + m (window > 0) or 0 .. q_pos0 + m
 * (window 0); every query's own position must be a key (q_pos0 + M <= n_keys).  The
 * exact (f64-summed) form of dfx_attention_ex with DFX_ATTN_EXACT; caches as there. */
int dfx_attention_causal(const float * q, const float * kc, const float * vt, int64_t v_ld, int64_t M,
                         int64_t n_keys, int H, int Hkv, int hd, int64_t q_pos0, int window, float * out,
                         void * stream);

/* Per-row sampler statistics over logits rows (src/diffuse-sampler.cpp:34-57, 241-252):
 * argmax (strict >, lowest index on ties), top-1 and top-2 values and entropy.
 * rows[i] selects row rows[i] of the [*][ld] logits matrix. */
typedef struct {
    int32_t token;       /* argmax */
    float   best;        /* top-1 logit */
    float   second;      /* top-2 logit as the reference loop defines it */
    float   entropy;     /* -sum p log p over p > 1e-10 */
} dfx_row_stat;
int dfx_row_stats(const float * logits, int64_t ld, const int32_t * rows, int64_t n_rows, int64_t V,
                  dfx_row_stat * out, void * stream);

/* Candidate records of masked positions from their row statistics (the push at
 * src/diffuse-sampler.cpp:253-255): {pos[i], argmax, confidence, entropy} with confidence =
 * the top-1 logit, or top-1 minus top-2 when margin != 0 (TOPK_MARGIN). */
typedef struct { int32_t pos; int32_t token; float confidence; float entropy; } dfx_candidate;
int dfx_make_candidates(const dfx_row_stat * stats, const int32_t * pos, int n, int margin, dfx_candidate * out,
                        void * stream);

/* Remask selection (src/diffuse-sampler.cpp:277-305): orders n candidates by the
 * policy's key (ENTROPY_EXIT: entropy ascending; LOW_CONFIDENCE / MASKGIT_PLUS:
 * top-1 logit descending; TOPK_MARGIN: top1-top2 descending), ties by position
 * ascending.  Writes order[0..n) (candidate indices) and *n_unmask = the count to
 * unmask (schedule count n_sched, or max(n_sched, #entropy < tau) for ENTROPY_EXIT,
 * capped at n).  Any n: up to 2048 candidates are sorted in one workgroup, more are
 * placed by rank (each candidate counts the ones before it). */
int dfx_select(const dfx_candidate * cand, int n, int remasking, float tau, int n_sched,
               int32_t * order, int32_t * n_unmask, void * stream);

/* dfx_make_candidates (margin for TOPK_MARGIN) followed by dfx_select in one launch
 * (src/diffuse-sampler.cpp:253-255 and 277-305 as one step): writes cand[0..n), order[0..n)
 * and *n_unmask exactly as the two calls do.  Up to 1024 candidates in one workgroup that
 * places each candidate by rank; more run as the two calls. */
int dfx_select_from_stats(const dfx_row_stat * stats, const int32_t * pos, int n, int remasking, float tau,
                          int n_sched, dfx_candidate * cand, int32_t * order, int32_t * n_unmask, void * stream);

/* Device-resident step bookkeeping of the denoising loop.  The sequence state is device
 * int32 arrays of N: seq (ids), prev (seq right after the last forward), masked (0/1),
 * lastc (step of the last change seen, -1 never).
 * dfx_step_prepare is compute_active_set (src/diffuse-cache.h:79-116) plus the row lists of
 * the step (src/diffuse-sampler.cpp:222-240): with full = 0 a position is active when it
 * changed (seq != prev; lastc = step), is masked, or changed within `keep` steps, and an
 * empty or complete active set makes the step full.  Writes, in position order, the pass
 * rows tok[a] = seq[act[a]], act[a] = position; the head rows (pass rows that are masked
 * positions, or their left neighbours when shift, or every pass row when head_all) as
 * hrows[k] = pass row, hmap[k] = position; the sampler rows srows[k] = masked position i
 * (max(i - 1, 0) when shift), spos[k] = i; counts = {M, n_head, n_cand, full}.
 * dfx_step_unmask is update_seq + unmask (src/diffuse-sampler.cpp:154, 316-323): prev = seq
 * when use_cache, then the first min(*n_unmask, n_cand) candidates cand[order[j]] write
 * their token into seq and clear masked (ustep[pos] = step when ustep != NULL);
 * hist[step] = the count, or -1 if the order named a candidate out of range. */
int dfx_step_prepare(int N, int step, int full, int keep, int shift, int head_all, const int32_t * seq,
                     const int32_t * prev, const int32_t * masked, int32_t * lastc, int32_t * tok, int32_t * act,
                     int32_t * hrows, int32_t * hmap, int32_t * srows, int32_t * spos, int32_t * counts, void * stream);
int dfx_step_unmask(int N, int use_cache, int step, int32_t * seq, int32_t * prev, int32_t * masked,
                    const dfx_candidate * cand, const int32_t * order, const int32_t * n_unmask, int n_cand,
                    int32_t * ustep, int32_t * hist, void * stream);

/* Greedy sample_token of the autoregressive sampler (src/ar-sampler.cpp:83-117) on one
 * device logits row, which it modifies: the repetition penalty over the recent tokens
 * (x/p for x > 0, else x*p, once per occurrence; none unless repeat_penalty > 1), then
 * the first index of the maximum (token 0 if row[0] is NaN or nothing exceeds -inf).
 * state (device int32 [4 + repeat_last_n]): [0] next token, [1] its position, [2] number
 * of recent tokens, [3] ring start, then the ring of recent tokens.  The chosen token is
 * written to state[0] and token_out[0], state[1] advances by one and the token enters
 * the ring (src/ar-sampler.cpp:236-242 keeps the last repeat_last_n tokens).  repeat_last_n
 * is at most 4096 (DFX_ERR_ARG otherwise). */
int dfx_ar_greedy(float * row, int64_t V, int32_t * state, int repeat_last_n, float repeat_penalty,
                  int32_t * token_out, void * stream);

/* Per-row layer impact of ar_profile_layers (src/ar-graph.cpp:219-228): out[m] = sum
 * over i of (x[m][i] - x_in[m][i])^2 with the difference and square in float and the
 * sum in double in increasing i.  x, x_in: device [M][d]; out: device double [M]. */
int dfx_layer_impact(const float * x, const float * x_in, int64_t M, int64_t d, double * out, void * stream);

/* ---- weight encoding, quantizer and synthetic models (host side) ---- */

/* Encode n_rows x n_cols f32 into GGUF blocks of `type` (Q4_K, Q6_K, Q8_0, F16, F32). */
int dfx_quantize_rows(int type, const float * src, int64_t n_rows, int64_t n_cols, void * dst);

/* diffuse-quantize (tools/quantize.cpp:126-357): scheme "q4_k_m", "q8_0", "q6_k" or "f16",
 * with the reference's per-tensor type mixture and keep rules. */
int dfx_quantize_file(const char * in_path, const char * out_path, const char * scheme, int n_threads);

/* Deterministic random-init model written as GGUF with the converters' keys and tensor
 * names: weights sigma*N(0,1) drawn per tensor from `seed`, rounded to f16, then
 * converted with `scheme`; norm weights 1.0; Dream adds Q/K/V biases. */
typedef struct {
    uint32_t    n_vocab, n_embd, n_head, n_head_kv, n_layer, n_ff, n_ctx_max;
    float       rope_theta, rms_norm_eps;
    uint32_t    mask_token_id;
    int32_t     is_dream;      /* model_type "dream" (+ Q/K/V biases), else "llada" */
    int32_t     tied_output;   /* omit output.weight (lm_head tied to token_embd) */
    uint64_t    seed;
    float       sigma;
    const char * scheme;
    int32_t     n_threads;     /* 0 = hardware threads, at most 16 */
} dfx_synth_spec;
int dfx_synth_model(const char * path, const dfx_synth_spec * spec);

/* ---- model / context (C form of include/diffuse.h) ---- */
typedef struct diffuse_model   dfx_model;
typedef struct diffuse_context dfx_context;

typedef struct {
    uint32_t n_vocab, n_embd, n_head, n_head_kv, n_layer, n_ff, n_ctx_max;
    float    rope_theta, rms_norm_eps;
    uint32_t mask_token_id;
    int32_t  is_dream;
} dfx_hparams;

/* remasking / schedule ids follow the enum order of include/diffuse.h:32-43 */
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
} dfx_sampler_params;

typedef struct {
    int    actual_steps;
    double total_ms, forward_ms, sample_ms;
    int    rows_per_step[256];      /* rows of each step's forward */
    int    unmasked_per_step[256];
    float  step_ms[256];            /* forward time of each step */
} dfx_gen_stats;

int  dfx_model_load(const char * path, dfx_model ** out);              /* diffuse-model.cpp:83-185 */
void dfx_model_free(dfx_model * m);
int  dfx_model_hparams(const dfx_model * m, dfx_hparams * out);
int  dfx_context_new(const dfx_model * m, int n_ctx, dfx_context ** out);  /* diffuse-graph.cpp:683 */
void dfx_context_free(dfx_context * c);
/* tokens[n] (host) -> logits_out[n][n_vocab] (host), src/diffuse-graph.cpp:676-680 */
int  dfx_forward(dfx_context * c, const int32_t * tokens, int n, float * logits_out);
/* The cached forward of one denoising step (diffuse_forward_cached, src/diffuse-graph.h:32-41,
 * src/diffuse-graph.cpp:596-673): the n_active rows at positions active_pos[] (distinct, in
 * [0, n_total)) run through every layer; their K/V replace those positions in the context's
 * cache (update_kv, src/diffuse-cache.h:124-140) and attention reads all n_total positions.
 * The cache must hold a full forward of n_total tokens: the context's last call was dfx_forward
 * with n = n_total, or dfx_forward_cached after it.  logits_out: [n_active][n_vocab] (host). */
int  dfx_forward_cached(dfx_context * c, const int32_t * active_tokens, const int32_t * active_pos, int n_active,
                        int n_total, float * logits_out);
/* diffuse_generate (src/diffuse-sampler.cpp:373-380); out[n_generate] host. */
int  dfx_generate(dfx_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                  const dfx_sampler_params * p, int32_t * out, dfx_gen_stats * stats);
/* Instrumentation: with profiling on, every GEMM the context launches is bracketed by
 * HIP events on its stream.  _read returns, for one weight type, the number of
 * launches, their summed duration, and their algorithmic FLOPs (2*M*N*K) and bytes
 * (weights + converted activations + f32 output).  Enabling resets the totals. */
/* Attention arithmetic of the context's forward passes (DFX_ATTN_EXACT, the default, or
 * DFX_ATTN_SPLIT_BF16; see dfx_attention_ex).  Build-defined; no counterpart in the reference. */
int  dfx_context_set_attention(dfx_context * c, int mode);
/* Loop of the context's dfx_generate calls at temperature 0 with a policy other than RANDOM:
 * 1 (the default) keeps the sequence state and the step bookkeeping on the device
 * (dfx_step_prepare / dfx_step_unmask; no step waits for its own selection) and replays each
 * step's layer stack from a HIP graph captured once per (rows, keys, attention mode); 2 is
 * the same loop with every kernel launched one by one; 0 runs the bookkeeping on the host
 * with one wait per step.  All give the same tokens.  Build-defined; no counterpart in the
 * reference. */
int  dfx_context_set_device_loop(dfx_context * c, int enable);
int  dfx_context_profile(dfx_context * c, int enable);
int  dfx_context_profile_read(dfx_context * c, int wtype, int64_t * launches, double * ms, double * flops,
                              double * bytes);
/* The same totals for one class of row counts: rows_class 1 = GEMMs over M > 96 rows (the
 * 64-row-tile Q4_K kernel's range), 2 = M <= 96, 3 = M >= 288 (a full forward of 288 or more
 * rows), 0 = all (as dfx_context_profile_read).
 * Build-defined instrumentation; no counterpart in the reference. */
int  dfx_context_profile_read_rows(dfx_context * c, int wtype, int rows_class, int64_t * launches, double * ms,
                                   double * flops, double * bytes);
/* ---- autoregressive API (include/diffuse.h:96-120; src/ar-graph.h, src/ar-sampler.cpp) ---- */
/* ar_sampler_params (include/diffuse.h:96-107) */
typedef struct {
    float    temperature;      /* <= 0: greedy */
    float    top_p;
    int      top_k;            /* 0 = off */
    float    repeat_penalty;
    int      repeat_last_n;
    uint32_t seed;
    int      layer_skip;       /* layers skipped after profiling the prompt (0 = off) */
    int      sliding_window;   /* keys within this many positions (0 = all) */
} dfx_ar_params;

typedef struct {
    double prefill_ms, decode_ms, total_ms;
    int    n_prompt, n_decoded, n_generated, n_skipped_layers;
} dfx_ar_stats;

/* Called after each generated token with its position; returning 0 stops the generation
 * (ar_token_callback, include/diffuse.h:110). */
typedef int (*dfx_ar_token_fn)(int32_t token, int pos, void * user);

/* One pass of the causal graph over the context's append-only cache
 * (ar_forward_prefill / ar_forward_batch / ar_forward_decode, src/ar-graph.h:16-39):
 * tokens[n_new] at positions n_past.. (n_past = 0 after reset != 0); logits_out:
 * [n_new][n_vocab] (host), or NULL.  sliding_window as in dfx_ar_params.  Layers marked by
 * dfx_ar_profile_layers stay skipped until the next profiling.  n_past + n_new must not
 * exceed the context's n_ctx.  The diffusion cache of dfx_forward_cached is invalidated. */
int  dfx_ar_forward(dfx_context * c, const int32_t * tokens, int n_new, int reset, int sliding_window,
                    float * logits_out);
/* ar_profile_layers (src/ar-graph.cpp:454-505): a prefill (n_past = 0) with every layer,
 * recording each layer's impact (sum of squared changes of the residual stream), then the
 * n_skip lowest-impact layers outside the first two and last two are marked skipped.
 * impact_out (optional, host float[n_layer]); skip_out (optional, host uint8[n_layer]). */
int  dfx_ar_profile_layers(dfx_context * c, const int32_t * tokens, int n_tokens, int sliding_window, int n_skip,
                           float * logits_out, float * impact_out, uint8_t * skip_out);
/* ar_generate (src/ar-sampler.cpp:143-314): out gets up to max(max_tokens, 1) ids and
 * *n_out their number (generation ends after an end token 151643 / 151645 / 151644, or
 * when cb returns 0); cb and stats may be NULL.  Temperature <= 0 samples on the device;
 * otherwise each row is sampled on the host with the reference's std:: algorithms. */
int  dfx_ar_generate(dfx_context * c, const int32_t * prompt, int n_prompt, int max_tokens, const dfx_ar_params * p,
                     int32_t * out, int * n_out, dfx_ar_stats * stats, dfx_ar_token_fn cb, void * user);

/* dfx_generate that also records, for each generated position, the step (0-based)
 * at which it was unmasked (-1 if still masked at the end).  Stands in for the
 * per-step callback of include/diffuse.h:67-68 for C callers. */
int  dfx_generate_trace(dfx_context * c, const int32_t * prompt, int n_prompt, int n_generate,
                        const dfx_sampler_params * p, int32_t * out, dfx_gen_stats * stats,
                        int32_t * unmask_step);

#ifdef __cplusplus
}
#endif
