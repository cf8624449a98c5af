"""ctypes binding of the C ABI in include/dfx.h (libdiffuse.so).

The Python-side binding a caller of the denoising path uses: device buffers,
kernel entry points, and the model / context / generate API that mirrors
diffuse-cpp's include/diffuse.h:71-91.  It loads the in-tree build
(diffuse-cpp_amd/lib/libdiffuse.so) and raises if that library is missing:
there is no CPU fallback.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdiffuse.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K = 0, 1, 8, 12, 14, 15
SCHED_COSINE, SCHED_LINEAR = 0, 1
LOW_CONFIDENCE, RANDOM, ENTROPY_EXIT, MASKGIT_PLUS, TOPK_MARGIN = 0, 1, 2, 3, 4
ATTN_SPLIT_BF16, ATTN_EXACT = 0, 1          # dfx_attention_ex modes (include/dfx.h)


class DfxError(RuntimeError):
    pass


class Hparams(C.Structure):
    _fields_ = [("n_vocab", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("n_layer", C.c_uint32), ("n_ff", C.c_uint32),
                ("n_ctx_max", C.c_uint32), ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float),
                ("mask_token_id", C.c_uint32), ("is_dream", C.c_int32)]


class SamplerParams(C.Structure):
    _fields_ = [("n_steps", C.c_int), ("temperature", C.c_float), ("schedule", C.c_int),
                ("remasking", C.c_int), ("seed", C.c_uint32), ("entropy_threshold", C.c_float),
                ("use_cache", C.c_int), ("cache_refresh", C.c_int), ("cache_keep_active", C.c_int)]

    @classmethod
    def make(cls, n_steps=32, temperature=0.0, schedule=SCHED_COSINE, remasking=LOW_CONFIDENCE,
             seed=42, entropy_threshold=1.5, use_cache=True, cache_refresh=0, cache_keep_active=0):
        # defaults of include/diffuse.h:45-55
        return cls(n_steps, temperature, schedule, remasking, seed, entropy_threshold,
                   1 if use_cache else 0, cache_refresh, cache_keep_active)


class GenStats(C.Structure):
    _fields_ = [("actual_steps", C.c_int), ("total_ms", C.c_double), ("forward_ms", C.c_double),
                ("sample_ms", C.c_double), ("rows_per_step", C.c_int * 256),
                ("unmasked_per_step", C.c_int * 256), ("step_ms", C.c_float * 256)]


class ArParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int), ("seed", C.c_uint32),
                ("layer_skip", C.c_int), ("sliding_window", C.c_int)]

    @classmethod
    def make(cls, temperature=0.0, top_p=0.9, top_k=40, repeat_penalty=1.1, repeat_last_n=64, seed=42,
             layer_skip=0, sliding_window=0):
        # defaults of ar_sampler_params, include/diffuse.h:96-107
        return cls(temperature, top_p, top_k, repeat_penalty, repeat_last_n, seed, layer_skip, sliding_window)


class ArStats(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("total_ms", C.c_double),
                ("n_prompt", C.c_int), ("n_decoded", C.c_int), ("n_generated", C.c_int),
                ("n_skipped_layers", C.c_int)]


AR_TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_int32, C.c_int, C.c_void_p)


class SynthSpec(C.Structure):
    _fields_ = [("n_vocab", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("n_layer", C.c_uint32), ("n_ff", C.c_uint32),
                ("n_ctx_max", C.c_uint32), ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float),
                ("mask_token_id", C.c_uint32), ("is_dream", C.c_int32), ("tied_output", C.c_int32),
                ("seed", C.c_uint64), ("sigma", C.c_float), ("scheme", C.c_char_p),
                ("n_threads", C.c_int32)]


ROW_STAT = np.dtype([("token", "<i4"), ("best", "<f4"), ("second", "<f4"), ("entropy", "<f4")])
CANDIDATE = np.dtype([("pos", "<i4"), ("token", "<i4"), ("confidence", "<f4"), ("entropy", "<f4")])

# Architectures of the benchmark configurations (hparams as the converters write them).
LLADA_8B = dict(n_vocab=126464, n_embd=4096, n_head=32, n_head_kv=32, n_layer=32, n_ff=12288,
                rope_theta=500000.0, rms_norm_eps=1e-5, mask_token_id=126336, is_dream=0)
DREAM_7B = dict(n_vocab=152064, n_embd=3584, n_head=28, n_head_kv=4, n_layer=28, n_ff=18944,
                rope_theta=1000000.0, rms_norm_eps=1e-6, mask_token_id=151666, is_dream=1)

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DfxError(f"{LIB_PATH} is not built (run `make -C diffuse-cpp_amd`)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    P, I64, I32, F, S = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_size_t
    sig = {
        "dfx_last_error": (C.c_char_p, []),
        "dfx_device_count": (I32, [C.POINTER(C.c_int)]),
        "dfx_malloc": (I32, [C.POINTER(C.c_void_p), S]),
        "dfx_free": (I32, [P]),
        "dfx_memcpy_h2d": (I32, [P, P, S, P]),
        "dfx_memcpy_d2h": (I32, [P, P, S, P]),
        "dfx_memcpy_d2d": (I32, [P, P, S, P]),
        "dfx_memset": (I32, [P, I32, S, P]),
        "dfx_stream_create": (I32, [C.POINTER(C.c_void_p)]),
        "dfx_stream_destroy": (I32, [P]),
        "dfx_stream_sync": (I32, [P]),
        "dfx_timer_start": (I32, [C.POINTER(C.c_void_p), P]),
        "dfx_timer_stop": (I32, [P, P, C.POINTER(C.c_float)]),
        "dfx_device_row_bytes": (I64, [I32, I64]),
        "dfx_device_type": (I32, [I32]),
        "dfx_repack_rows": (I32, [I32, P, I64, I64, P]),
        "dfx_dequant": (I32, [I32, P, I64, I64, P, P]),
        "dfx_embed": (I32, [I32, P, I64, P, I64, P, P]),
        "dfx_act_bytes": (S, [I32, I64, I64]),
        "dfx_act_convert": (I32, [I32, P, I64, I64, P, P]),
        "dfx_rmsnorm_convert": (I32, [I32, P, P, I64, I64, F, P, P]),
        "dfx_swiglu_convert": (I32, [I32, P, I64, I64, P, P]),
        "dfx_gemm_ws_bytes": (S, [I64, I64, I64]),
        "dfx_gemm": (I32, [I32, P, I64, I64, P, I64, P, P, P, P, P]),
        "dfx_gemm_noalloc": (I32, [I32, P, I64, I64, P, I64, P, P, P, P]),
        "dfx_gemm_counted": (I32, [I32, P, I64, I64, P, I64, P, P, P, P, P, P]),
        "dfx_gemm_tile_cnt_bytes": (S, [I64, I64]),
        "dfx_gemm_swiglu": (I32, [I32, P, I64, I64, P, I64, P, I64, P, P]),
        "dfx_gemm_rope": (I32, [I32, P, I64, I64, P, I64, P, I32, P, I32, I32, I32, P, P, P, P, I64, P, P]),
        "dfx_gemm_force_tile": (I32, [I32, C.c_char_p]),
        "dfx_rope_store": (I32, [P, P, I64, I32, I32, I32, P, P, P, P, I64, P]),
        "dfx_attention": (I32, [P, P, P, I64, I64, I64, I32, I32, I32, P, P]),
        "dfx_attention_ex": (I32, [P, P, P, I64, I64, I64, I32, I32, I32, P, I32, P]),
        "dfx_row_stats": (I32, [P, I64, P, I64, I64, P, P]),
        "dfx_select": (I32, [P, I32, I32, F, I32, P, P, P]),
        "dfx_select_from_stats": (I32, [P, P, I32, I32, F, I32, P, P, P, P]),
        "dfx_make_candidates": (I32, [P, P, I32, I32, P, P]),
        "dfx_quantize_rows": (I32, [I32, P, I64, I64, P]),
        "dfx_quantize_file": (I32, [C.c_char_p, C.c_char_p, C.c_char_p, I32]),
        "dfx_synth_model": (I32, [C.c_char_p, C.POINTER(SynthSpec)]),
        "dfx_model_load": (I32, [C.c_char_p, C.POINTER(C.c_void_p)]),
        "dfx_model_free": (None, [P]),
        "dfx_model_hparams": (I32, [P, C.POINTER(Hparams)]),
        "dfx_context_new": (I32, [P, I32, C.POINTER(C.c_void_p)]),
        "dfx_context_free": (None, [P]),
        "dfx_forward": (I32, [P, P, I32, P]),
        "dfx_forward_cached": (I32, [P, P, P, I32, I32, P]),
        "dfx_generate": (I32, [P, P, I32, I32, C.POINTER(SamplerParams), P, C.POINTER(GenStats)]),
        "dfx_generate_trace": (I32, [P, P, I32, I32, C.POINTER(SamplerParams), P, C.POINTER(GenStats), P]),
        "dfx_attention_causal": (I32, [P, P, P, I64, I64, I64, I32, I32, I32, I64, I32, P, P]),
        "dfx_context_set_device_loop": (I32, [P, I32]),
        "dfx_step_prepare": (I32, [I32, I32, I32, I32, I32, I32, P, P, P, P, P, P, P, P, P, P, P, P]),
        "dfx_step_unmask": (I32, [I32, I32, I32, P, P, P, P, P, P, I32, P, P, P]),
        "dfx_ar_greedy": (I32, [P, I64, P, I32, F, P, P]),
        "dfx_layer_impact": (I32, [P, P, I64, I64, P, P]),
        "dfx_ar_forward": (I32, [P, P, I32, I32, I32, P]),
        "dfx_ar_profile_layers": (I32, [P, P, I32, I32, I32, P, P, P]),
        "dfx_ar_generate": (I32, [P, P, I32, I32, C.POINTER(ArParams), P, C.POINTER(C.c_int), C.POINTER(ArStats),
                                  AR_TOKEN_FN, P]),
        "dfx_context_profile": (I32, [P, I32]),
        "dfx_context_set_attention": (I32, [P, I32]),
        "dfx_context_profile_read_rows": (I32, [P, I32, I32, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                                                C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "dfx_context_profile_read": (I32, [P, I32, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                                           C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def check(rc, what=""):
    if rc != 0:
        raise DfxError(f"{what} failed ({rc}): {lib().dfx_last_error().decode()}")


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


class Buf:
    """A device allocation; upload/download through numpy arrays."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().dfx_malloc(C.byref(p), max(self.nbytes, 1)), "dfx_malloc")
        self.ptr = p

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        b.upload(arr)
        return b

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib().dfx_memcpy_h2d(self.ptr, _ptr(arr), arr.nbytes, None), "h2d")

    def download(self, dtype, count=None, shape=None):
        dtype = np.dtype(dtype)
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(lib().dfx_memcpy_d2h(_ptr(out), self.ptr, out.nbytes, None), "d2h")
        return out.reshape(shape) if shape is not None else out

    def zero(self):
        check(lib().dfx_memset(self.ptr, 0, self.nbytes, None), "memset")
        sync()

    def free(self):
        if self.ptr:
            lib().dfx_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync(stream=None):
    check(lib().dfx_stream_sync(stream), "sync")


def device_count():
    n = C.c_int(0)
    rc = lib().dfx_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def q4k_slot_order():
    """Element index held by each slot of a 64-element group of a Q4_K activation
    buffer (slot 8i+s: s<4 -> 4i+P[s], s>=4 -> 32+4i+P[s-4], P = 0,2,1,3)."""
    P = (0, 2, 1, 3)
    return np.array([(32 if s >= 4 else 0) + 4 * i + P[s % 4] for i in range(8) for s in range(8)], np.int64)


def q6k_slot_order():
    """Element index held by each slot of a 128-element half super-block of a Q6_K
    activation buffer (slot 64g + 8(i + 4p) + s -> 32q + 16g + 4i + P[s % 4],
    q = p + 2 (s >= 4), P = 0,2,1,3)."""
    P = (0, 2, 1, 3)
    order = np.empty(128, np.int64)
    for g in range(2):
        for p in range(2):
            for i in range(4):
                for s in range(8):
                    q = p + (2 if s >= 4 else 0)
                    order[64 * g + 8 * (i + 4 * p) + s] = 32 * q + 16 * g + 4 * i + P[s % 4]
    return order


def act_frag_index(M, K):
    """Half index of (row m, slot sl) in the fragment-ordered q of Q4_K / Q6_K
    activation buffers: sl = 128*step + 64*hl + 8*kk + j goes to
    (((m/32) * (K/128) + step) * 8 + kk) * 512 + (m%32 + 32*hl) * 8 + j."""
    m = np.arange(M, dtype=np.int64)[:, None]
    sl = np.arange(K, dtype=np.int64)[None, :]
    step, w = sl >> 7, sl & 127
    hl, kk, j = w >> 6, (w >> 3) & 7, w & 7
    return ((((m >> 5) * (K >> 7) + step) * 8 + kk) * 64 + (m & 31) + 32 * hl) * 8 + j


def act_parts(act_buf, wtype, M, K):
    """Split a downloaded activation buffer (layout of dfx_act_bytes) into (q, d, bs);
    q is returned in element order."""
    raw = act_buf.download(np.uint8)

    def a256(x):
        return (x + 255) // 256 * 256
    m_q = (M + 31) // 32 * 32 if wtype in (TYPE_Q4_K, TYPE_Q6_K) else M
    if wtype in (TYPE_Q4_K, TYPE_Q6_K):
        allq = raw[:m_q * K * 2].view(np.float16)
        stored = allq[act_frag_index(M, K)]             # [M][K] in slot order
        g = 64 if wtype == TYPE_Q4_K else 128
        stored = stored.reshape(M, K // g, g)
        q = np.empty_like(stored)
        q[:, :, q4k_slot_order() if wtype == TYPE_Q4_K else q6k_slot_order()] = stored
        q = q.reshape(M, K)
    else:
        q = raw[:M * K * 2].view(np.float16).reshape(M, K)
    d_off = a256(m_q * K * 2)
    if wtype in (TYPE_Q4_K, TYPE_Q6_K):
        nd, nbs = M * (K // 256), M * (K // 16)
    elif wtype == TYPE_Q8_0:
        nd, nbs = M * (K // 32), 0
    else:
        return q, None, None
    if wtype in (TYPE_Q4_K, TYPE_Q6_K):   # super-block major over the padded rows
        d = raw[d_off:d_off + (K // 256) * m_q * 4].view(np.float32).reshape(K // 256, m_q)[:, :M].T.copy()
        nd = (K // 256) * m_q
    else:
        d = raw[d_off:d_off + nd * 4].view(np.float32).reshape(M, -1)
    bs_off = a256(d_off + nd * 4)
    bs = raw[bs_off:bs_off + nbs * 2].view(np.float16).reshape(M, -1) if nbs else None
    return q, d, bs


def repack(gguf_type, raw, n_rows, n_cols):
    """GGUF row bytes -> device layout bytes (host side)."""
    rb = lib().dfx_device_row_bytes(gguf_type, n_cols)
    if rb < 0:
        raise DfxError(f"no device layout for type {gguf_type} with {n_cols} columns")
    out = np.empty(rb * n_rows, dtype=np.uint8)
    raw = np.ascontiguousarray(raw)
    check(lib().dfx_repack_rows(gguf_type, _ptr(raw), n_rows, n_cols, _ptr(out)), "repack")
    return out


def force_tile(wtype, spec):
    """Force the Q4_K / Q6_K GEMM tile for later calls (None restores the built-in choice)."""
    check(lib().dfx_gemm_force_tile(wtype, spec.encode() if spec else None), "force_tile")


def quantize_rows(gguf_type, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_rows, n_cols = x.shape
    from_block = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144),
                  TYPE_Q6_K: (256, 210)}[gguf_type]
    out = np.empty(n_rows * (n_cols // from_block[0]) * from_block[1], dtype=np.uint8)
    check(lib().dfx_quantize_rows(gguf_type, _ptr(x), n_rows, n_cols, _ptr(out)), "quantize_rows")
    return out


def synth_model(path, arch, scheme="q4_k_m", seed=0, sigma=0.02, n_threads=0, tied_output=False,
                n_ctx_max=4096):
    spec = SynthSpec(arch["n_vocab"], arch["n_embd"], arch["n_head"], arch["n_head_kv"],
                     arch["n_layer"], arch["n_ff"], n_ctx_max, arch["rope_theta"],
                     arch["rms_norm_eps"], arch["mask_token_id"], arch.get("is_dream", 0),
                     1 if tied_output else 0, seed, sigma, scheme.encode(), n_threads)
    check(lib().dfx_synth_model(str(path).encode(), C.byref(spec)), "dfx_synth_model")


def quantize_file(src, dst, scheme, n_threads=0):
    check(lib().dfx_quantize_file(str(src).encode(), str(dst).encode(), scheme.encode(), n_threads),
          "dfx_quantize_file")


class Model:
    def __init__(self, path):
        h = C.c_void_p()
        check(lib().dfx_model_load(str(path).encode(), C.byref(h)), "dfx_model_load")
        self.h = h
        hp = Hparams()
        check(lib().dfx_model_hparams(h, C.byref(hp)), "hparams")
        self.hparams = hp

    def close(self):
        if self.h:
            lib().dfx_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    def __init__(self, model, n_ctx):
        h = C.c_void_p()
        check(lib().dfx_context_new(model.h, n_ctx, C.byref(h)), "dfx_context_new")
        self.h, self.model = h, model

    def forward(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        V = self.model.hparams.n_vocab
        out = np.empty((len(tokens), V), dtype=np.float32)
        check(lib().dfx_forward(self.h, _ptr(tokens), len(tokens), _ptr(out)), "dfx_forward")
        return out

    def forward_cached(self, active_tokens, active_pos, n_total):
        """Logits [n_active][V] of the active rows, attending over all n_total cached
        positions (the cache must hold a forward of n_total tokens)."""
        at = np.ascontiguousarray(active_tokens, dtype=np.int32)
        ap = np.ascontiguousarray(active_pos, dtype=np.int32)
        V = self.model.hparams.n_vocab
        out = np.empty((len(at), V), dtype=np.float32)
        check(lib().dfx_forward_cached(self.h, _ptr(at), _ptr(ap), len(at), int(n_total), _ptr(out)),
              "dfx_forward_cached")
        return out

    def generate(self, prompt, n_generate, params, stats=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_generate, dtype=np.int32)
        st = stats if stats is not None else GenStats()
        check(lib().dfx_generate(self.h, _ptr(prompt), len(prompt), n_generate, C.byref(params),
                                 _ptr(out), C.byref(st)), "dfx_generate")
        return out

    def generate_trace(self, prompt, n_generate, params, stats=None):
        """(tokens, unmask_step): step at which each generated position was unmasked."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_generate, dtype=np.int32)
        steps = np.empty(n_generate, dtype=np.int32)
        st = stats if stats is not None else GenStats()
        check(lib().dfx_generate_trace(self.h, _ptr(prompt), len(prompt), n_generate, C.byref(params),
                                       _ptr(out), C.byref(st), _ptr(steps)), "dfx_generate_trace")
        return out, steps

    def ar_forward(self, tokens, reset=False, sliding_window=0):
        """One causal pass of the autoregressive graph: logits [n_new][V] of tokens at
        positions n_past.. (n_past = 0 with reset)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(t), self.model.hparams.n_vocab), dtype=np.float32)
        check(lib().dfx_ar_forward(self.h, _ptr(t), len(t), 1 if reset else 0, sliding_window, _ptr(out)),
              "dfx_ar_forward")
        return out

    def ar_profile_layers(self, tokens, n_skip, sliding_window=0):
        """(logits, impact, skip) of ar_profile_layers' prefill."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        L = self.model.hparams.n_layer
        out = np.empty((len(t), self.model.hparams.n_vocab), dtype=np.float32)
        imp = np.empty(L, dtype=np.float32)
        skip = np.empty(L, dtype=np.uint8)
        check(lib().dfx_ar_profile_layers(self.h, _ptr(t), len(t), sliding_window, n_skip, _ptr(out), _ptr(imp),
                                          _ptr(skip)), "dfx_ar_profile_layers")
        return out, imp, skip

    def ar_generate(self, prompt, max_tokens, params, stats=None, callback=None):
        """Generated ids of ar_generate; callback(token, pos) -> bool (False stops)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(max_tokens, 1), dtype=np.int32)
        n = C.c_int()
        st = stats if stats is not None else ArStats()
        fn = AR_TOKEN_FN(lambda t, p, u: 1 if callback(t, p) else 0) if callback else AR_TOKEN_FN()
        check(lib().dfx_ar_generate(self.h, _ptr(prompt), len(prompt), max_tokens, C.byref(params), _ptr(out),
                                    C.byref(n), C.byref(st), fn, None), "dfx_ar_generate")
        return out[:n.value].copy()

    def set_device_loop(self, enable=True, graphs=True):
        """Step bookkeeping of greedy dfx_generate on the device (default; its layer stacks
        replayed from captured graphs unless graphs=False) or on the host."""
        mode = (1 if graphs else 2) if enable else 0
        check(lib().dfx_context_set_device_loop(self.h, mode), "dfx_context_set_device_loop")

    def set_attention(self, mode):
        """ATTN_EXACT (the default) or ATTN_SPLIT_BF16 for this context's forward passes."""
        check(lib().dfx_context_set_attention(self.h, int(mode)), "dfx_context_set_attention")

    def profile(self, enable=True):
        check(lib().dfx_context_profile(self.h, 1 if enable else 0), "dfx_context_profile")

    def profile_read(self, wtype, rows_class=0):
        """{launches, ms, flops, bytes} of the GEMMs on weights of type wtype since profiling began;
        rows_class 1 = launches over more than 96 rows, 2 = at most 96, 3 = at least 288, 0 = all."""
        n, ms, fl, by = C.c_int64(), C.c_double(), C.c_double(), C.c_double()
        check(lib().dfx_context_profile_read_rows(self.h, wtype, rows_class, C.byref(n), C.byref(ms), C.byref(fl),
                                                  C.byref(by)), "dfx_context_profile_read_rows")
        return dict(launches=n.value, ms=ms.value, flops=fl.value, bytes=by.value)

    def close(self):
        if self.h:
            lib().dfx_context_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
