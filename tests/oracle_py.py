"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so) and a numpy GGUF
reader, for the parity tests.  Test infrastructure only."""
import ctypes as C
import os
import struct

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(REPO, "oracle", "_build", "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 8, 12, 14, 15
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292),
         2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 30: (1, 2)}

_o = None


def oracle():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        L = C.CDLL(ORACLE_SO)
        P, I64, I = C.c_void_p, C.c_int64, C.c_int
        L.orc_fp16_to_fp32.restype = C.c_float
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_fp32_to_fp16.restype = C.c_uint16
        L.orc_fp32_to_fp16.argtypes = [C.c_float]
        L.orc_dequant_row.argtypes = [I, P, P, I64]
        L.orc_quantize_row_q8_K.argtypes = [P, P, I64]
        L.orc_quantize_row_q8_0.argtypes = [P, P, I64]
        L.orc_vec_dot.argtypes = [I, I64, P, P, P]
        L.orc_mul_mat.argtypes = [I, P, I64, I64, P, I64, P, I]
        L.orc_rms_norm_mul.argtypes = [P, P, I64, I64, C.c_float, P]
        L.orc_rope_table.argtypes = [I, I, C.c_float, P]
        L.orc_rope_neox.argtypes = [P, I64, I, I, P, P]
        L.orc_silu.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_attention.argtypes = [P, P, P, I, I, I, I, P, I]
        L.orc_tokens_to_unmask.argtypes = [I, I, I, I]
        L.orc_entropy.restype = C.c_float
        L.orc_entropy.argtypes = [P, I]
        L.orc_top2.argtypes = [P, I, P, P, P]
        L.orc_order_candidates.argtypes = [P, I, I, C.c_float, I]
        L.orc_forward_full.argtypes = [P, P, I, P, P, I]
        L.orc_forward_cached.argtypes = [P, P, P, I, I, P, P, P, I]
        L.orc_generate.argtypes = [P, P, I, I, P, P, P, I]
        L.orc_attention_causal.argtypes = [P, P, P, I, I, I, I, P, P, I, P, I]
        L.orc_ar_forward.argtypes = [P, P, I, P, P, I, I, I]
        L.orc_ar_choose_skip.argtypes = [P, I, I, P]
        L.orc_rng_new.restype = P
        L.orc_rng_new.argtypes = [C.c_uint32]
        L.orc_rng_free.argtypes = [P]
        L.orc_ar_sample.argtypes = [P, I, P, P, I, P]
        L.orc_ar_generate.argtypes = [P, P, I, I, P, P, P, P, I]
        _o = L
    return _o


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def row_bytes(t, n):
    b, s = BLOCK[t]
    assert n % b == 0
    return n // b * s


# ---------------------------------------------------------------- codecs
def dequant(t, raw, n):
    out = np.empty(n, dtype=np.float32)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    assert oracle().orc_dequant_row(t, ptr(raw), ptr(out), n) == 0
    return out


def quantize_q8_K(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 256 * 292, dtype=np.uint8)
    oracle().orc_quantize_row_q8_K(ptr(x), ptr(out), x.size)
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    oracle().orc_quantize_row_q8_0(ptr(x), ptr(out), x.size)
    return out


def act_convert(wtype, x):
    """f32 value each activation takes inside GGML mul_mat for weight type wtype."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    out = np.empty_like(x)
    for m in range(M):
        if wtype in (Q4_K, Q6_K):
            out[m] = dequant(Q8_K, quantize_q8_K(x[m]), K)
        elif wtype == Q8_0:
            out[m] = dequant(Q8_0, quantize_q8_0(x[m]), K)
        else:
            out[m] = x[m].astype(np.float16).astype(np.float32)
    return out


def mul_mat(wtype, W, N, K, X, n_threads=8):
    X = np.ascontiguousarray(X, dtype=np.float32)
    M = X.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert oracle().orc_mul_mat(wtype, ptr(W), N, K, ptr(X), M, ptr(Y), n_threads) == 0
    return Y


def rms_norm_mul(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    oracle().orc_rms_norm_mul(ptr(x), ptr(w), x.shape[0], x.shape[1], eps, ptr(y))
    return y


def rope_table(n_pos, hd, base):
    tab = np.empty(n_pos * hd, dtype=np.float32)
    oracle().orc_rope_table(n_pos, hd, base, ptr(tab))
    return tab


def attention(q, k, v, n_threads=8):
    """q [M][H][hd], k/v [n_keys][Hkv][hd] (GQA: head h reads KV head h // (H/Hkv)) -> [M][H][hd]."""
    M, H, hd = q.shape
    rep = H // k.shape[1]
    ke = np.ascontiguousarray(np.repeat(k, rep, axis=1), dtype=np.float32)
    ve = np.ascontiguousarray(np.repeat(v, rep, axis=1), dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty((M, H, hd), np.float32)
    oracle().orc_attention(ptr(q), ptr(ke), ptr(ve), M, k.shape[0], H, hd, ptr(out), n_threads)
    return out


def attention_causal(q, k, v, qpos, kpos, window=0, n_threads=8):
    """attention with key n visible to query m when kpos[n] <= qpos[m] (and, with a window
    w > 0, qpos[m] - kpos[n] < w); shapes as attention()."""
    M, H, hd = q.shape
    rep = H // k.shape[1]
    ke = np.ascontiguousarray(np.repeat(k, rep, axis=1), dtype=np.float32)
    ve = np.ascontiguousarray(np.repeat(v, rep, axis=1), dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    qp = np.ascontiguousarray(qpos, dtype=np.int32)
    kp = np.ascontiguousarray(kpos, dtype=np.int32)
    out = np.empty((M, H, hd), np.float32)
    oracle().orc_attention_causal(ptr(q), ptr(ke), ptr(ve), M, k.shape[0], H, hd, ptr(qp), ptr(kp), window,
                                  ptr(out), n_threads)
    return out


def entropy(row):
    row = np.ascontiguousarray(row, dtype=np.float32)
    return oracle().orc_entropy(ptr(row), row.size)


def top2(row):
    row = np.ascontiguousarray(row, dtype=np.float32)
    b, bv, sv = C.c_int(), C.c_float(), C.c_float()
    oracle().orc_top2(ptr(row), row.size, C.byref(b), C.byref(bv), C.byref(sv))
    return b.value, bv.value, sv.value


CAND = np.dtype([("pos", "<i4"), ("token", "<i4"), ("confidence", "<f4"), ("entropy", "<f4")])


def order_candidates(cand, remasking, tau, n_sched):
    c = np.ascontiguousarray(cand.copy(), dtype=CAND)
    n = oracle().orc_order_candidates(ptr(c), len(c), remasking, tau, n_sched)
    return c, n


def ar_sample(row, params, recent, rng):
    row = np.ascontiguousarray(row, dtype=np.float32)
    rec = np.ascontiguousarray(recent, dtype=np.int32)
    return oracle().orc_ar_sample(ptr(row), row.size, C.byref(params), ptr(rec), len(rec), rng)


def choose_skip(impact, n_skip):
    imp = np.ascontiguousarray(impact, dtype=np.float32)
    skip = np.zeros(len(imp), dtype=np.uint8)
    n = oracle().orc_ar_choose_skip(ptr(imp), len(imp), n_skip, ptr(skip))
    return skip, n


def tokens_to_unmask(step, total, masked, schedule):
    return oracle().orc_tokens_to_unmask(step, total, masked, schedule)


# ---------------------------------------------------------------- GGUF (numpy)
class GGUF:
    """Minimal independent GGUF v3 reader (tensor infos + KV scalars/strings)."""

    def __init__(self, path):
        self.path = path
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        b = self.buf
        pos = 0

        def rd(fmt):
            nonlocal pos
            v = struct.unpack_from("<" + fmt, b, pos)
            pos += struct.calcsize("<" + fmt)
            return v[0]

        def rstr():
            nonlocal pos
            n = rd("Q")
            s = bytes(b[pos:pos + n]).decode()
            pos += n
            return s

        scal = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}

        def rval(t):
            if t in scal:
                return rd(scal[t])
            if t == 8:
                return rstr()
            if t == 9:
                at, n = rd("I"), rd("Q")
                return [rval(at) for _ in range(n)]
            raise ValueError(f"bad gguf type {t}")

        assert rd("I") == 0x46554747, "not GGUF"
        self.version = rd("I")
        nt, nkv = rd("Q"), rd("Q")
        self.kv = {}
        for _ in range(nkv):
            k = rstr()
            self.kv[k] = rval(rd("I"))
        self.tensors = {}
        order = []
        for _ in range(nt):
            name = rstr()
            nd = rd("I")
            ne = [rd("Q") for _ in range(nd)]
            t = rd("I")
            off = rd("Q")
            self.tensors[name] = dict(type=t, ne=ne, offset=off)
            order.append(name)
        align = self.kv.get("general.alignment", 32)
        data0 = (pos + align - 1) // align * align
        for name in order:
            ti = self.tensors[name]
            n0 = ti["ne"][0]
            rows = int(np.prod(ti["ne"][1:])) if len(ti["ne"]) > 1 else 1
            nb = row_bytes(ti["type"], n0) * rows
            start = data0 + ti["offset"]
            ti["data"] = self.buf[start:start + nb]
            ti["start"] = start
            ti["rows"] = rows

    def tensor(self, name):
        return self.tensors.get(name)


# ---------------------------------------------------------------- model for the oracle
class OrcTensor(C.Structure):
    _fields_ = [("type", C.c_int), ("ne0", C.c_int64), ("ne1", C.c_int64), ("data", C.c_void_p)]


class OrcLayer(C.Structure):
    _fields_ = [(n, OrcTensor) for n in ("attn_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv", "ffn_norm",
                                         "ffn_gate", "ffn_up", "ffn_down")]


class OrcModel(C.Structure):
    _fields_ = [("n_vocab", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("n_layer", C.c_uint32), ("n_ff", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float), ("mask_token_id", C.c_uint32),
                ("is_dream", C.c_int), ("tok_embd", OrcTensor), ("output_norm", OrcTensor),
                ("output", OrcTensor), ("layers", C.POINTER(OrcLayer))]


class OrcKV(C.Structure):
    _fields_ = [("n_tokens", C.c_int), ("k", C.c_void_p), ("v", C.c_void_p)]


class OrcSamplerParams(C.Structure):
    _fields_ = [("n_steps", C.c_int), ("temperature", C.c_float), ("schedule", C.c_int), ("remasking", C.c_int),
                ("seed", C.c_uint32), ("entropy_threshold", C.c_float), ("use_cache", C.c_int),
                ("cache_refresh", C.c_int), ("cache_keep_active", C.c_int)]


class OrcArCache(C.Structure):
    _fields_ = [("n_ctx_max", C.c_int), ("n_past", C.c_int), ("sliding_window", C.c_int), ("k", C.c_void_p),
                ("v", C.c_void_p), ("skip", C.c_void_p), ("impact", C.c_void_p)]


class OrcArParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int), ("seed", C.c_uint32),
                ("layer_skip", C.c_int), ("sliding_window", C.c_int)]

    @classmethod
    def make(cls, temperature=0.0, top_p=0.9, top_k=40, repeat_penalty=1.1, repeat_last_n=64, seed=42,
             layer_skip=0, sliding_window=0):
        """Defaults of ar_sampler_params (include/diffuse.h:96-107)."""
        return cls(temperature, top_p, top_k, repeat_penalty, repeat_last_n, seed, layer_skip, sliding_window)


class OracleArCache:
    """Append-only AR cache of the oracle (k/v expanded to n_head, f32)."""

    def __init__(self, om, n_ctx_max, sliding_window=0):
        m = om.m
        self.k = np.zeros(m.n_layer * n_ctx_max * m.n_embd, dtype=np.float32)
        self.v = np.zeros_like(self.k)
        self.skip = np.zeros(m.n_layer, dtype=np.uint8)
        self.impact = np.zeros(m.n_layer, dtype=np.float32)
        self.c = OrcArCache(n_ctx_max, 0, sliding_window, self.k.ctypes.data, self.v.ctypes.data,
                            self.skip.ctypes.data, self.impact.ctypes.data)


class OrcGenStats(C.Structure):
    _fields_ = [("actual_steps", C.c_int), ("rows_per_step", C.c_int * 256), ("unmasked_per_step", C.c_int * 256)]


def _first(kv, suffix, default=None):
    for p in ("diffuse", "qwen2", "llama"):
        if f"{p}.{suffix}" in kv:
            return kv[f"{p}.{suffix}"]
    return default


class OracleModel:
    """Binds a GGUF file's tensors (memory-mapped) into the oracle's model struct,
    with the loader's key resolution (src/diffuse-model.cpp:105-158)."""

    def __init__(self, path):
        g = self.g = GGUF(path)
        kv = g.kv
        m = self.m = OrcModel()
        m.n_layer = _first(kv, "block_count")
        m.n_head = _first(kv, "attention.head_count")
        m.n_head_kv = _first(kv, "attention.head_count_kv")
        m.n_embd = _first(kv, "embedding_length")
        m.n_ff = _first(kv, "feed_forward_length")
        m.rope_theta = _first(kv, "rope.freq_base", 1000000.0)
        m.rms_norm_eps = _first(kv, "attention.layer_norm_rms_epsilon", 1e-6)
        m.mask_token_id = _first(kv, "mask_token_id", 0)
        te = g.tensor("token_embd.weight")
        m.n_vocab = _first(kv, "vocab_size", 0) or te["ne"][1]
        m.is_dream = 1 if kv.get("diffuse.model_type") == "dream" else 0
        self._keep = []
        m.tok_embd = self._t("token_embd.weight")
        m.output_norm = self._t("output_norm.weight")
        m.output = self._t("output.weight") if g.tensor("output.weight") else self._t("token_embd.weight")
        layers = (OrcLayer * m.n_layer)()
        for i in range(m.n_layer):
            for f, n in (("attn_norm", "attn_norm.weight"), ("wq", "attn_q.weight"), ("wk", "attn_k.weight"),
                         ("wv", "attn_v.weight"), ("wo", "attn_output.weight"), ("bq", "attn_q.bias"),
                         ("bk", "attn_k.bias"), ("bv", "attn_v.bias"), ("ffn_norm", "ffn_norm.weight"),
                         ("ffn_gate", "ffn_gate.weight"), ("ffn_up", "ffn_up.weight"),
                         ("ffn_down", "ffn_down.weight")):
                setattr(layers[i], f, self._t(f"blk.{i}.{n}"))
        self._layers = layers
        m.layers = layers

    def _t(self, name):
        ti = self.g.tensor(name)
        if ti is None:
            return OrcTensor(0, 0, 0, None)
        arr = np.ascontiguousarray(ti["data"])
        self._keep.append(arr)
        return OrcTensor(ti["type"], ti["ne"][0], ti["rows"], arr.ctypes.data)

    @property
    def dims(self):
        m = self.m
        hd = m.n_embd // m.n_head
        return dict(d=m.n_embd, H=m.n_head, Hkv=m.n_head_kv, hd=hd, V=m.n_vocab, L=m.n_layer, F=m.n_ff)

    def forward_full(self, tokens, kv_tokens=None, n_threads=8):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        logits = np.empty((n, self.m.n_vocab), dtype=np.float32)
        kv = None
        if kv_tokens is not None:
            kv = self.new_kv(kv_tokens)
        rc = oracle().orc_forward_full(C.byref(self.m), ptr(tokens), n, ptr(logits),
                                       C.byref(kv[0]) if kv else None, n_threads)
        assert rc == 0
        return (logits, kv) if kv else logits

    def forward_full_perturbed(self, tokens, rel=1e-7, layer=1, seed=9, n_threads=8):
        """forward_full with the F32 attention-norm weights of one layer multiplied by
        (1 + rel * N(0, 1)): a probe of how far the oracle's own logits move under a
        perturbation at the level of f32 rounding (the conditioning of the input)."""
        lay = self._layers[layer]
        t0 = OrcTensor(lay.attn_norm.type, lay.attn_norm.ne0, lay.attn_norm.ne1, lay.attn_norm.data)
        assert t0.type == 0, "F32 norm weights only"
        base = np.ctypeslib.as_array(C.cast(t0.data, C.POINTER(C.c_float)), shape=(t0.ne0,)).astype(np.float64)
        pert = np.ascontiguousarray(
            (base * (1 + rel * np.random.default_rng(seed).standard_normal(base.shape))).astype(np.float32))
        lay.attn_norm = OrcTensor(t0.type, t0.ne0, t0.ne1, pert.ctypes.data)
        try:
            return self.forward_full(tokens, n_threads=n_threads)
        finally:
            lay.attn_norm = t0

    def new_kv(self, n_tokens):
        d = self.m.n_embd
        k = np.zeros(self.m.n_layer * n_tokens * d, dtype=np.float32)
        v = np.zeros_like(k)
        return (OrcKV(n_tokens, k.ctypes.data, v.ctypes.data), k, v)

    def forward_cached(self, kv, active_tokens, active_pos, n_total, n_threads=8):
        at = np.ascontiguousarray(active_tokens, dtype=np.int32)
        ap = np.ascontiguousarray(active_pos, dtype=np.int32)
        cached = np.array([i for i in range(n_total) if i not in set(ap.tolist())], dtype=np.int32)
        logits = np.empty((len(at), self.m.n_vocab), dtype=np.float32)
        rc = oracle().orc_forward_cached(C.byref(self.m), ptr(at), ptr(ap), len(at), n_total, C.byref(kv[0]),
                                         ptr(cached), ptr(logits), n_threads)
        assert rc == 0
        return logits

    def ar_forward(self, cache, tokens, last_only=False, profile=False, n_threads=8):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = 1 if last_only else len(t)
        logits = np.empty((rows, self.m.n_vocab), dtype=np.float32)
        rc = oracle().orc_ar_forward(C.byref(self.m), ptr(t), len(t), C.byref(cache.c), ptr(logits),
                                     1 if last_only else 0, 1 if profile else 0, n_threads)
        assert rc == 0
        return logits

    def ar_generate(self, prompt, max_tokens, params, n_threads=8):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(max_tokens, 1), dtype=np.int32)
        n = C.c_int()
        skip = np.zeros(self.m.n_layer, dtype=np.uint8)
        rc = oracle().orc_ar_generate(C.byref(self.m), ptr(prompt), len(prompt), max_tokens, C.byref(params),
                                      ptr(out), C.byref(n), ptr(skip), n_threads)
        assert rc == 0
        return out[:n.value], skip

    def generate(self, prompt, n_generate, n_steps=16, temperature=0.0, schedule=0, remasking=0, seed=42,
                 entropy_threshold=1.5, use_cache=True, cache_refresh=0, cache_keep_active=0, n_threads=8):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        p = OrcSamplerParams(n_steps, temperature, schedule, remasking, seed, entropy_threshold,
                             1 if use_cache else 0, cache_refresh, cache_keep_active)
        out = np.empty(n_generate, dtype=np.int32)
        st = OrcGenStats()
        rc = oracle().orc_generate(C.byref(self.m), ptr(prompt), len(prompt), n_generate, C.byref(p), ptr(out),
                                   C.byref(st), n_threads)
        assert rc == 0
        return out, st
