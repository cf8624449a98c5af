"""End-to-end parity of the HIP path (through the C ABI) with the CPU oracle:
per-step logits (rel-L2 <= 1e-2, >= 99% argmax agreement) and the
denoising loop, replayed step by step through the oracle on the GPU's own trajectory."""
import numpy as np
import pytest

import dfx
import oracle_py as O
from conftest import forward_inputs, rel_l2

pytestmark = pytest.mark.gpu

LOGITS_REL_L2 = 1e-2
ARGMAX_AGREE = 0.99


@pytest.mark.parametrize("arch,scheme", [(a, s) for a in ("llada", "dream") for s in ("q4_k_m", "q8_0", "f16")] +
                         [("llada_longk", "q4_k_m"), ("llada_longk", "f16")])
def test_forward_logits_match_oracle(gpu, request, arch, scheme):
    models = request.getfixturevalue("longk_models" if arch == "llada_longk" else "tiny_models")
    path = models[(arch, scheme)]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    ctx.set_attention(dfx.ATTN_EXACT)
    for toks in forward_inputs(om.dims["V"]):
        n = len(toks)
        ref = om.forward_full(toks)
        got = ctx.forward(toks)
        assert rel_l2(got, ref) <= LOGITS_REL_L2, (n, rel_l2(got, ref))
        assert np.mean(got.argmax(1) == ref.argmax(1)) >= ARGMAX_AGREE
        if scheme != "f16":
            # quantised weights with exact attention: every op repeats the oracle's
            # arithmetic, so the logits are the same floats (F16 GEMMs accumulate in
            # another order)
            assert np.array_equal(got, ref), (n, rel_l2(got, ref), np.mean(got == ref))
    ctx.close()
    model.close()


@pytest.mark.parametrize("arch,scheme", [(a, s) for a in ("llada", "dream") for s in ("q4_k_m", "q8_0", "f16")] +
                         [("llada_longk", "q4_k_m"), ("llada_longk", "f16")])
def test_forward_default_attention_meets_bar(gpu, request, arch, scheme):
    """The default split-bf16 attention (f32-accurate products, another rounding than the
    oracle's f64 sums) through the whole forward.  Where the oracle's own logits are
    stable (they move by < 1e-4 under f32-level perturbations: every F16 case, and the
    quantised inputs without a rounding cascade) the north-star bar holds, and the logits
    stay within 1e-3 of the exact mode's.  Where they are not (int8 activations: one
    flipped rounding spreads through attention into a cascade, see
    test_oracle_conditioning) the result is held to the size of such cascades, 5e-2,
    with the oracle's instability on that input shown."""
    from test_oracle_conditioning import oracle_spread
    models = request.getfixturevalue("longk_models" if arch == "llada_longk" else "tiny_models")
    path = models[(arch, scheme)]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    for toks in forward_inputs(om.dims["V"]):
        n = len(toks)
        ref = om.forward_full(toks)
        ctx.set_attention(dfx.ATTN_EXACT)
        exact = ctx.forward(toks)
        ctx.set_attention(dfx.ATTN_SPLIT_BF16)
        got = ctx.forward(toks)
        err = rel_l2(got, ref)
        if scheme == "f16" or oracle_spread(om, toks) < 1e-4:
            assert err <= LOGITS_REL_L2, (n, err)
            assert np.mean(got.argmax(1) == ref.argmax(1)) >= ARGMAX_AGREE
            assert rel_l2(got, exact) <= 1e-3, (n, rel_l2(got, exact))
        else:
            assert err <= 5e-2, (n, err)
    ctx.close()
    model.close()


class Replay:
    """The reference loop (src/diffuse-sampler.cpp:60-340 with src/diffuse-cache.h) run
    on the oracle, but unmasking what the GPU unmasked (teacher forcing).  At every step
    the GPU's choice must be the oracle's, except across near-ties of the ordering key."""

    def __init__(self, om, prompt, n_gen, p):
        self.om, self.p = om, p
        self.P, self.N = len(prompt), len(prompt) + n_gen
        self.V = om.dims["V"]
        self.mask = int(om.m.mask_token_id)
        self.seq = np.concatenate([prompt, np.full(n_gen, self.mask, np.int32)]).astype(np.int32)
        self.masked = np.zeros(self.N, bool)
        self.masked[self.P:] = True
        self.logits = np.zeros((self.N, self.V), np.float32)
        self.kv = om.new_kv(self.N)
        self.prev = np.full(self.N, -1, np.int32)
        self.last_changed = np.full(self.N, -1)
        self.cache_init = False
        self.shift = bool(om.m.is_dream)

    def step(self, s):
        p = self.p
        full = not p["use_cache"] or not self.cache_init or (p["cache_refresh"] > 0 and s > 0 and
                                                              s % p["cache_refresh"] == 0)
        if not full:
            act = []
            for i in range(self.N):
                changed = self.seq[i] != self.prev[i]
                if changed:
                    self.last_changed[i] = s
                recent = p["cache_keep_active"] > 0 and self.last_changed[i] >= 0 and \
                    s - self.last_changed[i] <= p["cache_keep_active"]
                if changed or self.masked[i] or recent:
                    act.append(i)
            if len(act) >= self.N or not act:
                full = True
        if full:
            self.logits[:] = self._full_kv() if p["use_cache"] else self.om.forward_full(self.seq)
        else:
            act = np.array(act, np.int32)
            self.logits[act] = self.om.forward_cached(self.kv, self.seq[act], act, self.N)
        if p["use_cache"]:
            self.prev = self.seq.copy()
            self.cache_init = True
        cand = []
        for i in np.nonzero(self.masked)[0]:
            row = self.logits[max(i - 1, 0) if self.shift else i]
            b, bv, sv = O.top2(row)
            conf = bv - sv if p["remasking"] == dfx.TOPK_MARGIN else bv
            cand.append((i, b, conf, O.entropy(row), row))
        return cand

    def _full_kv(self):
        logits, kv = self.om.forward_full(self.seq, kv_tokens=self.N)
        self.kv = kv
        return logits


def key_of(c, remasking):
    return c[3] if remasking == dfx.ENTROPY_EXIT else -c[2]


# The loop is replayed with the exact attention, whose logits are the oracle's floats on
# quantised models, so that a cascade of flipped activation roundings (one f32-level
# change in the attention spreads into ~1e-2 moves of the logits on these models; see
# test_oracle_conditioning) cannot hide or fake a loop difference.  Two cases run the
# default split-bf16 attention: config-2 semantics on LLaDA Q4_K_M and the F16 model.
@pytest.mark.parametrize("arch,scheme,remasking,use_cache,B,attn", [
    ("llada", "q4_k_m", dfx.LOW_CONFIDENCE, False, 64, dfx.ATTN_EXACT),     # config-0 semantics at test size
    ("llada", "q4_k_m", dfx.ENTROPY_EXIT, True, 64, dfx.ATTN_EXACT),        # config-2 semantics
    ("llada", "q8_0", dfx.MASKGIT_PLUS, True, 48, dfx.ATTN_EXACT),
    ("llada", "f16", dfx.TOPK_MARGIN, True, 40, dfx.ATTN_EXACT),
    ("dream", "q4_k_m", dfx.ENTROPY_EXIT, True, 64, dfx.ATTN_EXACT),        # config-1 semantics (shift + GQA + bias)
    ("dream", "q4_k_m", dfx.LOW_CONFIDENCE, False, 32, dfx.ATTN_EXACT),
    ("llada", "q4_k_m", dfx.ENTROPY_EXIT, True, 64, dfx.ATTN_SPLIT_BF16),
    ("llada", "f16", dfx.TOPK_MARGIN, True, 40, dfx.ATTN_SPLIT_BF16),
])
def test_generate_replays_through_oracle(gpu, tiny_models, arch, scheme, remasking, use_cache, B, attn):
    path = tiny_models[(arch, scheme)]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, om.dims["V"] - 16, 32).astype(np.int32)
    n_steps = 16
    ctx = dfx.Context(model, len(prompt) + B)
    ctx.set_attention(attn)
    params = dfx.SamplerParams.make(n_steps=n_steps, remasking=remasking, use_cache=use_cache, entropy_threshold=1.5)
    toks, when = ctx.generate_trace(prompt, B, params)
    assert (when >= 0).all() and (when < n_steps).all()

    pd = dict(use_cache=use_cache, cache_refresh=0, cache_keep_active=0, remasking=remasking)
    rep = Replay(om, prompt, B, pd)
    n_masked = B
    for s in range(n_steps):
        if n_masked == 0:
            break
        cand = rep.step(s)
        n_sched = O.tokens_to_unmask(s, n_steps, n_masked, 0)
        gpu_set = set((np.nonzero(when == s)[0] + len(prompt)).tolist())
        keys = sorted(cand, key=lambda c: (key_of(c, remasking), c[0]))
        n_un = n_sched
        if remasking == dfx.ENTROPY_EXIT:
            n_easy = sum(1 for c in cand if c[3] < 1.5)
            n_un = min(max(n_sched, n_easy), len(cand))
        assert len(gpu_set) == n_un, (s, len(gpu_set), n_un)
        ora_set = {c[0] for c in keys[:n_un]}
        if gpu_set != ora_set:
            # only a near-tie at the cut may differ
            cut = key_of(keys[n_un - 1], remasking)
            tol = 1e-2 * max(1.0, abs(cut))
            for i in gpu_set ^ ora_set:
                c = next(c for c in cand if c[0] == i)
                assert abs(key_of(c, remasking) - cut) <= tol, (s, i, key_of(c, remasking), cut)
        for i in gpu_set:
            c = next(c for c in cand if c[0] == i)
            t = toks[i - len(prompt)]
            if t != c[1]:        # argmax flips only between near-equal logits
                assert abs(c[4][t] - c[4][c[1]]) <= 1e-2 * max(1.0, abs(c[4][c[1]])), (s, i)
            rep.seq[i] = t
            rep.masked[i] = False
        n_masked -= len(gpu_set)
    assert n_masked == 0
    ctx.close()
    model.close()


def test_generate_cache_off_equals_full_forward_loop(gpu, tiny_models):
    """Without the cache every step is a full forward: the GPU's stats must say so."""
    path = tiny_models[("llada", "q4_k_m")]
    model = dfx.Model(path)
    ctx = dfx.Context(model, 96)
    st = dfx.GenStats()
    prompt = np.arange(32, dtype=np.int32)
    ctx.generate(prompt, 64, dfx.SamplerParams.make(n_steps=16, use_cache=False), st)
    assert st.actual_steps == 16
    assert list(st.rows_per_step[:16]) == [96] * 16
    assert sum(st.unmasked_per_step[:16]) == 64
    st2 = dfx.GenStats()
    ctx.generate(prompt, 64, dfx.SamplerParams.make(n_steps=16, use_cache=True), st2)
    rows = list(st2.rows_per_step[:16])
    assert rows[0] == 96 and all(r < 96 for r in rows[1:])
    ctx.close()
    model.close()


def test_contexts_generate_concurrently(gpu, tiny_models):
    """Independent sequences (the batched long-context workload's unit): several contexts
    share one model (read-only after load, as in the reference, main-bench.cpp:153) and
    generate at the same time from host threads, each on its own stream.  Every sequence
    must come out exactly as when it runs alone."""
    import threading
    path = tiny_models[("llada", "q8_0")]
    model = dfx.Model(path)
    V = model.hparams.n_vocab
    params = dfx.SamplerParams.make(n_steps=8, remasking=dfx.ENTROPY_EXIT, use_cache=True, entropy_threshold=1.5)
    prompts = [np.random.default_rng(40 + i).integers(0, V - 64, 48).astype(np.int32) for i in range(4)]
    ctxs = [dfx.Context(model, 48 + 32) for _ in prompts]
    alone = [c.generate(p, 32, params) for c, p in zip(ctxs, prompts)]
    together = [None] * len(prompts)
    errors = []

    def run(i):
        try:
            together[i] = ctxs[i].generate(prompts[i], 32, params)
        except Exception as e:   # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(prompts))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for a, b in zip(alone, together):
        assert b is not None and np.array_equal(a, b)
    for c in ctxs:
        c.close()
    model.close()
