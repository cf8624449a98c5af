"""Parity of the autoregressive path on the GPU (dfx_ar_*, dfx_attention_causal,
dfx_ar_greedy) with the oracle's restatement of src/ar-graph.cpp and src/ar-sampler.cpp:
causal prefill and decode logits (the same floats on quantised weights), the sliding
window, the layer-impact profile and skip choice, the greedy kernel's rules, and whole
ar_generate runs compared token for token (greedy on the device, sampled on the host)."""
import numpy as np
import pytest

import dfx
import oracle_py as O
from conftest import TINY_LLADA6, eos_model, rel_l2

pytestmark = pytest.mark.gpu

L = dfx.lib


@pytest.fixture(scope="module")
def ar_models(tiny_models, model_dir):
    out = dict(tiny_models)
    for name, arch, scheme in (("llada6", TINY_LLADA6, "q4_k_m"), ("llada6", TINY_LLADA6, "f32")):
        p = model_dir / f"{name}-{scheme}.gguf"
        dfx.synth_model(p, arch, scheme=scheme, seed=19, sigma=0.05, n_threads=4)
        out[(name, scheme)] = str(p)
    return out


def _tokens(V, n, seed):
    return np.random.default_rng(seed).integers(0, V, n).astype(np.int32)


def _same(got, ref, scheme, what):
    """Quantised weights: the same floats.  F16 / F32 GEMMs sum in another order (f32
    accumulation): F32 within f32 rounding, F16 within the logits bar."""
    if scheme in ("q4_k_m", "q8_0"):
        assert np.array_equal(got, ref), (what, rel_l2(got, ref), np.mean(got == ref))
    elif scheme == "f32":
        assert rel_l2(got, ref) <= 1e-5, (what, rel_l2(got, ref))
    else:
        assert rel_l2(got, ref) <= 1e-2 and np.mean(got.argmax(1) == ref.argmax(1)) >= 0.99, (what, rel_l2(got, ref))


# ---------------------------------------------------------------- kernel level
CAUSAL_SHAPES = [  # M, n_keys, q_pos0, window, H, Hkv, hd
    (7, 30, 23, 0, 4, 2, 128), (7, 30, 23, 5, 4, 2, 128), (1, 300, 299, 0, 8, 8, 64), (33, 33, 0, 0, 4, 4, 128),
    (33, 33, 0, 8, 6, 3, 64), (16, 100, 40, 1, 2, 2, 128),
    # score rows longer than the LDS holds: the three-pass kernel
    (3, 3000, 2997, 0, 2, 1, 128), (20, 2800, 2700, 700, 4, 2, 64)]


@pytest.mark.parametrize("M,n_keys,q_pos0,window,H,Hkv,hd", CAUSAL_SHAPES)
def test_attention_causal_matches_oracle(gpu, M, n_keys, q_pos0, window, H, Hkv, hd):
    """dfx_attention_causal against the oracle's causal attention (same f64 sums, masked keys
    weigh exactly zero): equal except where two f64 summation orders straddle an f32
    rounding boundary (at most one ulp, about one element in 10^6-10^7)."""
    rng = np.random.default_rng(M * 1000 + n_keys)
    q = rng.standard_normal((M, H, hd)).astype(np.float32)
    k = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v_ld = (n_keys + 15) // 16 * 16 + 16
    vt = np.full((Hkv, hd, v_ld), np.nan, np.float32)
    vt[:, :, :n_keys] = v.transpose(1, 2, 0)
    qb, kb, vb, ob = dfx.Buf.of(q), dfx.Buf.of(k), dfx.Buf.of(vt), dfx.Buf(M * H * hd * 4)
    dfx.check(L().dfx_attention_causal(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, q_pos0, window, ob.ptr,
                                       None), "attention_causal")
    got = ob.download(np.float32, shape=(M, H, hd))
    ref = O.attention_causal(q, k, v, np.arange(q_pos0, q_pos0 + M), np.arange(n_keys), window)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps > 0).mean() <= 1e-5, (int(ulps.max()), int((ulps > 0).sum()))


@pytest.mark.parametrize("M,n_keys,q_pos0,window,H,Hkv,hd", [
    (1, 192, 191, 0, 28, 4, 128),      # Dream-7B decode: one row, GQA 28 / 4
    (1, 1024, 1023, 0, 8, 2, 64),      # the most keys of the few-row kernel
    (4, 700, 696, 100, 4, 1, 128),     # four rows with a window
    (2, 65, -1, 0, 4, 4, 128)])        # bidirectional (no mask)
def test_attention_few_rows_matches_oracle(gpu, M, n_keys, q_pos0, window, H, Hkv, hd):
    """At most 4 query rows and 1024 keys (decoding): one workgroup per row and head.  The same
    f64 sums of exact products as the oracle in another order: equal floats except where two
    orders straddle an f32 rounding boundary (at most one ulp, rare)."""
    rng = np.random.default_rng(M * 7 + n_keys)
    q = rng.standard_normal((M, H, hd)).astype(np.float32)
    k = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v_ld = (n_keys + 15) // 16 * 16 + 16
    vt = np.full((Hkv, hd, v_ld), np.nan, np.float32)
    vt[:, :, :n_keys] = v.transpose(1, 2, 0)
    qb, kb, vb, ob = dfx.Buf.of(q), dfx.Buf.of(k), dfx.Buf.of(vt), dfx.Buf(M * H * hd * 4)
    if q_pos0 >= 0:
        dfx.check(L().dfx_attention_causal(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, q_pos0, window,
                                           ob.ptr, None), "attention_causal")
        ref = O.attention_causal(q, k, v, np.arange(q_pos0, q_pos0 + M), np.arange(n_keys), window)
    else:
        dfx.check(L().dfx_attention(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, ob.ptr, None), "attention")
        ref = O.attention(q, k, v)
    got = ob.download(np.float32, shape=(M, H, hd))
    ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps > 0).sum() <= 2, (int(ulps.max()), int((ulps > 0).sum()))


def test_attention_causal_rejects_queries_past_the_keys(gpu):
    b = dfx.Buf(1 << 16)
    rc = L().dfx_attention_causal(b.ptr, b.ptr, b.ptr, 32, 4, 20, 2, 2, 128, 17, 0, b.ptr, None)
    assert rc == -2 and b"within the keys" in L().dfx_last_error()


def _greedy_ref(row, recent, penalty):
    return O.ar_sample(row, O.OrcArParams.make(temperature=0.0, repeat_penalty=penalty), recent, 0)


def test_ar_greedy_kernel_rules(gpu):
    """dfx_ar_greedy against the oracle's sample_token at temperature 0 on rows with ties,
    NaN / -inf, negative logits and a penalty ring that wraps; checks the state update."""
    rng = np.random.default_rng(3)
    V, R = 5000, 4
    cases = []
    row = rng.standard_normal(V).astype(np.float32)
    row[[17, 4000]] = row.max() + 1.0                      # tie: the first index wins
    cases.append((row, [], 1.1))
    cases.append((row, [17], 1.3))                         # penalised: the second copy wins
    cases.append((row, [17, 4000, 17], 1.3))
    neg = -np.abs(rng.standard_normal(V)).astype(np.float32)
    cases.append((neg, [int(neg.argmax())], 2.0))          # negative logits: multiplied
    nan0 = row.copy()
    nan0[0] = np.nan
    cases.append((nan0, [], 1.1))
    cases.append((np.full(V, -np.inf, np.float32), [], 1.1))
    cases.append((row, [17, 4000], 1.0))                   # penalty 1: none applied
    for row, recent, pen in cases:
        st = np.zeros(4 + R, np.int32)
        st[1] = 41
        st[2] = min(len(recent), R)
        st[3] = 2
        for j, t in enumerate(recent[:R]):
            st[4 + (2 + j) % R] = t
        rb, sb, tb = dfx.Buf.of(row), dfx.Buf.of(st), dfx.Buf(4)
        dfx.check(L().dfx_ar_greedy(rb.ptr, V, sb.ptr, R, pen, tb.ptr, None), "ar_greedy")
        tok = int(tb.download(np.int32, 1)[0])
        want = _greedy_ref(row, recent, pen)
        assert tok == want, (recent, pen, tok, want)
        s2 = sb.download(np.int32, 4 + R)
        assert s2[0] == tok and s2[1] == 42
        ring_before = [st[4 + (st[3] + j) % R] for j in range(st[2])]
        ring_after = [s2[4 + (s2[3] + j) % R] for j in range(s2[2])]
        assert ring_after == (ring_before + [tok])[-R:]


# ---------------------------------------------------------------- forward passes
AR_CASES = [("llada", "q4_k_m"), ("dream", "q4_k_m"), ("dream", "q8_0"), ("llada", "f16"), ("llada6", "f32")]


@pytest.mark.parametrize("arch,scheme", AR_CASES)
@pytest.mark.parametrize("window", [0, 5])
def test_ar_prefill_and_decode_match_oracle(gpu, ar_models, arch, scheme, window):
    path = ar_models[(arch, scheme)]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    toks = _tokens(om.dims["V"], 24, 4)
    cache = O.OracleArCache(om, 64, window)
    got = ctx.ar_forward(toks[:20], reset=True, sliding_window=window)
    _same(got, om.ar_forward(cache, toks[:20]), scheme, "prefill")
    for i in range(20, 24):
        got = ctx.ar_forward(toks[i:i + 1], sliding_window=window)
        _same(got, om.ar_forward(cache, toks[i:i + 1]), scheme, f"decode {i}")
    # a batch of 3 after the decodes (ar_forward_batch), then a reset
    more = _tokens(om.dims["V"], 3, 5)
    _same(ctx.ar_forward(more, sliding_window=window), om.ar_forward(cache, more), scheme, "batch")
    cache2 = O.OracleArCache(om, 64, window)
    _same(ctx.ar_forward(toks[:6], reset=True, sliding_window=window), om.ar_forward(cache2, toks[:6]), scheme,
          "reset")
    ctx.close()
    model.close()


def test_ar_long_context(gpu, ar_models):
    """2600-position prompt (score rows past the LDS: the three-pass attention), then two
    decodes, full causal and with a window.  Over this many rows a one-ulp attention
    difference (two f64 summation orders) can move one int8 activation step, so the check is
    the logits bar plus at least 99% of the rows bit-identical."""
    path = ar_models[("llada", "q4_k_m")]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 2608)
    toks = _tokens(om.dims["V"], 2602, 6)
    for window in (0, 700):
        cache = O.OracleArCache(om, 2608, window)
        got = ctx.ar_forward(toks[:2600], reset=True, sliding_window=window)
        ref = om.ar_forward(cache, toks[:2600])
        same_rows = np.mean(np.all(got == ref, axis=1))
        assert rel_l2(got, ref) <= 1e-2 and np.mean(got.argmax(1) == ref.argmax(1)) >= 0.99, window
        assert same_rows >= 0.99, (window, same_rows)
        for i in (2600, 2601):
            g1, r1 = ctx.ar_forward(toks[i:i + 1], sliding_window=window), om.ar_forward(cache, toks[i:i + 1])
            assert rel_l2(g1, r1) <= 1e-2 and g1.argmax() == r1.argmax(), (window, i)
    ctx.close()
    model.close()


def test_ar_profile_layers_matches_oracle(gpu, ar_models):
    path = ar_models[("llada6", "q4_k_m")]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    toks = _tokens(om.dims["V"], 30, 7)
    logits, imp, skip = ctx.ar_profile_layers(toks[:26], n_skip=2)
    cache = O.OracleArCache(om, 64)
    ref = om.ar_forward(cache, toks[:26], profile=True)
    assert np.array_equal(logits, ref)
    assert np.array_equal(imp, cache.impact), (imp, cache.impact)
    want, n = O.choose_skip(cache.impact, 2)
    assert n == 2 and np.array_equal(skip, want)
    cache.skip[:] = want
    for i in range(26, 30):     # decodes leave the skipped layers out
        assert np.array_equal(ctx.ar_forward(toks[i:i + 1]), om.ar_forward(cache, toks[i:i + 1])), i
    ctx.close()
    model.close()


# ---------------------------------------------------------------- ar_generate
GEN_CASES = [
    ("llada", "q4_k_m", dict()),                                           # greedy, penalty 1.1 over 64
    ("llada", "q4_k_m", dict(repeat_penalty=1.5, repeat_last_n=3)),       # the ring wraps
    ("dream", "q4_k_m", dict(sliding_window=4)),
    ("llada6", "q4_k_m", dict(layer_skip=2)),
    ("dream", "q8_0", dict(repeat_penalty=1.0)),
    ("llada", "q4_k_m", dict(temperature=0.8, seed=7)),                    # top-k 40, top-p 0.9
    ("dream", "q4_k_m", dict(temperature=1.2, top_k=0, top_p=1.0, seed=3)),
    ("llada", "q8_0", dict(temperature=0.5, top_k=5, top_p=0.5, repeat_penalty=1.5, seed=11)),
    ("llada6", "q4_k_m", dict(temperature=0.9, layer_skip=1, sliding_window=6, seed=5)),
]


@pytest.mark.parametrize("arch,scheme,kw", GEN_CASES)
def test_ar_generate_matches_oracle(gpu, ar_models, arch, scheme, kw):
    path = ar_models[(arch, scheme)]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    prompt = _tokens(om.dims["V"], 10, 8)
    st = dfx.ArStats()
    got = ctx.ar_generate(prompt, 24, dfx.ArParams.make(**kw), stats=st)
    ref, skip = om.ar_generate(prompt, 24, O.OrcArParams.make(**kw))
    assert list(got) == list(ref), (kw, list(got), list(ref))
    assert st.n_generated == len(got) == 24 and st.n_decoded == 23 and st.n_prompt == 10
    assert st.n_skipped_layers == int(skip.sum())
    ctx.close()
    model.close()


def test_ar_generate_end_token_callback_and_zero(gpu, ar_models, tmp_path):
    path = eos_model(tmp_path / "eos.gguf")
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 32)
    prompt = np.arange(5, 12, dtype=np.int32)
    got = ctx.ar_generate(prompt, 6, dfx.ArParams.make())
    ref, _ = om.ar_generate(prompt, 6, O.OrcArParams.make())
    assert list(got) == list(ref) and len(got) == 1 and got[0] in (151643, 151645)
    assert list(ctx.ar_generate(prompt, 0, dfx.ArParams.make())) == list(ref)   # max_tokens 0: one token
    ctx.close()
    model.close()
    # the callback stops the generation after the token it returns false for
    path = ar_models[("llada", "q4_k_m")]
    om = O.OracleModel(path)
    model = dfx.Model(path)
    ctx = dfx.Context(model, 64)
    prompt = _tokens(om.dims["V"], 10, 9)
    seen = []
    got = ctx.ar_generate(prompt, 20, dfx.ArParams.make(), callback=lambda t, p: seen.append((t, p)) or p < 12)
    ref, _ = om.ar_generate(prompt, 20, O.OrcArParams.make())
    assert list(got) == list(ref[:3]) and seen == [(int(t), 10 + i) for i, t in enumerate(ref[:3])]
    ctx.close()
    model.close()
