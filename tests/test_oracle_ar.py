"""Independent pins of the oracle's autoregressive path (orc_ar_*).

The oracle restates src/ar-graph.cpp (causal graph over an append-only cache, sliding
window, layer skip, layer-impact profile) and src/ar-sampler.cpp (sample_token,
ar_generate).  Here:
  * the causal forward goes through transformers' own Llama / Qwen2 in float64 with its
    default causal mask, and the sliding window through an explicit 4-D mask built from
    the reference's rule (src/ar-graph.cpp:70-88: key k visible to query q when k <= q
    and q - k < window);
  * skipped layers are removed from the transformers model, and the layer impacts are
    measured there with forward hooks (sum of squared layer output - input);
  * prefill + decode steps must give the prefill's rows exactly (the cache holds the same
    floats as a longer prefill would compute);
  * the sampler is checked by properties that do not restate it: greedy picks of
    hand-made rows, the sampled distribution against softmax(l / T), the top-k / top-p
    support, determinism per seed, and the end-token rule of ar_generate.
"""
import numpy as np
import pytest

import oracle_py as O
from conftest import TINY_DREAM, TINY_LLADA, TINY_LLADA6, eos_model
from test_oracle_vs_transformers import BAR, _synth, compare, hf_model

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ar_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("ar")
    out = {}
    for name, arch in (("llada", TINY_LLADA), ("dream", TINY_DREAM), ("llada6", TINY_LLADA6)):
        for scheme in ("f32", "q4_k_m"):
            out[(name, scheme)] = _synth(d / f"{name}-{scheme}.gguf", arch, scheme, seed=31)
    return out


def _tokens(V, n, seed):
    return np.random.default_rng(seed).integers(0, V, n).astype(np.int32)


def hf_causal(model, tokens, window=0):
    ids = torch.from_numpy(np.asarray(tokens, dtype=np.int64))[None]
    n = ids.shape[1]
    q = np.arange(n)[:, None]
    k = np.arange(n)[None, :]
    vis = (k <= q) & ((window <= 0) | (q - k < window))
    mask = torch.from_numpy(np.where(vis, 0.0, -np.inf))[None, None]
    with torch.no_grad():
        return model(input_ids=ids, attention_mask=mask).logits[0].numpy()


def ar_prefill(om, toks, window=0, skip=None):
    cache = O.OracleArCache(om, len(toks) + 8, window)
    if skip is not None:
        cache.skip[:] = skip
    return om.ar_forward(cache, toks, n_threads=4), cache


@pytest.mark.parametrize("name", ["llada", "dream"])
def test_ar_prefill_matches_transformers_causal(ar_models, name):
    model, om = hf_model(ar_models[(name, "f32")])
    for n, seed in ((1, 1), (9, 2), (40, 3)):
        toks = _tokens(om.dims["V"], n, seed)
        ids = torch.from_numpy(toks.astype(np.int64))[None]
        with torch.no_grad():
            ref = model(input_ids=ids).logits[0].numpy()   # transformers' own causal mask
        got, _ = ar_prefill(om, toks)
        r = compare(got, ref)
        assert r["rel_l2"] <= BAR["f32"] and r["argmax"] == 1.0, (name, n, r)


@pytest.mark.parametrize("window", [1, 4, 17])
def test_ar_sliding_window_matches_transformers(ar_models, window):
    model, om = hf_model(ar_models[("dream", "f32")])
    toks = _tokens(om.dims["V"], 40, 5)
    got, _ = ar_prefill(om, toks, window=window)
    r = compare(got, hf_causal(model, toks, window))
    assert r["rel_l2"] <= BAR["f32"] and r["argmax"] == 1.0, (window, r)
    # and the window matters: the full causal mask gives other logits
    assert compare(got, hf_causal(model, toks, 0))["rel_l2"] > 100 * BAR["f32"]


def test_ar_layer_skip_matches_transformers(ar_models):
    path = ar_models[("llada6", "f32")]
    model, om = hf_model(path)
    skip = np.array([0, 0, 1, 0, 1, 0], np.uint8)
    model.model.layers = torch.nn.ModuleList([ly for i, ly in enumerate(model.model.layers) if not skip[i]])
    model.config.num_hidden_layers = int((skip == 0).sum())
    for i, ly in enumerate(model.model.layers):
        ly.self_attn.layer_idx = i
    toks = _tokens(om.dims["V"], 24, 7)
    got, _ = ar_prefill(om, toks, skip=skip)
    r = compare(got, hf_causal(model, toks))
    assert r["rel_l2"] <= BAR["f32"] and r["argmax"] == 1.0, r


def test_ar_layer_impact_matches_transformers(ar_models):
    model, om = hf_model(ar_models[("llada6", "f32")])
    toks = _tokens(om.dims["V"], 24, 8)
    imp_ref = []

    def hook(mod, args, kwargs, out):
        x_in = args[0] if args else kwargs["hidden_states"]
        x_out = out[0] if isinstance(out, tuple) else out
        imp_ref.append(float(((x_out - x_in) ** 2).sum()))
    hs = [ly.register_forward_hook(hook, with_kwargs=True) for ly in model.model.layers]
    hf_causal(model, toks)
    for h in hs:
        h.remove()
    cache = O.OracleArCache(om, 32)
    om.ar_forward(cache, toks, profile=True, n_threads=4)
    np.testing.assert_allclose(cache.impact, imp_ref, rtol=1e-5)
    # the profile pass runs every layer even with a skip mask set
    cache2 = O.OracleArCache(om, 32)
    cache2.skip[:] = [0, 0, 1, 1, 0, 0]
    om.ar_forward(cache2, toks, profile=True, n_threads=4)
    np.testing.assert_array_equal(cache2.impact, cache.impact)


def test_choose_skip_ranks_and_protects():
    """Lowest impacts first, ties by layer index; layers 0, 1, L-2, L-1 never skipped."""
    imp = np.array([0.1, 0.2, 5.0, 3.0, 3.0, 9.0, 0.0, 0.05], np.float32)
    skip, n = O.choose_skip(imp, 2)
    assert n == 2 and list(np.nonzero(skip)[0]) == [3, 4]
    skip, n = O.choose_skip(imp, 10)
    assert n == 4 and list(np.nonzero(skip)[0]) == [2, 3, 4, 5]
    skip, n = O.choose_skip(imp, 0)
    assert n == 0 and not skip.any()


@pytest.mark.parametrize("scheme", ["f32", "q4_k_m"])
@pytest.mark.parametrize("window", [0, 3])
def test_ar_decode_reproduces_prefill_rows(ar_models, scheme, window):
    """Prefill of n-3 tokens then three one-token passes gives, bit for bit, the rows of a
    prefill of all n (the append-only cache holds what the longer prefill computes)."""
    om = O.OracleModel(ar_models[("dream", scheme)])
    toks = _tokens(om.dims["V"], 20, 9)
    full, _ = ar_prefill(om, toks, window=window)
    cache = O.OracleArCache(om, 32, window)
    rows = [om.ar_forward(cache, toks[:17], n_threads=4)]
    for t in toks[17:]:
        rows.append(om.ar_forward(cache, [t], n_threads=4))
    np.testing.assert_array_equal(np.concatenate(rows), full)
    assert cache.c.n_past == 20
    last = O.OracleArCache(om, 32, window)
    np.testing.assert_array_equal(om.ar_forward(last, toks, last_only=True, n_threads=4)[0], full[-1])


# ---------------------------------------------------------------- sampler
def test_sample_greedy_rules():
    P = O.OrcArParams.make
    rng = O.oracle().orc_rng_new(1)
    try:
        row = np.array([1.0, 3.0, 3.0, -2.0, 2.8], np.float32)
        assert O.ar_sample(row, P(repeat_penalty=1.0), [], rng) == 1            # first maximum
        assert O.ar_sample(row, P(repeat_penalty=1.5), [1], rng) == 2           # 3/1.5 = 2 < 3
        assert O.ar_sample(row, P(repeat_penalty=1.5), [1, 2], rng) == 4        # both penalised
        assert O.ar_sample(row, P(repeat_penalty=1.05), [1, 2, 2], rng) == 1    # 3/1.05 > 2.8 > 3/1.05^2
        neg = np.array([-1.0, -0.5, -0.6], np.float32)
        assert O.ar_sample(neg, P(repeat_penalty=2.0), [1], rng) == 2           # -0.5 * 2 = -1
        assert O.ar_sample(np.array([np.nan, 5, 6], np.float32), P(), [], rng) == 0
        assert O.ar_sample(np.full(4, -np.inf, np.float32), P(), [], rng) == 0
        assert O.ar_sample(row, P(repeat_penalty=1.5), [99, -1], rng) == 1      # out-of-range ids ignored
    finally:
        O.oracle().orc_rng_free(rng)


def _draws(row, params, n, seed=3):
    rng = O.oracle().orc_rng_new(seed)
    try:
        return np.array([O.ar_sample(row, params, [], rng) for _ in range(n)])
    finally:
        O.oracle().orc_rng_free(rng)


def test_sample_temperature_distribution():
    row = np.array([0.3, 1.2, -0.4, 0.9, 0.0, 2.0, -1.0, 0.5], np.float32)
    T = 0.8
    got = np.bincount(_draws(row, O.OrcArParams.make(temperature=T, top_k=0, top_p=1.0, repeat_penalty=1.0),
                             20000), minlength=8)
    p = np.exp(row / T - (row / T).max())
    p /= p.sum()
    chi2 = float(((got - 20000 * p) ** 2 / (20000 * p)).sum())
    assert chi2 < 30.0, (chi2, got, p)    # 7 degrees of freedom: p(chi2 > 30) < 1e-4


def test_sample_top_k_and_top_p_support():
    rng = np.random.default_rng(4)
    row = rng.standard_normal(300).astype(np.float32)
    k = 10
    top = set(np.argsort(-row)[:k].tolist())
    d = _draws(row, O.OrcArParams.make(temperature=1.0, top_k=k, top_p=1.0, repeat_penalty=1.0), 3000)
    assert set(d.tolist()) <= top
    # top-p: probabilities 0.5, 0.3, 0.15, 0.05 and top_p 0.7 keep the first two only
    lp = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    d = _draws(lp, O.OrcArParams.make(temperature=1.0, top_k=0, top_p=0.7, repeat_penalty=1.0), 4000)
    assert set(d.tolist()) == {0, 1}
    assert abs(np.mean(d == 0) - 0.625) < 0.03
    # the same seed gives the same draws
    np.testing.assert_array_equal(d, _draws(lp, O.OrcArParams.make(temperature=1.0, top_k=0, top_p=0.7,
                                                                         repeat_penalty=1.0), 4000))


def test_ar_generate_stops_at_end_token(tmp_path):
    om = O.OracleModel(eos_model(tmp_path / "eos.gguf"))
    out, _ = om.ar_generate(np.arange(5, 12, dtype=np.int32), 6, O.OrcArParams.make(), n_threads=4)
    assert len(out) == 1 and out[0] in (151643, 151645), out
    # max_tokens = 0 still samples the prefill's token (src/ar-sampler.cpp:231-247)
    out0, _ = om.ar_generate(np.arange(5, 12, dtype=np.int32), 0, O.OrcArParams.make(), n_threads=4)
    assert len(out0) == 1 and out0[0] == out[0]


def test_ar_generate_layer_skip_choice(ar_models):
    """ar_generate with layer_skip profiles the prompt and skips the lowest-impact
    unprotected layers (the mask returned equals choose_skip of the impacts)."""
    om = O.OracleModel(ar_models[("llada6", "q4_k_m")])
    prompt = _tokens(om.dims["V"], 12, 10)
    out, skip = om.ar_generate(prompt, 5, O.OrcArParams.make(layer_skip=1), n_threads=4)
    cache = O.OracleArCache(om, 32)
    om.ar_forward(cache, prompt, profile=True, n_threads=4)
    want, n = O.choose_skip(cache.impact, 1)
    assert n == 1
    np.testing.assert_array_equal(skip, want)
    assert len(out) == 5
