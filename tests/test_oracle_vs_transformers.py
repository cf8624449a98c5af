"""Independent pin of the oracle's forward composition.

The oracle (oracle/oracle.cpp run_layers) restates the reference graph of
src/diffuse-graph.cpp:11-160.  Here the same GGUF weights go into Hugging Face
transformers' own Llama (LLaDA's backbone) and Qwen2 (Dream's) implementations,
run in float64 with an all-zero 4-D attention mask (bidirectional, as the reference
graph: no causal mask, src/diffuse-graph.cpp:107-114), and the two sets of logits are
compared with the reference's own comparison metrics (tools/compare-logits.py:96-129:
max / mean abs diff, cosine, argmax agreement; here also relative L2).

transformers is a separate implementation of the layer wiring (residuals, SwiGLU
order, GQA head grouping, Q/K/V bias, rotate-half RoPE, tied head), so a mistake
in the oracle's composition fails here, whereas the oracle's self-consistency tests
(cached == full) would not see it.  The negative controls below plant such mistakes
on the transformers side and check that the comparison then fails.

HF's RMSNorm and rotary tables compute in float32 internally; they are replaced by
float64 forms of the same formulas so that the reference side carries no f32
rounding of its own.  F32 weights (the converters' default output type,
tools/convert-llada.py --type f32) leave the oracle with only f32 rounding, hence
the tight bar; F16 weights add GGML's f16 activation conversion before every
mul_mat (the vec_dot_type of F16), a ~1e-4-level difference per product.
"""
import numpy as np
import pytest

import oracle_py as O
from conftest import TINY_DREAM, TINY_LLADA

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")


def _synth(path, arch, scheme, seed, tied=False):
    import dfx
    dfx.synth_model(path, arch, scheme=scheme, seed=seed, sigma=0.05, n_threads=4, tied_output=tied)
    return str(path)


def _mat(g, name):
    """GGUF tensor as float64 [ne1][ne0] (= torch Linear [out][in])."""
    ti = g.tensor(name)
    if ti is None:
        return None
    n0, rows, t = ti["ne"][0], ti["rows"], ti["type"]
    raw = np.asarray(ti["data"])
    if t == O.F32:
        a = raw.view(np.float32).reshape(rows, n0)
    elif t == O.F16:
        a = raw.view(np.float16).reshape(rows, n0)
    else:
        rb = O.row_bytes(t, n0)
        a = np.stack([O.dequant(t, raw[r * rb:(r + 1) * rb], n0) for r in range(rows)])
    return torch.from_numpy(np.array(a, dtype=np.float64))


def _f64_norm(mod):
    eps = mod.variance_epsilon

    def fwd(x):
        return mod.weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))
    mod.forward = fwd


def _f64_rope(rot, hd, base):
    inv = torch.tensor([base ** (-(2.0 * i) / hd) for i in range(hd // 2)], dtype=torch.float64)

    def fwd(x, position_ids):
        f = position_ids[:, :, None].to(torch.float64) * inv[None, None, :]
        emb = torch.cat((f, f), dim=-1)
        return emb.cos(), emb.sin()
    rot.forward = fwd


def hf_model(path, swap_gate_up=False, rope_interleaved=False, gqa_modulo=False):
    """transformers model (float64) holding the GGUF file's weights."""
    g = O.GGUF(path)
    om = O.OracleModel(path)
    D = om.dims
    dream = bool(om.m.is_dream)
    tied = g.tensor("output.weight") is None
    common = dict(vocab_size=D["V"], hidden_size=D["d"], intermediate_size=D["F"], num_hidden_layers=D["L"],
                  num_attention_heads=D["H"], num_key_value_heads=D["Hkv"], rms_norm_eps=float(om.m.rms_norm_eps),
                  rope_theta=float(om.m.rope_theta), max_position_embeddings=4096, tie_word_embeddings=tied,
                  attn_implementation="eager")
    if dream:
        from transformers import Qwen2Config, Qwen2ForCausalLM
        model = Qwen2ForCausalLM(Qwen2Config(**common))
    else:
        from transformers import LlamaConfig, LlamaForCausalLM
        model = LlamaForCausalLM(LlamaConfig(attention_bias=False, mlp_bias=False, **common))
    model = model.double().eval()
    hd = D["hd"]

    def interleave(w, n_heads):
        # rotate pairs (2i, 2i+1) instead of (i, i + hd/2): the other RoPE convention
        w = w.reshape(n_heads, 2, hd // 2, -1).transpose(1, 2).reshape(n_heads * hd, -1)
        return w

    def head_modulo(w, n_heads, n_kv):
        # query head h made to read KV head h % n_kv instead of h // (n_heads / n_kv)
        rep = n_heads // n_kv
        perm = [(h % rep) * n_kv + h // rep for h in range(n_heads)]
        return w.reshape(n_heads, hd, -1)[perm].reshape(n_heads * hd, -1)

    with torch.no_grad():
        base = model.model
        base.embed_tokens.weight.copy_(_mat(g, "token_embd.weight"))
        base.norm.weight.copy_(_mat(g, "output_norm.weight").reshape(-1))
        if not tied:
            model.lm_head.weight.copy_(_mat(g, "output.weight"))
        for i, ly in enumerate(base.layers):
            p = f"blk.{i}."
            at, mlp = ly.self_attn, ly.mlp
            ly.input_layernorm.weight.copy_(_mat(g, p + "attn_norm.weight").reshape(-1))
            ly.post_attention_layernorm.weight.copy_(_mat(g, p + "ffn_norm.weight").reshape(-1))
            wq, wk = _mat(g, p + "attn_q.weight"), _mat(g, p + "attn_k.weight")
            if rope_interleaved:
                wq, wk = interleave(wq, D["H"]), interleave(wk, D["Hkv"])
            if gqa_modulo:
                wq = head_modulo(wq, D["H"], D["Hkv"])
            at.q_proj.weight.copy_(wq)
            at.k_proj.weight.copy_(wk)
            at.v_proj.weight.copy_(_mat(g, p + "attn_v.weight"))
            at.o_proj.weight.copy_(_mat(g, p + "attn_output.weight"))
            if dream:
                bq = _mat(g, p + "attn_q.bias").reshape(-1)
                at.q_proj.bias.copy_(head_modulo(bq[:, None], D["H"], D["Hkv"]).reshape(-1) if gqa_modulo else bq)
                at.k_proj.bias.copy_(_mat(g, p + "attn_k.bias").reshape(-1))
                at.v_proj.bias.copy_(_mat(g, p + "attn_v.bias").reshape(-1))
            wg, wu = _mat(g, p + "ffn_gate.weight"), _mat(g, p + "ffn_up.weight")
            if swap_gate_up:
                wg, wu = wu, wg
            mlp.gate_proj.weight.copy_(wg)
            mlp.up_proj.weight.copy_(wu)
            mlp.down_proj.weight.copy_(_mat(g, p + "ffn_down.weight"))
        for mod in model.modules():
            if type(mod).__name__.endswith("RMSNorm"):
                _f64_norm(mod)
        _f64_rope(base.rotary_emb, hd, float(om.m.rope_theta))
    return model, om


def hf_logits(model, tokens):
    ids = torch.from_numpy(np.asarray(tokens, dtype=np.int64))[None]
    n = ids.shape[1]
    mask = torch.zeros(1, 1, n, n, dtype=torch.float64)   # bidirectional: nothing masked
    with torch.no_grad():
        return model(input_ids=ids, attention_mask=mask).logits[0].numpy()


def compare(got, ref):
    """tools/compare-logits.py:96-129 metrics plus relative L2."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    cos = np.sum(got * ref, 1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1))
    return dict(max_abs=float(np.abs(got - ref).max()), mean_abs=float(np.abs(got - ref).mean()),
                min_cos=float(cos.min()), argmax=float(np.mean(got.argmax(1) == ref.argmax(1))),
                rel_l2=float(np.linalg.norm(got - ref) / np.linalg.norm(ref)))


# bars: F32 weights leave f32 rounding only; F16 adds the f16 activation conversion
BAR = {"f32": 1e-5, "f16": 2e-3}

CASES = [("llada", TINY_LLADA, False), ("dream", TINY_DREAM, False), ("llada_tied", TINY_LLADA, True)]


@pytest.fixture(scope="module")
def hf_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("hf")
    out = {}
    for name, arch, tied in CASES:
        for scheme in ("f32", "f16"):
            out[(name, scheme)] = _synth(d / f"{name}-{scheme}.gguf", arch, scheme, seed=21, tied=tied)
    return out


def _tokens(V, n, seed):
    return np.random.default_rng(seed).integers(0, V, n).astype(np.int32)


@pytest.mark.parametrize("name", [c[0] for c in CASES])
@pytest.mark.parametrize("scheme", ["f32", "f16"])
def test_oracle_forward_matches_transformers(hf_models, name, scheme):
    model, om = hf_model(hf_models[(name, scheme)])
    for n, seed in ((1, 1), (7, 2), (48, 3)):
        toks = _tokens(om.dims["V"], n, seed)
        got, ref = om.forward_full(toks, n_threads=4), hf_logits(model, toks)
        r = compare(got, ref)
        assert r["rel_l2"] <= BAR[scheme], (name, scheme, n, r)
        assert r["min_cos"] > 1 - 10 * BAR[scheme], (name, scheme, n, r)
        if scheme == "f32":
            assert r["argmax"] == 1.0, (name, scheme, n, r)
        else:
            # f16 activation rounding may reorder a near-tie: every disagreement must be
            # a pair of reference logits closer than twice that row's largest difference
            for i in np.nonzero(got.argmax(1) != ref.argmax(1))[0]:
                gap = ref[i, ref[i].argmax()] - ref[i, got[i].argmax()]
                assert gap <= 2 * np.abs(got[i] - ref[i]).max(), (name, n, i, gap)
            assert r["argmax"] >= 0.9, (name, scheme, n, r)


@pytest.mark.parametrize("mistake,name", [("swap_gate_up", "llada"), ("rope_interleaved", "llada"),
                                          ("gqa_modulo", "dream"), ("swap_gate_up", "dream")])
def test_planted_mistakes_fail_the_pin(hf_models, mistake, name):
    """The same comparison with one composition mistake planted on the reference side:
    the F32 bar must fail by orders of magnitude."""
    model, om = hf_model(hf_models[(name, "f32")], **{mistake: True})
    toks = _tokens(om.dims["V"], 48, 3)
    r = compare(om.forward_full(toks, n_threads=4), hf_logits(model, toks))
    assert r["rel_l2"] > 100 * BAR["f32"], (mistake, r)


def test_causal_mask_fails_the_pin(hf_models):
    """The reference graph has no causal mask; transformers' default (causal) attention
    must disagree with the oracle on a multi-token input."""
    model, om = hf_model(hf_models[("llada", "f32")])
    toks = _tokens(om.dims["V"], 48, 3)
    ids = torch.from_numpy(toks.astype(np.int64))[None]
    with torch.no_grad():
        causal = model(input_ids=ids).logits[0].numpy()
    r = compare(om.forward_full(toks, n_threads=4), causal)
    assert r["rel_l2"] > 100 * BAR["f32"], r
