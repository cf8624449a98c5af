"""CPU checks of the C ABI library: exports, encoders, GGUF files, weight repacking."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import dfx
import oracle_py as O
from conftest import REPO, TINY_DREAM, TINY_LLADA

rng = np.random.default_rng(99)


def header_functions(path):
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(dfx_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_function():
    lib = dfx.lib()
    names = header_functions(os.path.join(REPO, "include", "dfx.h"))
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_cpp_api_symbols_exported():
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", dfx.LIB_PATH], capture_output=True, text=True).stdout
    for sym in ("diffuse_model_load(", "diffuse_model_free(", "diffuse_model_hparams(", "diffuse_context_new(",
                "diffuse_context_free(", "diffuse_forward(", "diffuse_generate(", "ar_generate(",
                "ar_speculative_generate("):
        assert sym in out, sym


def test_reference_callers_compile_against_diffuse_h(tmp_path):
    """A program written against diffuse.h (defaults of include/diffuse.h:15-55 as
    tests/test-forward.cpp:16-34 asserts them) builds and links with libdiffuse."""
    src = tmp_path / "caller.cpp"
    src.write_text(r'''
#include "diffuse.h"
#include <cstdio>
int main() {
    diffuse_hparams hp; diffuse_sampler_params sp;
    if (hp.n_vocab != 0 || hp.rope_theta != 500000.0f || hp.rms_norm_eps != 1e-5f || hp.n_embd_head() != 0) return 1;
    if (sp.n_steps != 32 || sp.temperature != 0.0f || sp.schedule != diffuse_schedule::COSINE ||
        sp.remasking != diffuse_remasking::LOW_CONFIDENCE || sp.seed != 42u || sp.entropy_threshold != 1.5f ||
        !sp.use_cache || sp.cache_refresh != 0 || sp.cache_keep_active != 0) return 2;
    if ((int)diffuse_remasking::TOPK_MARGIN != 4 || (int)diffuse_schedule::LINEAR != 1) return 3;
    diffuse_model * (*load)(const std::string &, int) = &diffuse_model_load;
    bool (*fwd)(diffuse_context *, const int32_t *, int, float *) = &diffuse_forward;
    printf("%d\n", load != nullptr && fwd != nullptr);
    return 0;
}''')
    exe = tmp_path / "caller"
    lib = os.path.dirname(dfx.LIB_PATH)
    subprocess.check_call(["g++", "-std=c++17", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe),
                           "-L", lib, "-ldiffuse", f"-Wl,-rpath,{lib}", "-Wl,--allow-shlib-undefined"])
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "1"


# tools/ar-cli.cpp is the reference's caller of the autoregressive API (ar_generate,
# ar_speculative_generate); it includes <omp.h>, hence -fopenmp
REF_CALLERS = ("tools/main-cli.cpp", "tools/main-bench.cpp", "tools/dump-logits.cpp", "tests/test-forward.cpp",
               "tools/ar-cli.cpp")


@pytest.mark.skipif(not os.path.isdir("/root/reference/tools"), reason="reference sources not present on this host")
@pytest.mark.parametrize("rel", REF_CALLERS)
def test_reference_callers_link_unchanged(tmp_path, rel):
    """The reference's own callers of diffuse.h compile, unmodified, against this
    include/diffuse.h and link against libdiffuse (drop-in check; nothing is run)."""
    exe = tmp_path / os.path.basename(rel).replace(".cpp", "")
    lib = os.path.dirname(dfx.LIB_PATH)
    subprocess.check_call(["g++", "-std=c++17", "-O0", "-fopenmp", "-I", os.path.join(REPO, "include"),
                           os.path.join("/root/reference", rel), "-o", str(exe), "-L", lib, "-ldiffuse",
                           f"-Wl,-rpath,{lib}", "-Wl,--allow-shlib-undefined"])
    assert exe.exists()


@pytest.mark.parametrize("typ,bound", [(dfx.TYPE_Q4_K, 0.12), (dfx.TYPE_Q6_K, 0.03), (dfx.TYPE_Q8_0, 0.006),
                                       (dfx.TYPE_F16, 1e-3)])
def test_encoder_roundtrip(typ, bound):
    """The library's encoders decode (by the oracle's pinned codecs) back to the input within
    the format's resolution; bound = worst |error| / block max |x|."""
    x = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    raw = dfx.quantize_rows(typ, x)
    rb = O.row_bytes(typ, 1024)
    y = np.stack([O.dequant(typ, raw[r * rb:(r + 1) * rb], 1024) for r in range(64)])
    blk = 32 if typ == dfx.TYPE_Q8_0 else 256
    err = np.abs(y - x).reshape(64, -1, blk).max(-1)
    scale = np.abs(x).reshape(64, -1, blk).max(-1)
    assert np.max(err / scale) <= bound


def test_repack_layouts():
    rows, cols = 3, 512
    x = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float32)
    q6 = dfx.quantize_rows(dfx.TYPE_Q6_K, x)
    d6 = dfx.repack(dfx.TYPE_Q6_K, q6, rows, cols).reshape(-1, 224)
    assert np.array_equal(d6[:, :210], q6.reshape(-1, 210)) and not d6[:, 210:].any()
    q8 = dfx.quantize_rows(dfx.TYPE_Q8_0, x)
    d8 = dfx.repack(dfx.TYPE_Q8_0, q8, rows, cols).reshape(-1, 272)
    b8 = q8.reshape(-1, 8, 34)
    assert np.array_equal(d8[:, :16].reshape(-1, 8, 2), b8[:, :, :2])
    assert np.array_equal(d8[:, 16:].reshape(-1, 8, 32), b8[:, :, 2:])
    q4 = dfx.quantize_rows(dfx.TYPE_Q4_K, x)
    assert np.array_equal(dfx.repack(dfx.TYPE_Q4_K, q4, rows, cols), q4)
    f32 = dfx.repack(dfx.TYPE_F32, x.view(np.uint8), rows, cols)   # F32 matrices stay F32
    assert np.array_equal(f32.view(np.float32).reshape(rows, cols), x)
    with pytest.raises(dfx.DfxError):
        dfx.repack(dfx.TYPE_Q4_K, q4, rows, 100)


def test_synth_file_matches_converter_conventions(tmp_path):
    p = tmp_path / "m.gguf"
    dfx.synth_model(p, TINY_DREAM, scheme="q4_k_m", seed=3, sigma=0.02, n_threads=2)
    g = O.GGUF(str(p))
    kv = g.kv
    assert kv["general.architecture"] == "diffuse" and kv["diffuse.model_type"] == "dream"
    for k in ("block_count", "attention.head_count", "attention.head_count_kv", "embedding_length",
              "feed_forward_length", "context_length", "vocab_size", "rope.freq_base",
              "attention.layer_norm_rms_epsilon", "mask_token_id"):
        assert f"diffuse.{k}" in kv, k
    L = TINY_DREAM["n_layer"]
    assert len(g.tensors) == 3 + 12 * L          # 9 per layer + Q/K/V biases
    # Q4_K_M mixture (tools/quantize.cpp:31-110): attn Q4_K, FFN Q4_K except first/last
    # layer Q6_K, output Q6_K, embedding F16, norms and biases F32
    T = {n: t["type"] for n, t in g.tensors.items()}
    assert T["token_embd.weight"] == O.F16 and T["output.weight"] == O.Q6_K and T["output_norm.weight"] == O.F32
    assert T["blk.0.attn_q.bias"] == O.F32 and T["blk.1.attn_k.weight"] == O.Q4_K
    assert T["blk.0.ffn_up.weight"] == O.Q6_K and T[f"blk.{L - 1}.ffn_down.weight"] == O.Q6_K
    assert T["blk.1.ffn_gate.weight"] == O.Q4_K
    assert g.tensors["blk.0.attn_k.weight"]["ne"] == [512, 128]
    norm = O.dequant(O.F32, np.ascontiguousarray(g.tensors["blk.0.attn_norm.weight"]["data"]), 512)
    assert np.all(norm == 1.0)


def test_quantize_file_equals_direct_generation(tmp_path):
    """F16 file -> quantizer gives byte-identical tensors to generating the quantized
    file directly (values are f16-rounded before conversion in both)."""
    f16, direct, quant = tmp_path / "f16.gguf", tmp_path / "direct.gguf", tmp_path / "quant.gguf"
    dfx.synth_model(f16, TINY_LLADA, scheme="f16", seed=9, n_threads=2)
    dfx.synth_model(direct, TINY_LLADA, scheme="q4_k_m", seed=9, n_threads=2)
    dfx.quantize_file(f16, quant, "q4_k_m", n_threads=2)
    a, b = O.GGUF(str(direct)), O.GGUF(str(quant))
    assert set(a.tensors) == set(b.tensors)
    for n in a.tensors:
        assert a.tensors[n]["type"] == b.tensors[n]["type"], n
        assert np.array_equal(np.asarray(a.tensors[n]["data"]), np.asarray(b.tensors[n]["data"])), n


def test_synth_is_deterministic_and_seeded(tmp_path):
    a, b, c = tmp_path / "a.gguf", tmp_path / "b.gguf", tmp_path / "c.gguf"
    for p, s in ((a, 1), (b, 1), (c, 2)):
        dfx.synth_model(p, TINY_LLADA, scheme="q8_0", seed=s, n_threads=3)
    ta, tb, tc = (np.asarray(O.GGUF(str(p)).tensors["blk.1.attn_q.weight"]["data"]) for p in (a, b, c))
    assert np.array_equal(ta, tb) and not np.array_equal(ta, tc)
    w = O.dequant(O.F16, np.ascontiguousarray(O.GGUF(str(a)).tensors["token_embd.weight"]["data"]), 512 * 1536)
    assert abs(w.std() - 0.02) < 0.001 and abs(w.mean()) < 0.001


def test_model_load_errors_are_reported(tmp_path):
    with pytest.raises(dfx.DfxError, match="cannot open"):
        dfx.Model(tmp_path / "missing.gguf")
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + b"\x00" * 60)
    with pytest.raises(dfx.DfxError):
        dfx.Model(bad)


def test_oracle_forward_cached_equals_full_when_inputs_unchanged(tiny_models):
    """Attention is key-order invariant (the cached path's [cached | active] concat) and the
    cached rows reuse exactly the K/V a full forward would compute: a cached pass over any
    subset reproduces the full forward's rows."""
    om = O.OracleModel(tiny_models[("llada", "q4_k_m")])
    toks = np.random.default_rng(0).integers(0, 1400, 40).astype(np.int32)
    full, kv = om.forward_full(toks, kv_tokens=40)
    act = np.array([3, 7, 8, 20, 39], np.int32)
    part = om.forward_cached(kv, toks[act], act, 40)
    assert np.max(np.abs(part - full[act])) <= 1e-4 * np.max(np.abs(full))


def test_oracle_gqa_equals_mha_with_repeated_heads(tmp_path):
    """A GQA model equals the MHA model whose K/V projections repeat each KV head's rows
    for the n_rep query heads that read it (grouped mapping h -> h // n_rep)."""
    arch = dict(TINY_DREAM)
    p = tmp_path / "gqa.gguf"
    dfx.synth_model(p, arch, scheme="f16", seed=4, sigma=0.05, n_threads=2)
    g = O.GGUF(str(p))
    om = O.OracleModel(str(p))
    H, Hkv, hd, d = arch["n_head"], arch["n_head_kv"], 64, arch["n_embd"]
    rep = H // Hkv
    toks = np.arange(12, dtype=np.int32) * 5
    ref = om.forward_full(toks)
    keep = []
    for il in range(arch["n_layer"]):
        for f, name in (("wk", "attn_k.weight"), ("wv", "attn_v.weight")):
            w = np.asarray(g.tensors[f"blk.{il}.{name}"]["data"]).view(np.uint16).reshape(Hkv, hd, d)
            big = np.ascontiguousarray(np.repeat(w, rep, axis=0).reshape(H * hd, d))
            keep.append(big)
            setattr(om._layers[il], f, O.OrcTensor(O.F16, d, H * hd, big.ctypes.data))
        for f, name in (("bk", "attn_k.bias"), ("bv", "attn_v.bias")):
            t = g.tensors[f"blk.{il}.{name}"]
            b = O.dequant(t["type"], np.ascontiguousarray(t["data"]), Hkv * hd).reshape(Hkv, hd)
            big = np.ascontiguousarray(np.repeat(b, rep, axis=0).reshape(-1))
            keep.append(big)
            setattr(om._layers[il], f, O.OrcTensor(O.F32, H * hd, 1, big.ctypes.data))
    om.m.n_head_kv = H
    mha = om.forward_full(toks)
    assert np.array_equal(mha, ref)
