import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "diffuse-cpp_amd")
for p in (PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


# Small architectures whose K dimensions are multiples of 256 (K-quant blocks),
# head_dim 128 / 64, so every code path of the 8B models runs at test size.
TINY_LLADA = dict(n_vocab=1536, n_embd=512, n_head=4, n_head_kv=4, n_layer=3, n_ff=1024,
                  rope_theta=500000.0, rms_norm_eps=1e-5, mask_token_id=1500, is_dream=0)
TINY_DREAM = dict(n_vocab=1280, n_embd=512, n_head=8, n_head_kv=2, n_layer=3, n_ff=768,
                  rope_theta=1000000.0, rms_norm_eps=1e-6, mask_token_id=1270, is_dream=1)
# K spans several 2048-element chunks (O: 2304 = 2048 + 256, down: 4608 = 3 chunks), so the
# O / down GEMMs split K and hand their chunk sums to the next RMSNorm.
# six layers, so that layers 2 and 3 can be skipped by the autoregressive layer skip (the
# first and last two are protected)
TINY_LLADA6 = dict(TINY_LLADA, n_layer=6)
# vocabulary reaching the end tokens of the autoregressive sampler (151643 / 151645 / 151644)
EOS_ARCH = dict(n_vocab=151680, n_embd=256, n_head=2, n_head_kv=2, n_layer=2, n_ff=512,
                rope_theta=1000000.0, rms_norm_eps=1e-6, mask_token_id=151666, is_dream=0)


def eos_model(path):
    """A model whose head scores only two end tokens: output rows 151643 = +u, 151645 = -u
    (u random), every other row zero, so greedy decoding ends at the first token."""
    import dfx
    import oracle_py as O
    dfx.synth_model(path, EOS_ARCH, scheme="f32", seed=5, sigma=0.05, n_threads=4)
    ti = O.GGUF(path).tensor("output.weight")
    assert ti["type"] == O.F32
    off = ti["start"]
    mm = np.memmap(path, dtype=np.uint8, mode="r+")
    w = mm[off:off + EOS_ARCH["n_vocab"] * EOS_ARCH["n_embd"] * 4].view(np.float32).reshape(EOS_ARCH["n_vocab"], -1)
    u = np.random.default_rng(6).standard_normal(EOS_ARCH["n_embd"]).astype(np.float32)
    w[:] = 0.0
    w[151643] = u
    w[151645] = -u
    mm.flush()
    del mm
    return str(path)


TINY_LLADA_LONGK = dict(n_vocab=1024, n_embd=2304, n_head=18, n_head_kv=18, n_layer=2, n_ff=4608,
                        rope_theta=500000.0, rms_norm_eps=1e-5, mask_token_id=1000, is_dream=0)


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


@pytest.fixture(scope="session")
def tiny_models(model_dir):
    """GGUF files: {(arch, scheme): path}, written by the library's generator.
    sigma 0.05 keeps the random-init logits from being near-uniform."""
    import dfx
    out = {}
    for arch_name, arch, seed in (("llada", TINY_LLADA, 11), ("dream", TINY_DREAM, 12)):
        for scheme in ("q4_k_m", "q8_0", "f16"):
            p = model_dir / f"{arch_name}-{scheme}.gguf"
            dfx.synth_model(p, arch, scheme=scheme, seed=seed, sigma=0.05, n_threads=4)
            out[(arch_name, scheme)] = str(p)
    return out


def forward_inputs(V):
    """The token sequences of the forward parity tests: n = 1, 17, 64, seed 3."""
    rng = np.random.default_rng(3)
    return [rng.integers(0, V, n).astype(np.int32) for n in (1, 17, 64)]


@pytest.fixture(scope="session")
def longk_models(model_dir):
    """GGUF files of TINY_LLADA_LONGK: {("llada_longk", scheme): path}."""
    import dfx
    out = {}
    for scheme in ("q4_k_m", "f16"):
        p = model_dir / f"llada_longk-{scheme}.gguf"
        dfx.synth_model(p, TINY_LLADA_LONGK, scheme=scheme, seed=13, sigma=0.05, n_threads=8)
        out[("llada_longk", scheme)] = str(p)
    return out


@pytest.fixture(scope="session")
def gpu():
    import dfx
    n = dfx.device_count()
    if n < 1:
        raise RuntimeError("no HIP device visible: the gpu tests need an MI355X")
    return n


def big_model(tag, arch, scheme, seed, sigma=0.02):
    """GGUF of a benchmark-size architecture (random-init N(0, sigma), norms 1.0), written
    once per machine under DFX_BENCH_DIR (default /tmp) with the benchmark's file naming,
    so the benchmark and these tests share one generated file."""
    import dfx
    d = os.environ.get("DFX_BENCH_DIR", "/tmp")
    p = os.path.join(d, f"dfx-{tag}-{scheme}-s{seed}.gguf")
    stamp = p + ".ok"
    if not (os.path.exists(p) and os.path.exists(stamp)):
        dfx.synth_model(p, arch, scheme=scheme, seed=seed, sigma=sigma, n_threads=16)
        with open(stamp, "w") as f:
            f.write("ok\n")
    return p


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
