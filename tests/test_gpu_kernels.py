"""Kernel-level parity of the HIP path (through the C ABI) against the CPU oracle."""
import contextlib
import ctypes as C

import numpy as np
import pytest

import dfx
import oracle_py as O
from conftest import rel_l2

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(7)
L = dfx.lib


def quant(typ, rows, cols, scale=0.02):
    x = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(scale)
    return dfx.quantize_rows(typ, x)


def to_device_weights(typ, raw, rows, cols):
    return dfx.Buf.of(dfx.repack(typ, raw, rows, cols))


def oracle_dequant_rows(typ, raw, rows, cols):
    rb = O.row_bytes(typ, cols)
    return np.stack([O.dequant(typ, raw[r * rb:(r + 1) * rb], cols) for r in range(rows)])


# ---------------------------------------------------------------- dequant: bit-exact
@pytest.mark.parametrize("typ,rows,cols", [(dfx.TYPE_Q4_K, 4096, 4096), (dfx.TYPE_Q4_K, 12288, 4096),
                                           (dfx.TYPE_Q6_K, 4096, 4096), (dfx.TYPE_Q8_0, 4096, 4096),
                                           (dfx.TYPE_F16, 512, 4096)])
def test_dequant_bit_exact(gpu, typ, rows, cols):
    raw = quant(typ, rows, cols)
    w = to_device_weights(typ, raw, rows, cols)
    out = dfx.Buf(rows * cols * 4)
    dfx.check(L().dfx_dequant(typ, w.ptr, rows, cols, out.ptr, None), "dequant")
    got = out.download(np.float32, shape=(rows, cols))
    rb = O.row_bytes(typ, cols)
    ref = np.empty_like(got)
    for r in range(rows):
        ref[r] = O.dequant(typ, raw[r * rb:(r + 1) * rb], cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("typ,size", [(dfx.TYPE_Q4_K, 144), (dfx.TYPE_Q6_K, 210)])
def test_dequant_random_blocks_bit_exact(gpu, typ, size):
    rows, cols = 64, 1024
    raw = rng.integers(0, 256, rows * cols // 256 * size, dtype=np.uint8).reshape(-1, size)
    for p in ((0, 2) if typ == dfx.TYPE_Q4_K else (208,)):
        raw[:, p + 1] &= 0x7B          # finite f16 scales
    raw = raw.reshape(-1)
    w = to_device_weights(typ, raw, rows, cols)
    out = dfx.Buf(rows * cols * 4)
    dfx.check(L().dfx_dequant(typ, w.ptr, rows, cols, out.ptr, None), "dequant")
    got = out.download(np.float32, shape=(rows, cols))
    assert np.array_equal(got.view(np.uint32), oracle_dequant_rows(typ, raw, rows, cols).view(np.uint32))


# ---------------------------------------------------------------- activation conversion
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bs", "<i2", 16)])
Q80 = np.dtype([("d", "<f2"), ("qs", "i1", 32)])


def oracle_act(wtype, X):
    """(q, d, bs) of GGML's conversion of X for weight type wtype, from the oracle."""
    M, K = X.shape
    if wtype in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K):
        b = np.stack([np.frombuffer(O.quantize_q8_K(X[m]).tobytes(), Q8K) for m in range(M)])
        return (b["qs"].reshape(M, K).astype(np.float16), b["d"].astype(np.float32),
                b["bs"].reshape(M, -1).astype(np.float16))
    if wtype == dfx.TYPE_Q8_0:
        b = np.stack([np.frombuffer(O.quantize_q8_0(X[m]).tobytes(), Q80) for m in range(M)])
        return b["qs"].reshape(M, K).astype(np.float16), b["d"].astype(np.float32), None
    return X.astype(np.float16), None, None


def same_bits(a, b):
    return a is None and b is None or np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


def check_act(act, wtype, ref, M, K):
    q, d, bs = dfx.act_parts(act, wtype, M, K)
    rq, rd, rbs = ref
    assert np.array_equal(q.astype(np.float32), rq.astype(np.float32)) and same_bits(d, rd) and same_bits(bs, rbs)


@pytest.mark.parametrize("typ", [dfx.TYPE_Q4_K, dfx.TYPE_Q8_0, dfx.TYPE_F16])
def test_act_convert_matches_oracle(gpu, typ):
    M, K = 37, 4096
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-2, 2, (M, 1))).astype(np.float32)
    x[3, 256:512] = 0.0
    x[5, :256] = 1.0        # ties on |max|: first index wins
    x[5, 100] = -1.0
    xb, ab = dfx.Buf.of(x), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "act_convert")
    check_act(ab, typ, oracle_act(typ, x), M, K)


@pytest.mark.parametrize("K", [4096, 1280, 5120, 9472])   # 1, 1, 2 and 4 blocks per wave
def test_rmsnorm_convert_matches_oracle(gpu, K):
    M, eps = 29, 1e-5
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    for typ in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K, dfx.TYPE_Q8_0, dfx.TYPE_F16):
        xb, wb, ab = dfx.Buf.of(x), dfx.Buf.of(w), dfx.Buf(L().dfx_act_bytes(typ, M, K))
        dfx.check(L().dfx_rmsnorm_convert(typ, xb.ptr, wb.ptr, M, K, eps, ab.ptr, None), "rmsnorm")
        check_act(ab, typ, oracle_act(typ, O.rms_norm_mul(x, w, eps)), M, K)


def test_swiglu_convert_matches_oracle(gpu):
    M, F = 19, 2048
    gu = rng.standard_normal((M, 2 * F)).astype(np.float32) * 2
    s = np.array([[O.oracle().orc_silu(float(v)) for v in r] for r in gu[:, :F]], np.float32) * gu[:, F:]
    for typ in (dfx.TYPE_Q4_K, dfx.TYPE_Q8_0, dfx.TYPE_F16):
        gb, ab = dfx.Buf.of(gu), dfx.Buf(L().dfx_act_bytes(typ, M, F))
        dfx.check(L().dfx_swiglu_convert(typ, gb.ptr, M, F, ab.ptr, None), "swiglu")
        check_act(ab, typ, oracle_act(typ, s), M, F)


# ---------------------------------------------------------------- GEMM
GEMM_CASES = [(dfx.TYPE_Q4_K, 4096, 4096, m) for m in (1, 5, 50, 96, 128, 255, 288)] + [
    (dfx.TYPE_Q4_K, 12288, 4096, 288), (dfx.TYPE_Q6_K, 4096, 4096, 64), (dfx.TYPE_Q6_K, 2048, 12288, 100),
    (dfx.TYPE_Q6_K, 1000, 4096, 288), (dfx.TYPE_Q8_0, 4096, 4096, 77), (dfx.TYPE_Q4_K, 4096, 12288, 288),
    # Q6_K 96-row DMA tiles: split K over 74 rows, whole K over 162
    (dfx.TYPE_Q6_K, 2048, 12288, 74), (dfx.TYPE_Q6_K, 3000, 4096, 162),
    (dfx.TYPE_Q8_0, 1024, 4096, 300),
    # batched long-context workload: one 512 + 256 sequence's step-0 rows on Q8_0 weights
    (dfx.TYPE_Q8_0, 4096, 4096, 768), (dfx.TYPE_Q8_0, 4096, 12288, 768),
    # Q8_0 grids wide enough for 64-row tiles (Q|K|V at 768 rows; gate|up over a ragged 300)
    (dfx.TYPE_Q8_0, 12288, 4096, 768), (dfx.TYPE_Q8_0, 24576, 4096, 300),
    # LLaDA-8B fused gate|up and vocab head at the benchmark's step 0
    (dfx.TYPE_Q4_K, 24576, 4096, 288), (dfx.TYPE_Q6_K, 126464, 4096, 288),
    # Dream-7B: fused Q|K|V, gate|up, down, vocab head (steps of 128 and 64 rows)
    (dfx.TYPE_Q4_K, 4608, 3584, 128), (dfx.TYPE_Q4_K, 37888, 3584, 64), (dfx.TYPE_Q4_K, 3584, 18944, 128),
    (dfx.TYPE_Q6_K, 152064, 3584, 64),
    # narrow GEMMs over few rows: one-wave (down at 24 rows) and two-wave workgroups (down at
    # 48 rows, O at 40, Q|K|V at 20)
    (dfx.TYPE_Q4_K, 3584, 18944, 24), (dfx.TYPE_Q4_K, 3584, 18944, 48), (dfx.TYPE_Q4_K, 3584, 3584, 40),
    (dfx.TYPE_Q4_K, 4608, 3584, 20),
    # wide GEMMs over few rows: two-wave register tiles with split K (24 rows), 64-row DMA tiles with
    # split K on a mid-width grid (40 rows)
    (dfx.TYPE_Q4_K, 37888, 3584, 24), (dfx.TYPE_Q4_K, 12288, 4096, 40)]


@contextlib.contextmanager
def forced_tile(wtype, spec):
    dfx.force_tile(wtype, spec)
    try:
        yield
    finally:
        dfx.force_tile(wtype, None)


def gpu_gemm(typ, raw, N, K, X, ws=True):
    M = X.shape[0]
    w = to_device_weights(typ, raw, N, K)
    xb, ab, yb = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K)), dfx.Buf(M * N * 4)
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    wsb = dfx.Buf(L().dfx_gemm_ws_bytes(M, N, K)) if ws else None
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, None, yb.ptr, wsb.ptr if ws else None, None), "gemm")
    return yb.download(np.float32, shape=(M, N))


@pytest.mark.parametrize("typ,N,K,M", GEMM_CASES)
def test_gemm_quantized_bit_exact(gpu, typ, N, K, M):
    """Q4_K / Q6_K / Q8_0: the GPU reproduces the oracle's GGML block dot products
    (integer sums, float scaling and accumulation in K order) bit for bit."""
    raw = quant(typ, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    got = gpu_gemm(typ, raw, N, K, X)
    ref = O.mul_mat(typ, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rel_l2(got, ref)


@pytest.mark.parametrize("tile", ["2x2x2", "4x1x2", "2x1x2", "1x1x4", "1x1x2", "2x1x4", "2x2x4", "w", "w1", "w3",
                                  "1x1x4v1", "1x1x2v1", "1x1x4v2", "1x1x2v2", "k", "ks", "k2", "k4"])
@pytest.mark.parametrize("N,K,M", [(1000, 2048, 77), (4096, 4096, 288)])
def test_gemm_q4k_every_tile_bit_exact(gpu, tile, N, K, M):
    """Every register tile of the Q4_K kernel (forced with dfx_gemm_force_tile), with ragged
    N and M, reproduces the oracle bit for bit."""
    raw = quant(dfx.TYPE_Q4_K, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    with forced_tile(dfx.TYPE_Q4_K, tile):
        got = gpu_gemm(dfx.TYPE_Q4_K, raw, N, K, X)
    ref = O.mul_mat(dfx.TYPE_Q4_K, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rel_l2(got, ref)


@pytest.mark.parametrize("tile", ["1x1x4s", "2x1x2s", "2x1x4s", "ws", "w1s", "w3s", "1x1x4v1s", "1x1x2v2s", "ks", "k4s"])
@pytest.mark.parametrize("N,K,M", [(512, 12288, 70), (1000, 3584, 33), (640, 2304, 40), (4096, 4096, 256)])
def test_gemm_q4k_split_k_bit_exact(gpu, tile, N, K, M):
    """Split K (one workgroup per 2048-element chunk, chunk sums added in order by the
    reduction) gives the same bits as the oracle's chunked K order; covers a short last
    chunk (3584 = 2048 + 1536) and a last chunk of one super-block (2304)."""
    raw = quant(dfx.TYPE_Q4_K, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    with forced_tile(dfx.TYPE_Q4_K, tile):
        got = gpu_gemm(dfx.TYPE_Q4_K, raw, N, K, X)
    ref = O.mul_mat(dfx.TYPE_Q4_K, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rel_l2(got, ref)


@pytest.mark.parametrize("tile", ["2x1n", "1x1n", "2x1s", "1x1s", "2x1x4n", "2x1x4s", "1x1x4s", "wn", "ws", "w3n", "w3s"])
@pytest.mark.parametrize("N,K,M", [(1000, 4096, 77), (640, 12288, 40), (300, 2304, 33)])
def test_gemm_q6k_tiles_and_split_bit_exact(gpu, tile, N, K, M):
    """Q6_K kernel tiles (register ring, and "w" the LDS-DMA kernel), with and without split K
    (scales up to +-127 exercise the exact f16 operand split), against the oracle bit for bit."""
    raw = quant(dfx.TYPE_Q6_K, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    with forced_tile(dfx.TYPE_Q6_K, tile):
        got = gpu_gemm(dfx.TYPE_Q6_K, raw, N, K, X)
    ref = O.mul_mat(dfx.TYPE_Q6_K, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rel_l2(got, ref)


@pytest.mark.parametrize("N,K,M", [(1000, 4096, 33), (4096, 4096, 288), (4096, 12288, 64), (4096, 4096, 768)])
def test_gemm_f16_matches_oracle(gpu, N, K, M):
    """F16: exact f16 products accumulated by MFMA in f32 (the oracle sums in f64)."""
    raw = quant(dfx.TYPE_F16, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    got = gpu_gemm(dfx.TYPE_F16, raw, N, K, X)
    ref = O.mul_mat(dfx.TYPE_F16, raw, N, K, X)
    assert rel_l2(got, ref) < 1e-6
    assert rel_l2(gpu_gemm(dfx.TYPE_F16, raw, N, K, X, ws=False), got) < 1e-6


def test_gemm_bias_and_residual_epilogue(gpu):
    typ, N, K, M = dfx.TYPE_Q4_K, 1024, 2048, 40
    raw = quant(typ, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    w = to_device_weights(typ, raw, N, K)
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    plain = dfx.Buf(M * N * 4)
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, None, plain.ptr, None, None), "gemm")
    p = plain.download(np.float32, shape=(M, N))
    bb, yb = dfx.Buf.of(bias), dfx.Buf(M * N * 4)
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, bb.ptr, None, yb.ptr, None, None), "gemm+bias")
    assert np.array_equal(yb.download(np.float32, shape=(M, N)), p + bias)
    rb = dfx.Buf.of(res)        # in-place residual: y = y + A W
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, rb.ptr, rb.ptr, None, None), "gemm+res")
    assert np.array_equal(rb.download(np.float32, shape=(M, N)), p + res)


GEMV_CASES = [(t, N, K, M) for t in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K)
              for (N, K) in ((64, 2304), (4608, 3584), (96, 8192), (4096, 12288), (1024, 18944)) for M in (1, 2, 3, 4)]
GEMV_CASES += [(dfx.TYPE_Q6_K, 152064, 3584, 1), (dfx.TYPE_Q4_K, 37888, 3584, 1)]


@pytest.mark.parametrize("typ,N,K,M", GEMV_CASES)
def test_gemv_bit_exact(gpu, typ, N, K, M):
    """At most four rows the matrix-vector kernels run (integer dot products on the int8
    plane, the exact float order over super-blocks and chunks, a short last chunk at
    K = 2304 / 3584 / 18944; one, two and four waves per column pair at 1, 2 and 3-5
    passes of 4096 elements): the oracle's
    values bit for bit, and the same bits as the
    matrix-core kernel forced by a tile override."""
    raw = quant(typ, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    got = gpu_gemm(typ, raw, N, K, X)
    ref = O.mul_mat(typ, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rel_l2(got, ref)
    with forced_tile(typ, "1x1x2"):
        mfma = gpu_gemm(typ, raw, N, K, X)
    assert np.array_equal(got.view(np.uint32), mfma.view(np.uint32))


def test_gemv_epilogues_and_row_map(gpu):
    """Bias, in-place residual and a row map through the matrix-vector kernel."""
    typ, N, K, M = dfx.TYPE_Q4_K, 1024, 4096, 3
    raw = quant(typ, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    w = to_device_weights(typ, raw, N, K)
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    ref = O.mul_mat(typ, raw, N, K, X)
    bias = rng.standard_normal(N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    bb, rb = dfx.Buf.of(bias), dfx.Buf.of(res)
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, bb.ptr, rb.ptr, rb.ptr, None, None), "gemm")
    assert np.array_equal(rb.download(np.float32, shape=(M, N)), (ref + bias) + res)


def test_act_convert_int8_plane(gpu):
    """At most four rows the Q4_K/Q6_K activation buffer also holds the int8 quants in
    natural order, equal to the f16 ones."""
    K = 4096
    for typ in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K):
        for M in (1, 4):
            x = rng.standard_normal((M, K)).astype(np.float32)
            xb, ab = dfx.Buf.of(x), dfx.Buf(L().dfx_act_bytes(typ, M, K))
            dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
            q, _, _ = dfx.act_parts(ab, typ, M, K)
            raw = ab.download(np.uint8)
            i8 = raw[len(raw) - (M * K + 255) // 256 * 256:][:M * K].view(np.int8).reshape(M, K)
            assert np.array_equal(i8.astype(np.float32), q.astype(np.float32))


def interleave16(typ, gate, up, F, K):
    """gate|up GGML rows interleaved in blocks of 16 (the fused SwiGLU GEMM's weight order)."""
    rb = O.row_bytes(typ, K)
    g = np.frombuffer(gate, np.uint8).reshape(F // 16, 1, 16 * rb)
    u = np.frombuffer(up, np.uint8).reshape(F // 16, 1, 16 * rb)
    return np.concatenate([g, u], axis=1).reshape(-1)


def oracle_swiglu(g, u):
    silu = np.vectorize(lambda v: O.oracle().orc_silu(float(v)), otypes=[np.float32])
    return silu(g) * u


@pytest.mark.parametrize("typ,F,K,M,tile", [
    (dfx.TYPE_Q4_K, 512, 4096, 77, None), (dfx.TYPE_Q4_K, 512, 4096, 77, "2x1x2s"),
    (dfx.TYPE_Q4_K, 1024, 4096, 130, "w"), (dfx.TYPE_Q4_K, 1024, 4096, 130, "ws"),
    (dfx.TYPE_Q4_K, 1024, 3584, 150, "w3"), (dfx.TYPE_Q4_K, 512, 12288, 5, "1x1x4s"),
    (dfx.TYPE_Q4_K, 2048, 4096, 1, None), (dfx.TYPE_Q4_K, 1024, 4096, 4, None), (dfx.TYPE_Q6_K, 512, 4096, 2, None),
    (dfx.TYPE_Q4_K, 2688, 3584, 24, None),   # wide, few rows: two-wave tiles, split K, SwiGLU in the reduction
    (dfx.TYPE_Q6_K, 512, 12288, 40, "2x1s"), (dfx.TYPE_Q4_K, 512, 12288, 40, "ks"), (dfx.TYPE_Q4_K, 512, 3584, 70, "k"), (dfx.TYPE_Q4_K, 768, 4096, 50, "k4"),
    (dfx.TYPE_Q6_K, 512, 4096, 66, "2x1n"), (dfx.TYPE_Q8_0, 512, 4096, 33, None),
    (dfx.TYPE_F16, 512, 4096, 33, None), (dfx.TYPE_F32, 256, 512, 20, None)])
def test_gemm_swiglu_epilogue_bit_exact(gpu, typ, F, K, M, tile):
    """dfx_gemm_swiglu on an interleaved gate|up matrix: the same bits as the plain GEMM's
    gate and up values put through GGML's silu(gate) * up, for every tile and with split K
    (the reduction applies the epilogue); for the integer-dot types also the oracle's
    mul_mat values.  Padding columns of a wider output row stay untouched."""
    gate, up = quant(typ, F, K), quant(typ, F, K)
    W = interleave16(typ, gate, up, F, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    wd = to_device_weights(typ, W, 2 * F, K)
    ldy = F + 32
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    yb = dfx.Buf.of(np.full((M, ldy), 7.0, np.float32))
    wsb = dfx.Buf(L().dfx_gemm_ws_bytes(M, 2 * F, K))
    with forced_tile(typ, tile) if tile else contextlib.nullcontext():
        dfx.check(L().dfx_gemm_swiglu(typ, wd.ptr, 2 * F, K, ab.ptr, M, yb.ptr, ldy, wsb.ptr, None), "swiglu")
        plain = gpu_gemm(typ, W, 2 * F, K, X)
    y = yb.download(np.float32, shape=(M, ldy))
    assert np.all(y[:, F:] == 7.0)
    pg = plain.reshape(M, F // 16, 2, 16)
    ref = oracle_swiglu(pg[:, :, 0, :].reshape(M, F), pg[:, :, 1, :].reshape(M, F))
    assert np.array_equal(y[:, :F].view(np.uint32), ref.view(np.uint32)), rel_l2(y[:, :F], ref)
    if typ in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K, dfx.TYPE_Q8_0):
        og = O.mul_mat(typ, gate, F, K, X)
        ou = O.mul_mat(typ, up, F, K, X)
        oref = oracle_swiglu(og, ou)
        assert np.array_equal(y[:, :F].view(np.uint32), oref.view(np.uint32)), rel_l2(y[:, :F], oref)


def test_gemm_swiglu_rejects_bad_shapes(gpu):
    typ, F, K, M = dfx.TYPE_Q4_K, 256, 256, 4
    wd = to_device_weights(typ, quant(typ, 2 * F, K), 2 * F, K)
    ab, yb = dfx.Buf(L().dfx_act_bytes(typ, M, K)), dfx.Buf(M * F * 4)
    assert L().dfx_gemm_swiglu(typ, wd.ptr, 2 * F - 16, K, ab.ptr, M, yb.ptr, F, None, None) != 0
    assert L().dfx_gemm_swiglu(typ, wd.ptr, 2 * F, K, ab.ptr, M, yb.ptr, F - 1, None, None) != 0


def rope_row_order(H, Hkv, hd):
    """Device row order of the fused RoPE GEMM: in each Q and K head, blocks of 32 rows hold
    dims 16j..16j+15 and then hd/2 + 16j..; V rows stay in order."""
    src = []
    for r in range((H + 2 * Hkv) * hd):
        if r >= (H + Hkv) * hd:
            src.append(r)
            continue
        head, i = divmod(r, hd)
        j, c = divmod(i, 32)
        src.append(head * hd + (16 * j + c if c < 16 else hd // 2 + 16 * j + c - 16))
    return np.array(src)


@pytest.mark.parametrize("typ,H,Hkv,hd,K,M,tile,bias", [
    (dfx.TYPE_Q4_K, 8, 2, 128, 2048, 77, None, False), (dfx.TYPE_Q4_K, 8, 8, 128, 4096, 130, "w", True),
    (dfx.TYPE_Q4_K, 4, 4, 128, 4096, 150, "w3", False), (dfx.TYPE_Q4_K, 6, 2, 64, 4096, 40, "2x1x2s", True),
    (dfx.TYPE_Q4_K, 4, 2, 128, 4096, 200, "ws", False), (dfx.TYPE_Q4_K, 8, 8, 128, 4096, 3, None, False),
    (dfx.TYPE_Q4_K, 4, 2, 128, 3584, 1, None, True), (dfx.TYPE_Q6_K, 4, 4, 64, 4096, 2, None, False),
    (dfx.TYPE_Q4_K, 4, 2, 128, 3584, 50, "ks", True), (dfx.TYPE_Q4_K, 6, 2, 64, 4096, 40, "k", True), (dfx.TYPE_Q4_K, 4, 2, 128, 4096, 74, "k2s", True),
    (dfx.TYPE_Q6_K, 4, 2, 128, 4096, 66, "2x1s", True), (dfx.TYPE_Q6_K, 4, 4, 64, 2048, 100, "2x1n", False),
    (dfx.TYPE_Q8_0, 4, 2, 128, 2048, 33, None, True), (dfx.TYPE_F16, 4, 1, 128, 2048, 45, None, True),
    (dfx.TYPE_F32, 2, 1, 64, 512, 20, None, False)])
def test_gemm_rope_epilogue_bit_exact(gpu, typ, H, Hkv, hd, K, M, tile, bias):
    """dfx_gemm_rope on the row-permuted Q|K|V matrix stores the same q, K-cache and
    transposed V-cache bits as dfx_gemm (+bias) on the unpermuted matrix followed by
    dfx_rope_store, for every tile, with split K (the reduction applies the epilogue), and
    when Q and K|V are two calls (col0); cache positions outside pos stay untouched."""
    N = (H + 2 * Hkv) * hd
    n_ctx = M + 37
    raw = quant(typ, N, K)
    rb = O.row_bytes(typ, K)
    order = rope_row_order(H, Hkv, hd)
    perm = np.frombuffer(raw, np.uint8).reshape(N, rb)[order].reshape(-1)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    X = rng.standard_normal((M, K)).astype(np.float32)
    pos = rng.permutation(n_ctx)[:M].astype(np.int32)
    tab = O.rope_table(n_ctx, hd, 500000.0)
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    pb, tb = dfx.Buf.of(pos), dfx.Buf.of(tab)
    ws = dfx.Buf(L().dfx_gemm_ws_bytes(M, N, K))

    def outputs():
        q, k, v = dfx.Buf(M * H * hd * 4), dfx.Buf(n_ctx * Hkv * hd * 4), dfx.Buf(n_ctx * Hkv * hd * 4)
        k.upload(np.full(n_ctx * Hkv * hd, 5.0, np.float32))
        v.upload(np.full(n_ctx * Hkv * hd, 5.0, np.float32))
        return q, k, v

    def fetch(q, k, v):
        return (q.download(np.float32, shape=(M, H, hd)), k.download(np.float32, shape=(n_ctx, Hkv, hd)),
                v.download(np.float32, shape=(Hkv, hd, n_ctx)))

    with forced_tile(typ, tile) if tile else contextlib.nullcontext():
        # reference: plain GEMM (+bias) on the unpermuted rows, then the RoPE kernel
        wd = to_device_weights(typ, raw, N, K)
        yb = dfx.Buf(M * N * 4)
        bb = dfx.Buf.of(b) if bias else None
        dfx.check(L().dfx_gemm(typ, wd.ptr, N, K, ab.ptr, M, bb.ptr if bias else None, None, yb.ptr, ws.ptr, None),
                  "gemm")
        r = outputs()
        dfx.check(L().dfx_rope_store(yb.ptr, pb.ptr, M, H, Hkv, hd, tb.ptr, r[0].ptr, r[1].ptr, r[2].ptr, n_ctx,
                                     None), "rope")
        ref = fetch(*r)
        # fused, one call
        wp = to_device_weights(typ, perm, N, K)
        pbias = dfx.Buf.of(b[order]) if bias else None
        g = outputs()
        dfx.check(L().dfx_gemm_rope(typ, wp.ptr, N, K, ab.ptr, M, pbias.ptr if bias else None, 0, pb.ptr, H, Hkv, hd,
                                    tb.ptr, g[0].ptr, g[1].ptr, g[2].ptr, n_ctx, ws.ptr, None), "gemm_rope")
        got = fetch(*g)
        # fused, Q and K|V as two calls over row slices of the same matrix
        nq = H * hd
        wq = to_device_weights(typ, perm[:nq * rb], nq, K)
        wkv = to_device_weights(typ, perm[nq * rb:], N - nq, K)
        bq = dfx.Buf.of(b[order][:nq]) if bias else None
        bkv = dfx.Buf.of(b[order][nq:]) if bias else None
        h = outputs()
        dfx.check(L().dfx_gemm_rope(typ, wq.ptr, nq, K, ab.ptr, M, bq.ptr if bias else None, 0, pb.ptr, H, Hkv, hd,
                                    tb.ptr, h[0].ptr, h[1].ptr, h[2].ptr, n_ctx, ws.ptr, None), "gemm_rope q")
        dfx.check(L().dfx_gemm_rope(typ, wkv.ptr, N - nq, K, ab.ptr, M, bkv.ptr if bias else None, nq, pb.ptr, H,
                                    Hkv, hd, tb.ptr, h[0].ptr, h[1].ptr, h[2].ptr, n_ctx, ws.ptr, None), "gemm_rope kv")
        two = fetch(*h)
    for a, e in ((got, ref), (two, ref)):
        for x, y in zip(a, e):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    untouched = np.setdiff1d(np.arange(n_ctx), pos)
    assert np.all(got[1][untouched] == 5.0) and np.all(got[2][:, :, untouched] == 5.0)


def test_gemm_rope_rejects_bad_arguments(gpu):
    typ, H, Hkv, hd, K, M = dfx.TYPE_Q4_K, 2, 1, 128, 256, 4
    N = (H + 2 * Hkv) * hd
    wd = to_device_weights(typ, quant(typ, N, K), N, K)
    ab, pb, tb = dfx.Buf(L().dfx_act_bytes(typ, M, K)), dfx.Buf(M * 4), dfx.Buf(64 * hd * 4)
    q, k, v = dfx.Buf(M * H * hd * 4), dfx.Buf(64 * Hkv * hd * 4), dfx.Buf(64 * Hkv * hd * 4)
    ok = (typ, wd.ptr, N, K, ab.ptr, M, None, 0, pb.ptr, H, Hkv, hd, tb.ptr, q.ptr, k.ptr, v.ptr, 64, None, None)
    for i, bad in ((7, 16), (7, 32), (11, 48), (10, 3), (15, None), (2, N - 16)):
        args = list(ok)
        args[i] = bad
        assert L().dfx_gemm_rope(*args) != 0, (i, bad)


# ---------------------------------------------------------------- RoPE + attention
@pytest.mark.parametrize("M,H,Hkv,hd,n_ctx", [(23, 8, 2, 128, 64), (77, 4, 4, 64, 96), (65, 28, 4, 128, 300)])
def test_rope_store_matches_oracle(gpu, M, H, Hkv, hd, n_ctx):
    qkv = rng.standard_normal((M, (H + 2 * Hkv) * hd)).astype(np.float32)
    pos = rng.permutation(n_ctx)[:M].astype(np.int32)
    tab = O.rope_table(n_ctx, hd, 1000000.0)
    qb, pb, tb = dfx.Buf.of(qkv), dfx.Buf.of(pos), dfx.Buf.of(tab)
    qo, kc, vc = dfx.Buf(M * H * hd * 4), dfx.Buf(n_ctx * Hkv * hd * 4), dfx.Buf(n_ctx * Hkv * hd * 4)
    kc.zero()
    vc.zero()
    dfx.check(L().dfx_rope_store(qb.ptr, pb.ptr, M, H, Hkv, hd, tb.ptr, qo.ptr, kc.ptr, vc.ptr, n_ctx, None),
              "rope")
    q_ref = qkv[:, :H * hd].reshape(M, H, hd).copy()
    k_ref = qkv[:, H * hd:(H + Hkv) * hd].reshape(M, Hkv, hd).copy()
    O.oracle().orc_rope_neox(O.ptr(q_ref), M, H, hd, O.ptr(pos), O.ptr(tab))
    O.oracle().orc_rope_neox(O.ptr(k_ref), M, Hkv, hd, O.ptr(pos), O.ptr(tab))
    assert np.array_equal(qo.download(np.float32, shape=(M, H, hd)), q_ref)
    kg = kc.download(np.float32, shape=(n_ctx, Hkv, hd))
    vg = vc.download(np.float32, shape=(Hkv, hd, n_ctx)).transpose(2, 0, 1)     # stored [Hkv][hd][n_ctx]
    assert np.array_equal(kg[pos], k_ref)
    assert np.array_equal(vg[pos], qkv[:, (H + Hkv) * hd:].reshape(M, Hkv, hd))
    untouched = np.setdiff1d(np.arange(n_ctx), pos)
    assert not kg[untouched].any() and not vg[untouched].any()


ATTN_SHAPES = [(288, 288, 32, 32, 128), (50, 288, 32, 32, 128), (128, 128, 28, 4, 128), (7, 768, 8, 2, 64),
               (3, 2000, 4, 4, 128), (2, 3000, 2, 1, 128), (17, 1, 4, 4, 128), (33, 21, 4, 2, 64),
               (768, 768, 32, 32, 128), (256, 768, 32, 32, 128), (65, 97, 6, 3, 64), (1, 33, 2, 2, 128),
               # score rows longer than the LDS holds (three-pass form), past 16k keys, both head sizes
               (19, 40000, 2, 1, 128), (5, 9000, 4, 2, 64)]


def attention_case(M, n_keys, H, Hkv, hd, mode):
    """Run one attention on random Q/K/V; returns (got, f64 reference, q, k, v).  The
    transposed value cache has a padded row (v_ld > n_keys) holding NaN past the
    sequence, which must not leak into the result."""
    q = rng.standard_normal((M, H, hd)).astype(np.float32)
    k = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v_ld = (n_keys + 15) // 16 * 16 + 16
    vt = np.full((Hkv, hd, v_ld), np.nan, np.float32)
    vt[:, :, :n_keys] = v.transpose(1, 2, 0)
    qb, kb, vb, ob = dfx.Buf.of(q), dfx.Buf.of(k), dfx.Buf.of(vt), dfx.Buf(M * H * hd * 4)
    dfx.check(L().dfx_attention_ex(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, ob.ptr, mode, None),
              "attention")
    got = ob.download(np.float32, shape=(M, H, hd))
    rep = H // Hkv
    kd = np.repeat(k.astype(np.float64), rep, axis=1)        # query head h reads KV head h // rep
    vd = np.repeat(v.astype(np.float64), rep, axis=1)
    s = np.einsum("mhd,nhd->hmn", q.astype(np.float64), kd) / np.sqrt(hd)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return got, np.einsum("hmn,nhd->mhd", p, vd), q, k, v


@pytest.mark.parametrize("M,n_keys,H,Hkv,hd", ATTN_SHAPES)
def test_attention_exact_matches_oracle_and_f64(gpu, M, n_keys, H, Hkv, hd):
    """DFX_ATTN_EXACT: bit-exact with the oracle (f64 accumulation of exact products,
    correctly rounded exp), and within 1e-6 of an independent f64 evaluation.  Covers
    the 16-row matrix-core kernel (score rows in LDS) and the VALU kernel (3000 keys)."""
    got, ref, q, k, v = attention_case(M, n_keys, H, Hkv, hd, dfx.ATTN_EXACT)
    assert rel_l2(got, ref) < 1e-6
    exact = O.attention(q, k, v)
    # The f64 sums (products exact) are added in another order than the oracle's; the f32
    # result agrees except where the f64 value lands within an f64 rounding of an f32
    # rounding boundary (about one element in ten million here): at most one f32 ulp.
    diff = got != exact
    assert diff.mean() <= 1e-6, int(diff.sum())
    ulps = np.abs(got.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1, int(ulps.max())
    # the plain entry point is this mode
    qb, kb = dfx.Buf.of(q), dfx.Buf.of(k)
    v_ld = (n_keys + 15) // 16 * 16 + 16
    vt = np.zeros((Hkv, hd, v_ld), np.float32)
    vt[:, :, :n_keys] = v.transpose(1, 2, 0)
    vb, ob = dfx.Buf.of(vt), dfx.Buf(M * H * hd * 4)
    dfx.check(L().dfx_attention(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, ob.ptr, None), "attention")
    assert np.array_equal(ob.download(np.float32, shape=(M, H, hd)), got)


@pytest.mark.parametrize("M,n_keys,H,Hkv,hd", ATTN_SHAPES)
def test_attention_split_bf16_matches_f64(gpu, M, n_keys, H, Hkv, hd):
    """The optional DFX_ATTN_SPLIT_BF16: f32 operands split into bf16 hi + mid + lo,
    products from their six leading terms (error per product < 2^-25 of it) on the bf16
    MFMA with f32 sums and f32 exp.  Bound: rel-L2 <= 1e-6 against an independent f64
    evaluation and the oracle (f32 arithmetic reaches a few 1e-7), every element within
    1e-5 absolute (outputs are O(1): averages of N(0, 1) values).  The
    3000-key and 2000-key cases take the f64 forms (score rows beyond the LDS) and so
    stay exact; row counts and key counts off the 32-row / 32-key tiles, one key,
    GQA and both head sizes cover the tile edges."""
    got, ref, q, k, v = attention_case(M, n_keys, H, Hkv, hd, dfx.ATTN_SPLIT_BF16)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-6, rel_l2(got, ref)
    assert np.abs(got - ref).max() <= 1e-5
    assert rel_l2(got, O.attention(q, k, v)) <= 1e-6


def test_attention_split_bf16_is_more_than_one_bf16_pass(gpu):
    """Large scores (|s| up to ~25) make the softmax sensitive to score error: one bf16
    pass (8 significant bits) misses the f64 result by more than 1e-3, two parts
    (16 bits) by more than the split form's bound.  Checks the split form keeps
    rel-L2 <= 1e-6 there, and that Q and K rounded to one and to two bf16 parts
    (evaluated here in f64) do not."""
    M, n_keys, H, Hkv, hd = 64, 256, 2, 2, 128
    got, ref, q, k, v = attention_case(M, n_keys, H, Hkv, hd, dfx.ATTN_SPLIT_BF16)
    del got
    q = (q * 6).astype(np.float32)
    qb, kb = dfx.Buf.of(q), dfx.Buf.of(k)
    v_ld = (n_keys + 15) // 16 * 16 + 16
    vt = np.zeros((Hkv, hd, v_ld), np.float32)
    vt[:, :, :n_keys] = v.transpose(1, 2, 0)
    vb, ob = dfx.Buf.of(vt), dfx.Buf(M * H * hd * 4)
    dfx.check(L().dfx_attention_ex(qb.ptr, kb.ptr, vb.ptr, v_ld, M, n_keys, H, Hkv, hd, ob.ptr,
                                   dfx.ATTN_SPLIT_BF16, None), "attention")
    got = ob.download(np.float32, shape=(M, H, hd))

    def f64_attn(qq, kk):
        s = np.einsum("mhd,nhd->hmn", qq.astype(np.float64), kk.astype(np.float64)) / np.sqrt(hd)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        return np.einsum("hmn,nhd->mhd", p, v.astype(np.float64))

    def to_bf16(x):
        u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        return u.astype(np.uint32).view(np.float32)

    def two_parts(x):
        h = to_bf16(x)
        return (h.astype(np.float64) + to_bf16(x - h).astype(np.float64))

    ref = f64_attn(q, k)
    assert rel_l2(got, ref) <= 1e-6, rel_l2(got, ref)
    assert rel_l2(f64_attn(to_bf16(q), to_bf16(k)), ref) > 1e-3
    assert rel_l2(f64_attn(two_parts(q), two_parts(k)), ref) > 1e-6


# ---------------------------------------------------------------- sampler kernels
@pytest.mark.parametrize("sigma", [0.5, 2.0, 8.0])
def test_row_stats_matches_oracle(gpu, sigma):
    """Sampler microbench shape: [256 x 126464] N(0, sigma) logits.  argmax / top-1 / top-2
    exact; entropy within 1e-4 relative + 2e-5 absolute.  The reference adds 126464 float terms
    one after another (the GPU sums in double): the rounding walk of its exp-sum, ~1e-5 of the
    sum, moves log(sum) and so the entropy by ~1e-5 absolute whatever the entropy's size, which
    dominates on peaked rows (entropy ~0.01 at sigma 8); measured against an f64 evaluation of
    these rows the reference formula stays within 0.37 of this bound."""
    R, V = 256, 126464
    x = (np.random.default_rng(4).standard_normal((R, V)) * sigma).astype(np.float32)
    x[0, [5, 77]] = x[0].max() + 1.0           # tie on the max: lowest index
    x[1, 0] = x[1].max() + 1.0                 # argmax at index 0
    rows = np.arange(R, dtype=np.int32)[::-1].copy()
    xb, rb, sb = dfx.Buf.of(x), dfx.Buf.of(rows), dfx.Buf(R * 16)
    dfx.check(L().dfx_row_stats(xb.ptr, V, rb.ptr, R, V, sb.ptr, None), "row_stats")
    st = np.frombuffer(sb.download(np.uint8).tobytes(), dtype=dfx.ROW_STAT)
    for i, r in enumerate(rows):
        b, bv, sv = O.top2(x[r])
        assert (st["token"][i], st["best"][i], st["second"][i]) == (b, np.float32(bv), np.float32(sv)), r
        e_ref = O.entropy(x[r])
        assert abs(st["entropy"][i] - e_ref) <= 1e-4 * abs(e_ref) + 2e-5, (r, st["entropy"][i], e_ref)


@pytest.mark.parametrize("remasking", [0, 2, 3, 4])
def test_select_bit_exact(gpu, remasking):
    for trial in range(10):
        n = int(rng.integers(1, 2049)) if trial else 2048
        c = np.zeros(n, dfx.CANDIDATE)
        c["pos"] = rng.permutation(4096)[:n]
        c["token"] = rng.integers(0, 1000, n)
        c["confidence"] = rng.integers(0, 20, n).astype(np.float32) * 0.25
        c["entropy"] = rng.integers(0, 12, n).astype(np.float32) * 0.25
        n_sched = int(rng.integers(1, n + 1))
        cb, ob, nb = dfx.Buf.of(c), dfx.Buf(n * 4), dfx.Buf(4)
        dfx.check(L().dfx_select(cb.ptr, n, remasking, 1.5, n_sched, ob.ptr, nb.ptr, None), "select")
        order = ob.download(np.int32)
        ref, n_ref = O.order_candidates(c, remasking, 1.5, n_sched)
        assert np.array_equal(c[order], ref)
        assert int(nb.download(np.int32)[0]) == n_ref


@pytest.mark.parametrize("remasking", [0, 2, 3, 4])
@pytest.mark.parametrize("n", [1, 17, 256, 1000, 1024, 1025])
def test_select_from_stats_equals_the_two_calls(gpu, remasking, n):
    """dfx_select_from_stats (candidates and selection in one launch, by rank up to 1024
    candidates) writes the candidates, the order and the unmask count of dfx_make_candidates
    + dfx_select, with many equal keys (ties broken by position)."""
    st = np.zeros(n, dfx.ROW_STAT)
    st["token"] = rng.integers(0, 1000, n)
    st["best"] = rng.integers(0, 20, n).astype(np.float32) * 0.25
    st["second"] = st["best"] - rng.integers(0, 8, n).astype(np.float32) * 0.25
    st["entropy"] = rng.integers(0, 12, n).astype(np.float32) * 0.25
    st["best"][:2] = [0.0, -0.0][:n]               # -0 and +0 compare equal: position decides
    pos = rng.permutation(4 * n)[:n].astype(np.int32)
    n_sched = int(rng.integers(1, n + 1))
    sb, pb = dfx.Buf.of(st), dfx.Buf.of(pos)
    outs = []
    for fused in (False, True):
        cb, ob, nb = dfx.Buf(n * 16), dfx.Buf(n * 4), dfx.Buf(4)
        if fused:
            dfx.check(L().dfx_select_from_stats(sb.ptr, pb.ptr, n, remasking, 1.5, n_sched, cb.ptr, ob.ptr, nb.ptr,
                                                None), "select_from_stats")
        else:
            dfx.check(L().dfx_make_candidates(sb.ptr, pb.ptr, n, 1 if remasking == 4 else 0, cb.ptr, None), "cand")
            dfx.check(L().dfx_select(cb.ptr, n, remasking, 1.5, n_sched, ob.ptr, nb.ptr, None), "select")
        outs.append((cb.download(np.uint8).tobytes(), ob.download(np.int32), int(nb.download(np.int32)[0])))
    assert outs[0][0] == outs[1][0]
    assert np.array_equal(outs[0][1], outs[1][1])
    assert outs[0][2] == outs[1][2]


@pytest.mark.parametrize("remasking", [0, 2, 4])
@pytest.mark.parametrize("n", [2049, 5000, 9000])
def test_select_beyond_one_workgroup_bit_exact(gpu, remasking, n):
    """More candidates than one workgroup sorts: placed by rank, the same order as the
    oracle (key, then position), with many equal keys."""
    c = np.zeros(n, dfx.CANDIDATE)
    c["pos"] = rng.permutation(4 * n)[:n]
    c["token"] = rng.integers(0, 1000, n)
    c["confidence"] = rng.integers(-20, 20, n).astype(np.float32) * 0.25
    c["confidence"][:3] = [0.0, -0.0, 0.0]          # -0 and +0 compare equal: position decides
    c["entropy"] = rng.integers(0, 12, n).astype(np.float32) * 0.25
    n_sched = int(rng.integers(1, n + 1))
    cb, ob, nb = dfx.Buf.of(c), dfx.Buf(n * 4), dfx.Buf(4)
    dfx.check(L().dfx_select(cb.ptr, n, remasking, 1.5, n_sched, ob.ptr, nb.ptr, None), "select")
    order = ob.download(np.int32)
    assert np.array_equal(np.sort(order), np.arange(n))
    ref, n_ref = O.order_candidates(c, remasking, 1.5, n_sched)
    assert np.array_equal(c[order], ref)
    assert int(nb.download(np.int32)[0]) == n_ref


def test_row_stats_all_minus_inf_row(gpu):
    """A row with no element above -inf: the reference's argmax stays at index 0 and its
    second-best at the -1e30 sentinel (src/diffuse-sampler.cpp:241-252)."""
    V = 4096
    x = np.full((2, V), -np.inf, np.float32)
    x[1] = rng.standard_normal(V).astype(np.float32)
    rows = np.arange(2, dtype=np.int32)
    xb, rb, sb = dfx.Buf.of(x), dfx.Buf.of(rows), dfx.Buf(2 * 16)
    dfx.check(L().dfx_row_stats(xb.ptr, V, rb.ptr, 2, V, sb.ptr, None), "row_stats")
    st = np.frombuffer(sb.download(np.uint8).tobytes(), dtype=dfx.ROW_STAT)
    b, bv, sv = O.top2(x[0])
    assert (b, bv, sv) == (0, -np.inf, np.float32(-1e30))
    assert (st["token"][0], st["best"][0], st["second"][0]) == (b, np.float32(bv), np.float32(sv))
    b, bv, sv = O.top2(x[1])
    assert (st["token"][1], st["best"][1], st["second"][1]) == (b, np.float32(bv), np.float32(sv))


@pytest.mark.parametrize("N,K,M", [(1000, 4096, 33), (4096, 4096, 288), (640, 12288, 64)])
def test_gemm_f32_matches_oracle(gpu, N, K, M):
    """F32 weights stay F32 (GGML's F32 mul_mat: no activation conversion): f32-accurate
    products and sums against the oracle's f32 products summed in double."""
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    raw = W.view(np.uint8).reshape(-1)
    X = rng.standard_normal((M, K)).astype(np.float32)
    got = gpu_gemm(dfx.TYPE_F32, raw, N, K, X)
    ref = O.mul_mat(dfx.TYPE_F32, raw, N, K, X)
    # f32 sums over K = 4096 .. 12288 products (measured 1e-6 .. 2e-6 from the double sums)
    assert rel_l2(got, ref) < 1e-5, rel_l2(got, ref)
    f64 = X.astype(np.float64) @ W.astype(np.float64).T
    assert rel_l2(got, f64) < 1e-5


# (N, K, M, forced tile): Q|K|V at 181, 256 and 288 rows (the default rule splits some of the
# 288 / 384 / 480 tiles over 512 workgroup slots) and gate|up at 288 rows (960 tiles: not
# split), gate|up at 181 rows (96-row tiles, 384 of them: split); forced (half the tiles split):
# Dream-7B's K = 3584 (a short second chunk), one and several tile rows, ragged M, the 96-row
# tile; N off a multiple of 128 and one-chunk K run as dfx_gemm
COUNTED_CASES = [(12288, 4096, 256, None), (12288, 4096, 288, None), (12288, 4096, 181, None), (24576, 4096, 288, None),
                 (4608, 3584, 200, "w1f"), (4096, 4096, 77, "w1f"), (2048, 4096, 33, "w1f"), (1024, 4096, 300, "w1f"),
                 (1000, 4096, 100, "w1f"), (512, 2048, 70, "w1f"), (24576, 4096, 181, None), (4096, 4096, 130, "w3f")]


@pytest.mark.parametrize("N,K,M,tile", COUNTED_CASES)
def test_gemm_counted_equals_dfx_gemm(gpu, N, K, M, tile):
    """dfx_gemm_counted (column tiles split over two workgroups of one launch, the later adding
    the chunk totals) gives dfx_gemm's bits, with bias and an in-place residual, on two calls in
    a row; the tile counters are zero again after each call."""
    typ = dfx.TYPE_Q4_K
    raw = quant(typ, N, K)
    w = to_device_weights(typ, raw, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    r0 = rng.standard_normal((M, N)).astype(np.float32)
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    bb = dfx.Buf.of(bias)
    ref_b, got_b = dfx.Buf.of(r0), dfx.Buf.of(r0)
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, bb.ptr, ref_b.ptr, ref_b.ptr, None, None), "gemm")
    ref = ref_b.download(np.float32, shape=(M, N))
    ws = dfx.Buf(L().dfx_gemm_ws_bytes(M, N, K))
    cnt = dfx.Buf(L().dfx_gemm_tile_cnt_bytes(M, N))
    cnt.zero()
    with forced_tile(typ, tile) if tile else contextlib.nullcontext():
        for call in range(2):
            got_b.upload(r0)
            dfx.check(L().dfx_gemm_counted(typ, w.ptr, N, K, ab.ptr, M, bb.ptr, got_b.ptr, got_b.ptr, ws.ptr, cnt.ptr,
                                           None), "gemm_counted")
            got = got_b.download(np.float32, shape=(M, N))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (call, rel_l2(got, ref))
            assert not cnt.download(np.int32).any()
    if (N, K, M) == (4096, 4096, 77):
        plain = dfx.Buf(M * N * 4)
        cnt.zero()
        with forced_tile(typ, tile):
            dfx.check(L().dfx_gemm_counted(typ, w.ptr, N, K, ab.ptr, M, None, None, plain.ptr, ws.ptr, cnt.ptr, None),
                      "gemm_counted")
        got = plain.download(np.float32, shape=(M, N))
        oracle = O.mul_mat(typ, raw, N, K, X)
        assert np.array_equal(got.view(np.uint32), oracle.view(np.uint32))
