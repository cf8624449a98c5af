"""dfx_gemm_noalloc: the GEMM whose split-K workspace is the library's own device array
(no allocation on any call) gives the bits of dfx_gemm with a caller workspace, call after
call on the same array (the second call smaller than the first), and refuses shapes whose
partial sums exceed the array."""
import numpy as np
import pytest

import dfx

pytestmark = pytest.mark.gpu
L = dfx.lib
rng = np.random.default_rng(31)


def _case(typ, N, K, M, residual=False):
    x = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    raw = dfx.quantize_rows(typ, x)
    w = dfx.Buf.of(dfx.repack(typ, raw, N, K))
    X = rng.standard_normal((M, K), dtype=np.float32)
    xb, ab = dfx.Buf.of(X), dfx.Buf(L().dfx_act_bytes(typ, M, K))
    dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
    res = rng.standard_normal((M, N), dtype=np.float32) if residual else None
    return w, ab, res


def _run(typ, w, ab, N, K, M, res, noalloc):
    yb = dfx.Buf.of(res) if res is not None else dfx.Buf(M * N * 4)
    rp = yb.ptr if res is not None else None
    if noalloc:
        dfx.check(L().dfx_gemm_noalloc(typ, w.ptr, N, K, ab.ptr, M, None, rp, yb.ptr, None), "gemm_noalloc")
    else:
        ws = dfx.Buf(L().dfx_gemm_ws_bytes(M, N, K))
        dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, rp, yb.ptr, ws.ptr, None), "gemm")
    return yb.download(np.float32, shape=(M, N))


# (type, N, K, M, residual): the first call of each pair is the larger; K spans 6 and 2
# 2048-element chunks, so the split-K path (partials in the array) runs
@pytest.mark.parametrize("calls", [
    [(dfx.TYPE_Q4_K, 4096, 12288, 64, True), (dfx.TYPE_Q4_K, 1024, 4096, 20, False)],
    [(dfx.TYPE_Q6_K, 2048, 12288, 100, False), (dfx.TYPE_Q6_K, 640, 4096, 33, True)],
    [(dfx.TYPE_F16, 4096, 12288, 64, False), (dfx.TYPE_F16, 1000, 4096, 33, False)],
])
def test_noalloc_gemm_matches_dfx_gemm(gpu, calls):
    for typ, N, K, M, residual in calls:
        w, ab, res = _case(typ, N, K, M, residual)
        want = _run(typ, w, ab, N, K, M, res, noalloc=False)
        got = _run(typ, w, ab, N, K, M, res, noalloc=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (typ, N, K, M)


def test_noalloc_gemm_refuses_partials_beyond_its_array(gpu):
    typ, N, K, M = dfx.TYPE_Q4_K, 16384, 4096, 288       # 288 * 16384 * 2 chunks * 4 B = 36 MiB
    w, ab, _ = _case(typ, N, K, M)                        # buffers of the real shape
    yb = dfx.Buf(M * N * 4)
    rc = L().dfx_gemm_noalloc(typ, w.ptr, N, K, ab.ptr, M, None, None, yb.ptr, None)
    assert rc == -1 and b"scratch" in L().dfx_last_error()
