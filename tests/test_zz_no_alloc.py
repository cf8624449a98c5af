"""dfx_gemm_noalloc: the GEMM whose split-K workspace is the library's own device array
(no allocation on any call) gives the bits of dfx_gemm with a caller workspace, call after
call on the same array (the second call smaller than the first), keeps K whole where the
partial sums would not fit the array, and works as the first call of a process made under
stream capture."""
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


def test_noalloc_gemm_without_room_to_split_keeps_k_whole(gpu):
    """A quantised shape whose split-K partials would exceed the array (LLaDA-8B gate|up at
    288 rows: 288 * 24576 * 2 chunks * 4 B = 54 MiB) runs with K whole: the chunk sums are
    added in chunk order either way, so the bits are dfx_gemm's (which splits)."""
    typ, N, K, M = dfx.TYPE_Q4_K, 24576, 4096, 288
    assert M * N * 2 * 4 > 32 << 20
    w, ab, res = _case(typ, N, K, M, residual=True)
    want = _run(typ, w, ab, N, K, M, res, noalloc=False)
    got = _run(typ, w, ab, N, K, M, res, noalloc=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


CAPTURE_SCRIPT = r"""
import ctypes as C, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import dfx
hip = C.CDLL("libamdhip64.so")
L = dfx.lib
rng = np.random.default_rng(5)
typ, N, K, M = dfx.TYPE_Q4_K, 4096, 12288, 64          # K of six chunks: split K, partials in the array
raw = dfx.quantize_rows(typ, rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
w = dfx.Buf.of(dfx.repack(typ, raw, N, K))
xb, ab = dfx.Buf.of(rng.standard_normal((M, K), dtype=np.float32)), dfx.Buf(L().dfx_act_bytes(typ, M, K))
dfx.check(L().dfx_act_convert(typ, xb.ptr, M, K, ab.ptr, None), "convert")
ws = dfx.Buf(L().dfx_gemm_ws_bytes(M, N, K))
want_b = dfx.Buf(M * N * 4)
dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, None, want_b.ptr, ws.ptr, None), "gemm")
dfx.sync()
want = want_b.download(np.float32, shape=(M, N))
st, graph, ex = C.c_void_p(), C.c_void_p(), C.c_void_p()
assert hip.hipStreamCreateWithFlags(C.byref(st), 1) == 0                # non-blocking
got_b = dfx.Buf(M * N * 4)
assert hip.hipStreamBeginCapture(st, 0) == 0                            # global capture mode
rc = L().dfx_gemm_noalloc(typ, w.ptr, N, K, ab.ptr, M, None, None, got_b.ptr, st)   # first call in this process
assert hip.hipStreamEndCapture(st, C.byref(graph)) == 0
dfx.check(rc, "gemm_noalloc under capture")
assert hip.hipGraphInstantiate(C.byref(ex), graph, None, None, 0) == 0
for rep in range(3):
    got_b.zero()
    dfx.check(L().dfx_gemm(typ, w.ptr, N, K, ab.ptr, M, None, None, want_b.ptr, ws.ptr, None), "gemm")
    dfx.sync()
    assert hip.hipGraphLaunch(ex, st) == 0
    assert hip.hipStreamSynchronize(st) == 0
    got = got_b.download(np.float32, shape=(M, N))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
print("capture ok")
"""


def test_noalloc_gemm_first_call_under_stream_capture(gpu, tmp_path):
    """The first dfx_gemm_noalloc call of a process (the one that looks up the array's device
    address) made inside a global-mode capture on a non-blocking stream: the capture succeeds,
    and every replay of the graph (with eager GEMMs and synchronisations between replays)
    gives dfx_gemm's bits.  A child process, so that no earlier call has done the lookup."""
    import os
    import subprocess
    import sys
    script = tmp_path / "capture.py"
    script.write_text(CAPTURE_SCRIPT)
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "diffuse-cpp_amd")
    r = subprocess.run([sys.executable, str(script), pkg], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "capture ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
