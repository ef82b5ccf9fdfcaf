"""snk_q4_gemm_noalloc (the matmul whose k-slice partials live in the library's fixed device array) against
snk_q4_gemm (the same kernels with a caller-given workspace), through the C ABI: bit for bit on two calls in a row,
the second with a smaller input (the array keeps the first call's contents, which must not leak into the second),
each epilogue, and a shape whose partials would exceed the array refused with its reason before anything runs."""
import ctypes as C

import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu


def setup_module(module):
    U.torch().cuda.init()


def operands(r, M, N, K):
    L = S.lib()
    st = U.stream()
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), st) == 0
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(U.dev(X)), M, K, K, None, 0.0, U.ptr(xa), st) == 0
    return Wq, X, wbuf, xa


def both(wbuf, xa, M, N, K, epi, y0):
    """(workspace entry point, no-allocation entry point) outputs on the same operands"""
    L = S.lib()
    st = U.stream()
    outN = N // 2 if epi == 2 else N
    ya, yb = U.dev(y0), U.dev(y0)
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    ws = U.empty(wsb)
    assert L.snk_q4_gemm(U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(ya), outN, epi, U.ptr(ws), wsb, st) == 0
    S.call(L.snk_q4_gemm_noalloc, U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(yb), outN, epi, st)
    n = M * outN
    return U.host(ya, np.float32)[:n].reshape(M, outN), U.host(yb, np.float32)[:n].reshape(M, outN)


@pytest.mark.parametrize("epi", [0, 1, 2])
def test_noalloc_equals_workspace_call(epi):
    r = np.random.default_rng(70 + epi)
    # a large call (k-split: partials of several slices) then a smaller one on the same array
    for M, N, K in ((32, 4096, 2560), (5, 1024, 4096)):
        Wq, X, wbuf, xa = operands(r, M, N, K)
        outN = N // 2 if epi == 2 else N
        y0 = r.normal(0, 1, (M, outN)).astype(np.float32)
        a, b = both(wbuf, xa, M, N, K, epi, y0)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (M, N, K, epi)
        if epi == 0:
            ref = O.mul_mat_q4_0(Wq, K, X)
            assert np.all(np.abs(b - ref) <= 2e-3 + 1e-3 * np.abs(ref))


def test_noalloc_refuses_shapes_beyond_the_array():
    L = S.lib()
    M, N, K = 64, 151936, 2560  # 64 x 151,936 fp32 partials: 38.9 MB > 32 MiB
    assert L.snk_q4_workspace_bytes(M, N, K) > 32 << 20
    buf = C.create_string_buffer(512)
    # refused on the host before any launch (the pointers are never touched)
    rc = L.snk_q4_gemm_noalloc(None, None, M, N, K, None, N, 0, U.stream(), buf, 512)
    assert rc == -1 and b"scratch array holds" in buf.value, buf.value


def test_noalloc_under_graph_capture():
    """A warm call (the device array's address looked up), then one call captured into a HIP graph and replayed
    several times, with eager work of the program between the replays: every replay bit for bit the eager result."""
    T = U.torch()
    L = S.lib()
    r = np.random.default_rng(77)
    M, N, K = 32, 2560, 4096
    Wq, X, wbuf, xa = operands(r, M, N, K)
    y_eager, y_graph = U.empty(M * N * 4), U.empty(M * N * 4)
    S.call(L.snk_q4_gemm_noalloc, U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y_eager), N, 0, U.stream())
    want = U.host(y_eager, np.float32)[:M * N].copy()
    g = T.cuda.CUDAGraph()
    side = T.cuda.Stream()
    side.wait_stream(T.cuda.current_stream())
    with T.cuda.stream(side):
        S.call(L.snk_q4_gemm_noalloc, U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y_graph), N, 0, U.stream())  # (warm)
        with T.cuda.graph(g, stream=side):
            S.call(L.snk_q4_gemm_noalloc, U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y_graph), N, 0,
                   C.c_void_p(side.cuda_stream))
    T.cuda.current_stream().wait_stream(side)
    for rep in range(4):
        y_graph.fill_(0xFF)  # eager work between the replays (a fill kernel, outside the graph)
        g.replay()
        got = U.host(y_graph, np.float32)[:M * N]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        # the eager call again on another output, between replays
        S.call(L.snk_q4_gemm_noalloc, U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y_eager), N, 0, U.stream())
        assert np.array_equal(U.host(y_eager, np.float32)[:M * N].view(np.uint32), want.view(np.uint32)), rep
