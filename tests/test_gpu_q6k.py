"""Q6_K weights (block_q6_K; the token table and tied LM head of real Qwen3 GGUFs, sn_load.inc.h:341-359,
kernels.metal:1010-1120) on the GPU against the oracle (ggml CPU semantics: dequantize_row_q6_K, quantize_row_q8_K_ref
activations, vec_dot_q6_K_q8_K), through the C ABI (include/sn_kernels.h).

Bar: dequantized weights and Q8_K activations bit-exact; matmul outputs within 1e-3 relative / 2e-3 absolute of the
oracle (the per-group integer dots are exact; only the fp32 order across blocks differs); a row's result bitwise
independent of the other rows.
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U
from tests.test_oracle import pack_q6_K

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-3


def setup_module(module):
    U.torch().cuda.init()


def random_q6k(r, N, K, d_scale=1e-4):
    """N rows of K/256 random valid Q6_K blocks (every quant and scale byte pattern occurs)"""
    nb = K // 256
    q = r.integers(0, 64, (N * nb, 256))
    sc = r.integers(-128, 128, (N * nb, 16))
    d = (r.standard_normal(N * nb) * d_scale).astype(np.float16)
    return pack_q6_K(q, sc, d).reshape(N, nb * 210)


def tiles(Wq, N, K):
    L = S.lib()
    t = U.empty(L.snk_q6k_tiles_bytes(N, K))
    assert L.snk_q6k_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(t), U.stream()) == 0
    return t


def xk_gpu(X, norm=None, eps=1e-6):
    L = S.lib()
    M, K = X.shape
    xk = U.empty(L.snk_xk_bytes(M, K))
    nw = U.dev(norm.astype(np.float32)) if norm is not None else None
    assert L.snk_quant_q8k(U.ptr(U.dev(X.astype(np.float32))), M, K, K, U.ptr(nw) if nw is not None else None, eps,
                           U.ptr(xk), U.stream()) == 0
    return xk


def gemm_q6k(t, xk, M, N, K):
    L = S.lib()
    y = U.empty(M * N * 4)
    assert L.snk_q6k_gemm(U.ptr(t), U.ptr(xk), M, N, K, U.ptr(y), N, U.stream()) == 0
    return U.host(y, np.float32)[:M * N].reshape(M, N)


def xk_decode(xk, M, K):
    """the records back to (q [M][K] int, d [M][K/256]): undoes the fragment order (lane m + 32 h of group G's fragment
    holds row m's int8 q of elements 16 G + 8 h .. + 7)"""
    nb = K // 256
    mt = (M + 31) // 32
    rec = U.host(xk, np.uint8)[:mt * nb * 8320].reshape(mt, nb, 8320)
    frag = rec[:, :, :8192].copy().view(np.int8).reshape(mt, nb, 16, 2, 32, 8)  # [mt][b][G][h][m][j]
    q = frag.transpose(0, 4, 1, 2, 3, 5).reshape(mt * 32, K)[:M].astype(np.int64)
    d = rec[:, :, 8192:8320].copy().view(np.float32).reshape(mt, nb, 32).transpose(0, 2, 1).reshape(mt * 32, nb)[:M]
    return q, d


def test_q6k_dequant_bit_exact():
    r = np.random.default_rng(70)
    N, K = 37, 512
    Wq = random_q6k(r, N, K)
    Wq[3, 208:210] = np.array([0], np.float16).view(np.uint8)  # d = 0
    Wq[5, 208:210] = np.array([-6.1e-5], np.float16).view(np.uint8)  # near the subnormal edge
    Wq[6, 208:210] = np.array([2e-7], np.float16).view(np.uint8)  # subnormal
    L = S.lib()
    out = U.empty(N * K * 4)
    assert L.snk_q6k_dequant(U.ptr(tiles(Wq, N, K)), N, K, U.ptr(out), U.stream()) == 0
    got = U.host(out, np.float32)[:N * K].reshape(N, K)
    want = O.dequantize_q6_K(Wq, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q8k_activations_bit_exact():
    r = np.random.default_rng(71)
    M, K = 21, 768
    X = (r.standard_normal((M, K)) * 2).astype(np.float32)
    X[2, 100] = -9.0  # a negative extreme
    X[3, 300], X[3, 301] = 4.0, -4.0  # equal |x|: the first is the extreme
    X[4, 256:512] = 0.0  # an all-zero block
    X[5, :] = 0.0
    q, d = xk_decode(xk_gpu(X), M, K)
    want = O.quantize_q8_K(X).reshape(M, K // 256, 292)
    wq = want[:, :, 4:260].copy().view(np.int8).reshape(M, K).astype(np.int64)
    wd = want[:, :, :4].copy().view(np.float32).reshape(M, K // 256)
    assert np.array_equal(q, wq)
    assert np.array_equal(d.view(np.uint32), wd.view(np.uint32))
    # with the output norm fused: the quantizer of the normed rows (the norm to fp32 rounding)
    nw = (1 + 0.1 * r.standard_normal(K)).astype(np.float32)
    qn, dn = xk_decode(xk_gpu(X, nw), M, K)
    Xn = O.rmsnorm(X, nw, 1e-6)
    wn = O.quantize_q8_K(Xn).reshape(M, K // 256, 292)
    diff = np.abs(qn - wn[:, :, 4:260].copy().view(np.int8).reshape(M, K).astype(np.int64))
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3  # one-step flips where the norm's last bit differs


@pytest.mark.parametrize("M,N,K", [(1, 1000, 256), (8, 4096, 2560), (32, 5000, 1024), (17, 2049, 768), (33, 300, 512),
                                   (64, 1000, 512), (100, 777, 256)])
def test_q6k_matmul_vs_oracle(M, N, K):
    r = np.random.default_rng(M * 7 + N)
    Wq = random_q6k(r, N, K)
    X = r.standard_normal((M, K)).astype(np.float32)
    got = gemm_q6k(tiles(Wq, N, K), xk_gpu(X), M, N, K)
    want = O.mul_mat_q6_K(Wq, K, X)
    err = np.abs(got - want)
    print(f"q6k {M}x{N}x{K}: max abs err {err.max():.3g}, max |y| {np.abs(want).max():.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(want))


def test_q6k_matmul_row_invariance():
    r = np.random.default_rng(73)
    N, K = 1500, 1024
    Wq = random_q6k(r, N, K)
    t = tiles(Wq, N, K)
    X = r.standard_normal((40, K)).astype(np.float32)
    full = gemm_q6k(t, xk_gpu(X), 40, N, K)
    for i in (0, 17, 39):
        one = gemm_q6k(t, xk_gpu(X[i:i + 1]), 1, N, K)
        assert np.array_equal(one[0].view(np.uint32), full[i].view(np.uint32)), i
