"""Q8_0 weights (block_q8_0, kernels.metal:9; the reference's mv_q8_0* kernels, :1995-2130, and Q8_0 dequant, :597-609)
on the GPU against the oracle (ggml CPU semantics: dequantize_row_q8_0, quantize_row_q8_0 activations,
vec_dot_q8_0_q8_0), through the C ABI (include/sn_kernels.h) and through sn.h with a Q8_0 model.

Tolerances: dequantized weights bit-exact (d * q); outputs within 1e-3 relative / 2e-3
absolute of the oracle (the integer block sums are exact; only the fp32 order across blocks differs); a row's result
bitwise independent of the other rows.
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-3
WT_Q8_0 = 8


def setup_module(module):
    U.torch().cuda.init()


def tiles(Wq, N, K):
    L = S.lib()
    wbuf = U.empty(L.snk_q8_tiles_bytes(N, K))
    assert L.snk_q8_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), U.stream()) == 0
    return wbuf


def gemm_q8(Wq, N, K, X, epi=0, y0=None, wbuf=None):
    L = S.lib()
    st = U.stream()
    M = X.shape[0]
    wbuf = tiles(Wq, N, K) if wbuf is None else wbuf
    x = U.dev(X.astype(np.float32))
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(x), M, K, K, None, 0.0, U.ptr(xa), st) == 0
    outN = N // 2 if epi == 2 else N
    y = U.dev(y0.astype(np.float32)) if y0 is not None else U.empty(M * outN * 4)
    wsb = L.snk_q8_workspace_bytes(M, N, K)
    ws = U.empty(wsb)
    assert L.snk_q8_gemm(U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y), outN, epi, U.ptr(ws), wsb, st) == 0
    return U.host(y, np.float32)[:M * outN].reshape(M, outN), U.host(xa, np.uint8)


def test_q8_dequant_bit_exact():
    # every int8 value (-128 too, which ggml's quantizer never writes) and fp16 scale specials: 0, subnormal, negative
    N, K = 40, 352
    r = np.random.default_rng(31)
    Wq = r.integers(0, 256, (N, K // 32 * 34), dtype=np.uint8)
    blocks = Wq.reshape(N, K // 32, 34)
    blocks[0, 0, 2:] = np.arange(32, dtype=np.uint8)  # q = 0..31
    blocks[0, 1, 2:] = np.arange(224, 256, dtype=np.uint8)  # q = -32..-1 (and -128 elsewhere)
    blocks[1, 0, 2:] = 128  # q = -128
    d = r.normal(0, 0.01, (N, K // 32)).astype(np.float16)
    d[2, 0] = 0.0
    d[2, 1] = np.float16(1e-6)  # subnormal
    d[3, :] = -np.abs(d[3, :])
    blocks[:, :, :2] = d.view(np.uint8).reshape(N, K // 32, 2)
    L = S.lib()
    wbuf = tiles(Wq, N, K)
    out = U.empty(N * K * 4)
    assert L.snk_q8_dequant(U.ptr(wbuf), N, K, U.ptr(out), U.stream()) == 0
    got = U.host(out, np.float32)[:N * K].reshape(N, K)
    want = O.dequantize_q8_0(Wq, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(8, 4096, 4096), (1, 1000, 256), (3, 160, 96), (17, 6144, 2560), (32, 2560, 9728),
                                   (33, 1024, 4096), (300, 1000, 512)])
def test_q8_matmul_vs_oracle(M, N, K):
    r = np.random.default_rng(M * 7 + N)
    Wq = O.quantize_q8_0_ref(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    Y, xa = gemm_q8(Wq, N, K, X)
    U.xa_decode(xa, M, K)  # checks the operand's corrections
    ref = O.mul_mat_q8_0(Wq, K, X)
    err = np.abs(Y - ref)
    print(f"Q8_0 {M}x{N}x{K}: max abs err {err.max():.3g}")
    assert np.allclose(Y, ref, rtol=RTOL, atol=ATOL), err.max()


def test_q8_epilogues_and_row_invariance():
    r = np.random.default_rng(32)
    N, K = 512, 1024
    Wq = O.quantize_q8_0_ref(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (33, K)).astype(np.float32)
    wbuf = tiles(Wq, N, K)
    Y, _ = gemm_q8(Wq, N, K, X, wbuf=wbuf)
    for i in (0, 16, 32):  # each row alone equals its row in the 33-row matmul, bit for bit
        Yi, _ = gemm_q8(Wq, N, K, X[i:i + 1], wbuf=wbuf)
        assert np.array_equal(Yi[0].view(np.uint32), Y[i].view(np.uint32))
    # 280 rows (row tiles in pairs, from other offsets) hold the same 33 rows' results
    Xl = np.concatenate([r.normal(0, 1, (200, K)).astype(np.float32), X, X[:47]])
    Yl, _ = gemm_q8(Wq, N, K, Xl, wbuf=wbuf)
    assert np.array_equal(Yl[200:233].view(np.uint32), Y.view(np.uint32))
    y0 = r.normal(0, 1, (33, N)).astype(np.float32)
    Ya, _ = gemm_q8(Wq, N, K, X, epi=1, y0=y0, wbuf=wbuf)
    assert np.allclose(Ya, y0 + Y, rtol=1e-6, atol=1e-6)


TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000)
MODEL_ATOL = 3e-2  # the end-to-end logit bound of the 2-layer test models (Q8_0 activation noise)


def test_q8_model_decode_vs_oracle(tmp_path):
    path = str(tmp_path / "tiny_q8.gguf")
    S.write_model(path, S.model_cfg(**TINY, wtype=WT_Q8_0), seed=13)
    ref = O.Qwen3(GGUF(path), n_seq=2, ctx=128)
    assert ref.wtype == WT_Q8_0
    r = np.random.default_rng(33)
    tok = r.integers(0, TINY["n_vocab"], 20).astype(np.int32)
    checked = 0
    with S.Engine(path, slots=2, ctx=128, max_rows=32) as eng:
        got = eng.step(tok, np.zeros(20, np.int32), np.arange(20, dtype=np.int32), np.array([19], np.int32), n_write=0)
        lg = eng.logits([0])
        rt, rl, _ = ref.step(tok, np.zeros(20, np.int32), np.arange(20, dtype=np.int32), np.array([19], np.int32))
        assert np.allclose(lg, rl, rtol=0, atol=MODEL_ATOL), float(np.abs(lg - rl).max())
        cur, pos = int(got[0]), 20
        for _ in range(6):  # greedy decode, fed its own tokens; compared where the oracle's top-2 gap is clear
            g1 = eng.step(np.array([cur], np.int32), np.zeros(1, np.int32), np.array([pos], np.int32),
                          np.array([0], np.int32))
            l1 = eng.logits([0])
            t1, r1, _ = ref.step(np.array([cur], np.int32), np.zeros(1, np.int32), np.array([pos], np.int32),
                                 np.array([0], np.int32))
            assert np.allclose(l1, r1, rtol=0, atol=MODEL_ATOL), float(np.abs(l1 - r1).max())
            i1, v1, i2, v2, _ = O.top2(r1[0])
            if v1 - v2 > 2 * MODEL_ATOL:
                assert g1[0] == t1[0]
                checked += 1
            cur, pos = int(t1[0]), pos + 1
    print(f"Q8_0 model: {checked} of 6 decode tokens compared")
