"""Q4_0 x Q8_0 matmul on the GPU against the oracle (ggml CPU semantics), through the C ABI (include/sn_kernels.h).

Tolerances: dequantized weights bit-exact with dequantize_row_q4_0; Q8_0 activations
bit-exact with the oracle's quantizer on identical inputs; outputs within 1e-3 relative / 2e-3 absolute of the oracle
(the only difference is the fp32 summation order).
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-3


def setup_module(module):
    U.torch().cuda.init()


def gemm_gpu(Wq, N, K, X, epi=0, y0=None, wbuf=None):
    L = S.lib()
    st = U.stream()
    M = X.shape[0]
    if wbuf is None:
        wraw = U.dev(Wq)
        wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
        assert L.snk_q4_repack(U.ptr(wraw), N, K, U.ptr(wbuf), st) == 0
    x = U.dev(X.astype(np.float32))
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(x), M, K, K, None, 0.0, U.ptr(xa), st) == 0
    outN = N // 2 if epi == 2 else N
    y = U.dev(y0.astype(np.float32)) if y0 is not None else U.empty(M * outN * 4)
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    ws = U.empty(wsb)
    assert L.snk_q4_gemm(U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y), outN, epi, U.ptr(ws), wsb, st) == 0
    return U.host(y, np.float32)[:M * outN].reshape(M, outN), U.host(xa, np.uint8)


def test_mfma_layout_probe():
    # A[i][k] at lane i + 16 (k // 8), slot k % 8; B[k][j] at lane j + 16 (k // 8), slot k % 8;
    # D[i][j] at lane j + 16 (i // 4), slot i % 4 -- the layout every kernel here assumes.
    r = np.random.default_rng(0)
    A = r.integers(-4, 5, (16, 32)).astype(np.float16)
    B = r.integers(-4, 5, (32, 16)).astype(np.float16)
    a = np.zeros((64, 8), np.float16)
    b = np.zeros((64, 8), np.float16)
    for lane in range(64):
        for s in range(8):
            a[lane, s] = A[lane % 16, 8 * (lane // 16) + s]
            b[lane, s] = B[8 * (lane // 16) + s, lane % 16]
    da, db = U.dev(a), U.dev(b)
    dd = U.empty(64 * 4 * 4)
    assert S.lib().snk_mfma_probe(U.ptr(da), U.ptr(db), U.ptr(dd), U.stream()) == 0
    d = U.host(dd, np.float32)[:256].reshape(64, 4)
    D = A.astype(np.float32) @ B.astype(np.float32)
    want = np.zeros((64, 4), np.float32)
    for lane in range(64):
        for v in range(4):
            want[lane, v] = D[4 * (lane // 16) + v, lane % 16]
    assert np.array_equal(d, want)


def test_dequant_bit_exact():
    r = np.random.default_rng(1)
    N, K = 200, 352  # rows not a multiple of 16, blocks not a multiple of 4
    w = r.normal(0, 0.02, (N, K)).astype(np.float32)
    w[0, :32] = 0
    Wq = O.quantize_q4_0(w)
    L = S.lib()
    wraw = U.dev(Wq)
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    st = U.stream()
    assert L.snk_q4_repack(U.ptr(wraw), N, K, U.ptr(wbuf), st) == 0
    out = U.empty(N * K * 4)
    assert L.snk_q4_dequant(U.ptr(wbuf), N, K, U.ptr(out), st) == 0
    got = U.host(out, np.float32)[:N * K].reshape(N, K)
    want = O.dequantize_q4_0(Wq, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_activation_quantization_bit_exact():
    r = np.random.default_rng(2)
    M, K = 37, 2560
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    X[3, :64] = 0.0
    X[5] *= 1e-3
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (16, K)).astype(np.float32))
    _, xa = gemm_gpu(Wq, 16, K, X)
    q, d = U.xa_decode(xa, M, K)
    blocks = O.quantize_q8_0(X).reshape(M, K // 32, 34)
    want_d = blocks[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float32)
    want_q = blocks[:, :, 2:].view(np.int8).astype(np.float32).reshape(M, K)
    # the same Q8_0 blocks, bit for bit: every scale and every integer
    assert np.array_equal(d, want_d)
    assert np.array_equal(q, want_q)


def test_config1_q4_matmul_4096x4096_b8():
    # W 4096x4096 ~ N(0, 0.02) quantized with ggml's reference quantizer, X [8, 4096] ~ N(0, 1)
    r = np.random.default_rng(1)
    N = K = 4096
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (8, K)).astype(np.float32)
    Y, _ = gemm_gpu(Wq, N, K, X)
    ref = O.mul_mat_q4_0(Wq, K, X)
    err = np.abs(Y - ref)
    print(f"config 1: max abs err {err.max():.3g}, max rel {np.max(err / (np.abs(ref) + 1e-30)):.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref))
    # the exact value: fp64 over the Q8_0 activations
    ex = O.mul_mat_q4_0_f64(Wq, K, O.dequantize_q8_0(O.quantize_q8_0(X), K))
    assert np.max(np.abs(Y - ex)) <= 1e-5 * np.max(np.abs(ex))


@pytest.mark.parametrize("M,N,K", [(1, 1000, 256), (3, 160, 96), (16, 512, 512), (17, 6144, 2560), (32, 2560, 9728),
                                   (33, 1024, 4096), (64, 304, 1024), (300, 1000, 512), (512, 2560, 1024)])
def test_matmul_shapes(M, N, K):
    r = np.random.default_rng(M * 7 + N)
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    Y, _ = gemm_gpu(Wq, N, K, X)
    ref = O.mul_mat_q4_0(Wq, K, X)
    assert np.all(np.abs(Y - ref) <= ATOL + RTOL * np.abs(ref))


def test_epilogue_add_and_swiglu():
    r = np.random.default_rng(3)
    M, F, K = 20, 256, 512
    Wg = O.quantize_q4_0(r.normal(0, 0.02, (F, K)).astype(np.float32))
    Wu = O.quantize_q4_0(r.normal(0, 0.02, (F, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    # add into an existing output
    y0 = r.normal(0, 1, (M, F)).astype(np.float32)
    Y, _ = gemm_gpu(Wg, F, K, X, epi=1, y0=y0)
    ref = y0 + O.mul_mat_q4_0(Wg, K, X)
    assert np.all(np.abs(Y - ref) <= ATOL + RTOL * np.abs(ref))
    # SwiGLU over gate / up stripes interleaved in pairs
    L = S.lib()
    st = U.stream()
    sb = L.snk_q4_stripes_bytes(F, K)
    gb, ub = U.empty(sb), U.empty(sb)
    assert L.snk_q4_repack(U.ptr(U.dev(Wg)), F, K, U.ptr(gb), st) == 0
    assert L.snk_q4_repack(U.ptr(U.dev(Wu)), F, K, U.ptr(ub), st) == 0
    per = sb // (F // 16)
    g = U.host(gb, np.uint8)[:sb].reshape(F // 16, per)
    u = U.host(ub, np.uint8)[:sb].reshape(F // 16, per)
    inter = np.stack([g, u], axis=1).reshape(-1)
    Y, _ = gemm_gpu(None, 2 * F, K, X, epi=2, wbuf=U.dev(inter))
    gg = O.mul_mat_q4_0(Wg, K, X).astype(np.float64)
    uu = O.mul_mat_q4_0(Wu, K, X).astype(np.float64)
    ref = gg / (1 + np.exp(-gg)) * uu
    assert np.all(np.abs(Y - ref) <= ATOL + RTOL * np.abs(ref))


def test_row_invariance_bitwise():
    # a row's result is the same whatever the other rows of the step (sn.h:1-3; qbench.m's b1 == b8 == b32)
    r = np.random.default_rng(4)
    N, K = 1536, 2560
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    # 300 rows: every matrix takes its row tiles in pairs (prompt rows); the 1..40-row subsets single tiles here
    X = r.normal(0, 1, (300, K)).astype(np.float32)
    L = S.lib()
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), U.stream()) == 0
    full, _ = gemm_gpu(None, N, K, X, wbuf=wbuf)
    for rows in ([0], [5, 6, 7], list(range(17)), list(range(8, 40)), list(range(43, 300))):
        part, _ = gemm_gpu(None, N, K, X[rows], wbuf=wbuf)
        assert np.array_equal(part.view(np.uint32), full[rows].view(np.uint32))


@pytest.mark.parametrize("N,K", [(6144, 2560), (19456, 2560), (2560, 9728)])
def test_row_invariance_prompt_shapes(N, K):
    """The Qwen3-4B layer matrices (q|k|v, gate|up, down) at 300 prompt rows, where one workgroup walks every k-slice
    of its tiles and adds them in slice order itself, against decode-sized subsets of the same rows, which the split
    launches and the consumer's slice sum serve: every row bit for bit the same (sn.h:1-3)."""
    r = np.random.default_rng(N + K)
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (300, K)).astype(np.float32)
    L = S.lib()
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), U.stream()) == 0
    full, _ = gemm_gpu(None, N, K, X, wbuf=wbuf)
    for rows in ([0], list(range(100, 132)), list(range(290, 300))):
        part, _ = gemm_gpu(None, N, K, X[rows], wbuf=wbuf)
        assert np.array_equal(part.view(np.uint32), full[rows].view(np.uint32)), rows
    ref = O.mul_mat_q4_0(Wq, K, X[:4])
    assert np.all(np.abs(full[:4] - ref) <= ATOL + RTOL * np.abs(ref))


def test_prompt_gate_up_swiglu_epilogue():
    """Prompt rows of an interleaved gate|up matrix with the SwiGLU + Q8_0 as the matmul's epilogue
    (snk_q4_gemm_swiglu): the fp32 rows and the down projection's operand are bit for bit the matmul with its SwiGLU
    output (snk_q4_gemm, epilogue 2) and the activation quantizer over those rows (snk_quant_act); below 256 rows the
    call declines (1) and launches nothing."""
    r = np.random.default_rng(12)
    F, K, M = 3072, 2560, 300
    N = 2 * F
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    L = S.lib()
    st = U.stream()
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), st) == 0
    Y, xa = gemm_gpu(None, N, K, X, epi=2, wbuf=wbuf)  # silu(gate) * up through the split-free launch and reduction
    dxa = U.dev(xa)
    h = U.dev(np.zeros((M, F), np.float32))
    xo = U.dev(np.zeros(L.snk_xa_bytes(M, F), np.uint8))
    assert L.snk_q4_gemm_swiglu(U.ptr(wbuf), U.ptr(dxa), M, N, K, U.ptr(h), U.ptr(xo), st) == 0
    gh = U.host(h, np.float32)[:M * F].reshape(M, F)
    assert np.array_equal(gh.view(np.uint32), Y.view(np.uint32))
    ref_xo = U.dev(np.zeros(L.snk_xa_bytes(M, F), np.uint8))
    assert L.snk_quant_act(U.ptr(U.dev(Y)), M, F, F, None, 0.0, U.ptr(ref_xo), st) == 0
    assert np.array_equal(U.host(xo, np.uint8), U.host(ref_xo, np.uint8))
    assert L.snk_q4_gemm_swiglu(U.ptr(wbuf), U.ptr(dxa), 200, N, K, U.ptr(h), U.ptr(xo), st) == 1


@pytest.fixture(scope="module")
def lm_head():
    """The Qwen3-4B LM head's shape (configs[2..4]: V = 151,936 rows of K = 2560), seeded N(0, 0.02) weights quantized
    with ggml's reference quantizer, and 300 activation rows with the full-width product of all of them."""
    r = np.random.default_rng(8)
    N, K = 151936, 2560
    Wq = O.quantize_q4_0(r.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    X = r.normal(0, 1, (300, K)).astype(np.float32)
    L = S.lib()
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), U.stream()) == 0
    full, _ = gemm_gpu(None, N, K, X, wbuf=wbuf)
    return Wq, X, wbuf, full


@pytest.mark.parametrize("M", [1, 8, 32, 300])
def test_lm_head_width_matmul(lm_head, M):
    """The LM head's launches (two stripes a wavefront, no k-split: the kernel instances every decode, draft and MoE
    step's output stage runs, sn_encode.inc.h:304-317) against the oracle at 1, 8 (drafts), 32 (decode) and 300 rows,
    and each row bit for bit equal to the same row of the 300-row product."""
    Wq, X, wbuf, full = lm_head
    N, K = 151936, 2560
    assert S.q4_plan(N, K) == (2, 1)
    Y, _ = gemm_gpu(None, N, K, X[:M], wbuf=wbuf)
    ref = O.mul_mat_q4_0(Wq, K, X[:M])
    err = np.abs(Y - ref)
    print(f"LM head M={M}: max abs err {err.max():.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref))
    assert np.array_equal(Y.view(np.uint32), full[:M].view(np.uint32))
    if M > 1:  # rows from the middle of the batch, alone
        part, _ = gemm_gpu(None, N, K, X[M // 2:M], wbuf=wbuf)
        assert np.array_equal(part.view(np.uint32), full[M // 2:M].view(np.uint32))


@pytest.mark.parametrize("N,K", [(6144, 2560), (19456, 2560), (2560, 9728), (200, 640), (98304, 2560)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_equals_mfma_bitwise(M, N, K):
    """The per-column integer-dot GEMV for few rows (snk_q4_gemm_plan_* with mt 0: 8 v_dot4 a block and row, then the
    MFMA kernels' fma(isum, dw * dx, acc) in the same order) against the default MFMA launch of the same plan: the
    same slice sums, bit for bit. Shapes: q|k|v (4-group slices), gate|up and down (8-group slices, a short last one),
    200 x 640 (a partial stripe set, a one-group last slice padded with a zero-scale group) and a wide matrix with the
    LM head's plan (one 20-group slice)."""
    L = S.lib()
    st = U.stream()
    r = np.random.default_rng(100 + M + N)
    nb = min(N, 4096)
    Wq = O.quantize_q4_0(r.normal(0, 0.02, (nb, K)).astype(np.float32))
    Wq = np.ascontiguousarray(np.tile(Wq, ((N + nb - 1) // nb, 1))[:N])
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), st) == 0
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    X[0, :32] = 0.0  # an all-zero block
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(U.dev(X)), M, K, K, None, 0.0, U.ptr(xa), st) == 0
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    out = []
    for mt in (1, 0):
        y, ws = U.empty(M * N * 4), U.empty(wsb)
        assert L.snk_q4_gemm_plan_sums(U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y), U.ptr(ws), wsb, mt, mt, 0, st) == 0
        out.append(U.host(y, np.float32)[:M * N].reshape(M, N))
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    assert np.count_nonzero(out[1]) > M * N // 2


@pytest.mark.parametrize("N,K", [(19456, 2560), (2560, 9728), (98304, 2560)])
def test_subnormal_scales_gemv_equals_mfma(N, K):
    """Blocks whose fp16 scales are subnormal: weight rows scaled by 1e-4 (d about 1e-6) and activation rows scaled by
    1e-5 (dx about 2e-7), so every kind of product dw * dx (normal x subnormal, subnormal x subnormal) occurs. The MFMA
    kernels form those products on the matrix core (an fp16 MFMA of the two scales, exact only if it keeps subnormal
    inputs); the GEMV forms them on the VALU in fp32. Both must give the same slice sums, bit for bit, and the tiny
    rows must not be flushed to zero. Shapes: gate|up and down (streaming kernel) and the LM head's plan (ring)."""
    L = S.lib()
    st = U.stream()
    M = 4
    r = np.random.default_rng(500 + N)
    nb = min(N, 4096)
    W = r.normal(0, 0.02, (nb, K)).astype(np.float32)
    W[::3] *= np.float32(1e-4)
    Wq = O.quantize_q4_0(W)
    d = Wq.reshape(nb, K // 32, 18)[:, :, :2].copy().view(np.float16)
    assert np.any((d != 0) & (np.abs(d.astype(np.float32)) < 6.1e-5))  # subnormal weight scales are present
    Wq = np.ascontiguousarray(np.tile(Wq, ((N + nb - 1) // nb, 1))[:N])
    wbuf = U.empty(L.snk_q4_stripes_bytes(N, K))
    assert L.snk_q4_repack(U.ptr(U.dev(Wq)), N, K, U.ptr(wbuf), st) == 0
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    X[1::2] *= np.float32(1e-5)
    xd = O.quantize_q8_0(X).reshape(M, K // 32, 34)[:, :, :2].copy().view(np.float16)
    assert np.all(np.abs(xd[1::2].astype(np.float32)) < 6.1e-5)  # the tiny rows' scales are subnormal
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(U.dev(X)), M, K, K, None, 0.0, U.ptr(xa), st) == 0
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    out = []
    for mt in (1, 0):
        y, ws = U.empty(M * N * 4), U.empty(wsb)
        assert L.snk_q4_gemm_plan_sums(U.ptr(wbuf), U.ptr(xa), M, N, K, U.ptr(y), U.ptr(ws), wsb, mt, mt, 0, st) == 0
        out.append(U.host(y, np.float32)[:M * N].reshape(M, N))
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    assert np.count_nonzero(out[0][1]) > N // 2 and np.count_nonzero(out[0][3]) > N // 2
    ref = O.mul_mat_q4_0(Wq[:nb], K, X)
    tiny = np.abs(ref[1]).max()
    assert 0 < tiny < 1e-3 * np.abs(ref[0]).max()
    assert np.all(np.abs(out[0][1, :nb] - ref[1]) <= 1e-3 * np.abs(ref[1]) + 1e-6 * tiny)
