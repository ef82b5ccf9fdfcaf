"""Row kernels of the step on the GPU against the oracle: the RMSNorm fused in front of the Q8_0 activation quantizer,
and per-head QK-norm + NEOX RoPE + the fp16 K/V cache write, through the C ABI (include/sn_kernels.h)."""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu


def setup_module(module):
    U.torch().cuda.init()


def test_rmsnorm_then_q8_0():
    r = np.random.default_rng(20)
    M, K, eps = 24, 2560, 1e-6
    X = (r.normal(0, 1, (M, K)) * r.uniform(0.01, 5, (M, 1))).astype(np.float32)
    w = r.normal(1, 0.1, K).astype(np.float32)
    L = S.lib()
    x, dw = U.dev(X), U.dev(w)
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(x), M, K, K, U.ptr(dw), eps, U.ptr(xa), U.stream()) == 0
    got = U.xa_values(U.host(xa, np.uint8), M, K)
    xn = O.rmsnorm(X, w, eps)
    want = O.dequantize_q8_0(O.quantize_q8_0(xn), K)
    # the norm's sum of squares runs in another order, so a value may sit one rounding step to the other side of a
    # quantization boundary; every value is within one Q8_0 step and nearly all are identical
    step = np.repeat(np.abs(O.quantize_q8_0(xn).reshape(M, -1, 34)[:, :, :2].copy().view(np.float16)[..., 0]
                            .astype(np.float32)), 32, axis=1)
    assert np.all(np.abs(got - want) <= step * 1.001 + 1e-30)
    assert np.mean(got == want) > 0.999


def _qk_rope_run(qkv, seq, pos, pt, page, qw, kw, eps, ts, H, KVH, D=128):
    """snk_qk_rope over the rows of qkv: (q rows after the kernel, k pool, v pool) as host arrays."""
    L = S.lib()
    R = qkv.shape[0]
    npg = pt.size
    d_qkv = U.dev(qkv)
    kp = U.empty(npg * KVH * page * D * 2)
    vp = U.empty(npg * KVH * page * D * 2)
    assert L.snk_qk_rope(U.ptr(d_qkv), (H + 2 * KVH) * D, R, H, KVH, U.ptr(U.dev(qw)), U.ptr(U.dev(kw)), eps, float(ts),
                         U.ptr(U.dev(seq)), U.ptr(U.dev(pos)), U.ptr(U.dev(pt)), pt.shape[1], page, U.ptr(kp),
                         U.ptr(vp), U.stream()) == 0
    q_out = U.host(d_qkv, np.float32)[:qkv.size].reshape(qkv.shape)
    kpool = U.k_cells(U.host(kp, np.uint16)[:npg * KVH * page * D].reshape(npg, KVH, page, D))
    vpool = U.host(vp, np.uint16)[:npg * KVH * page * D].reshape(npg, KVH, page, D)
    return q_out, kpool, vpool


# 7 rows take the wavefront-per-head launch, 200 rows (at least 128) the workgroup-per-row launch
@pytest.mark.parametrize("page,R", [(32, 7), (64, 7), (32, 200)])
def test_qk_norm_rope_and_cache_write(page, R):
    r = np.random.default_rng(21)
    H, KVH, D, eps, base = 32, 8, 128, 1e-6, 1e6
    if R == 7:
        seq = np.array([0, 0, 1, 2, 2, 2, 3], np.int32)
        pos = np.array([0, 1, 5, 4095, 100, 33, 2048], np.int32)
    else:  # distinct (sequence, position) cells, positions spread over [0, 4096)
        cells = r.choice(4 * 4096, R, replace=False)
        seq, pos = (cells // 4096).astype(np.int32), (cells % 4096).astype(np.int32)
    maxp = 4096 // page
    npg = 4 * maxp
    pt = r.permutation(npg).astype(np.int32).reshape(4, maxp)
    qkv = r.normal(0, 2, (R, (H + 2 * KVH) * D)).astype(np.float32)
    qw = r.normal(1, 0.1, D).astype(np.float32)
    kw = r.normal(1, 0.1, D).astype(np.float32)
    ts = np.float32(np.power(np.float32(base), np.float32(-2.0 / D)))
    q_out, kpool, vpool = _qk_rope_run(qkv, seq, pos, pt, page, qw, kw, eps, ts, H, KVH)
    for i in range(R):
        cs = O.rope_cache(int(pos[i]), ts, D)
        pg, off = pt[seq[i], pos[i] // page], pos[i] % page
        for h in range(H):
            want = O.qk_norm_rope(qkv[i, h * D:(h + 1) * D], qw, eps, cs)
            assert np.allclose(q_out[i, h * D:(h + 1) * D], want, rtol=2e-5, atol=2e-6), (i, h)
        for h in range(KVH):
            k = O.qk_norm_rope(qkv[i, (H + h) * D:(H + h + 1) * D], kw, eps, cs)
            got = kpool[pg, h, off].view(np.float16).astype(np.float32)
            assert np.allclose(got, k.astype(np.float16).astype(np.float32), rtol=2e-3, atol=1e-3), (i, h)
            v = qkv[i, (H + KVH + h) * D:(H + KVH + h + 1) * D]
            assert np.array_equal(vpool[pg, h, off], v.astype(np.float16).view(np.uint16)), (i, h)


def test_qk_rope_launch_shapes_agree_bitwise():
    """A row's q, k and v come out with the same bits from the workgroup-per-row launch (a 160-row step) and from the
    wavefront-per-head launch (the same rows in steps of 40), so a prompt's rows match the rows decode makes."""
    r = np.random.default_rng(23)
    H, KVH, D, eps, page = 32, 8, 128, 1e-6, 32
    R = 160
    cells = r.choice(4 * 4096, R, replace=False)
    seq, pos = (cells // 4096).astype(np.int32), (cells % 4096).astype(np.int32)
    pt = r.permutation(4 * 128).astype(np.int32).reshape(4, 128)
    qkv = r.normal(0, 3, (R, (H + 2 * KVH) * D)).astype(np.float32)
    qw = r.normal(1, 0.1, D).astype(np.float32)
    kw = r.normal(1, 0.1, D).astype(np.float32)
    ts = np.float32(np.power(np.float32(1e6), np.float32(-2.0 / D)))
    q_all, k_all, v_all = _qk_rope_run(qkv, seq, pos, pt, page, qw, kw, eps, ts, H, KVH)
    for a in range(0, R, 40):
        sl = slice(a, a + 40)
        q_part, k_part, v_part = _qk_rope_run(qkv[sl].copy(), seq[sl], pos[sl], pt, page, qw, kw, eps, ts, H, KVH)
        assert np.array_equal(q_part.view(np.uint32), q_all[sl].view(np.uint32))
        for i in range(a, a + 40):
            pg, off = pt[seq[i], pos[i] // page], pos[i] % page
            assert np.array_equal(k_part[pg, :, off], k_all[pg, :, off]), i
            assert np.array_equal(v_part[pg, :, off], v_all[pg, :, off]), i
