"""Pins the CPU oracle before anything is checked against it (CPU only).

Each oracle function is checked against something that does not restate its own formula: closed forms computed a
different way, invariants, brute force, the reference's golden fixture, or numpy's own IEEE routines. The reference
holds no numeric golden vectors for this path (its real-model goldens need GGUFs that are not here), so these are the
pins; tests/golden/ holds fixtures generated from the pinned oracle for regression.
"""
import itertools
import math

import numpy as np
import pytest

from oracle import oracle as O


def rng(seed):
    return np.random.default_rng(seed)


# ---- fp16 -------------------------------------------------------------------------------------------------------------
def test_f16_conversion_matches_numpy_rne():
    r = rng(1)
    x = np.concatenate([r.normal(0, 1, 2000), r.normal(0, 1e-5, 500), r.normal(0, 3e4, 200),
                        [0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 2 ** -24, 2 ** -25, 3 * 2 ** -26, np.inf, -np.inf]]
                       ).astype(np.float32)
    got = O.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- Q4_0 ---------------------------------------------------------------------------------------------------------------
def _block(d_bits: int, qs: np.ndarray) -> np.ndarray:
    return np.concatenate([np.array([d_bits & 255, d_bits >> 8], np.uint8), qs.astype(np.uint8)])


@pytest.mark.parametrize("d", [0.0, 1.0, -1.0, 0.0123, -3.5, 6.1e-5, 5.96e-8, -5.96e-8, 65504.0])
def test_dequant_q4_0_every_nibble(d):
    # every (low, high) nibble pair: element j = low nibble of byte j, element j+16 = high nibble; value d*(q-8)
    dh = np.float16(d)
    vals = np.arange(16, dtype=np.uint8)
    qs = (vals | (vals[::-1] << 4)).astype(np.uint8)  # byte j: low j, high 15-j
    blk = _block(int(dh.view(np.uint16)), qs)
    got = O.dequantize_q4_0(blk, 32)[0]
    df = np.float64(dh)
    want = np.concatenate([(np.arange(16) - 8) * df, (np.arange(15, -1, -1) - 8) * df]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quantize_q4_0_invariants():
    r = rng(2)
    x = r.normal(0, 0.02, (64, 256)).astype(np.float32)
    x[3, 5] = 0.5  # a block whose extreme is positive
    x[4, 40:72] = 0.0  # an all-zero block
    q = O.quantize_q4_0(x)
    blocks = q.reshape(-1, 18)
    xb = x.reshape(-1, 32)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    nib = np.concatenate([blocks[:, 2:] & 15, blocks[:, 2:] >> 4], axis=1).astype(np.int64)
    assert nib.min() >= 0 and nib.max() <= 15
    for i in range(len(xb)):
        xi = xb[i].astype(np.float64)
        k = int(np.argmax(np.abs(xi)))  # the first of the largest magnitude
        if xi[k] == 0.0:
            assert d[i] == 0.0 and np.all(nib[i] == 8)
            continue
        # the extreme element is exactly the -8 level: d = max / -8
        assert np.float16(np.float32(xi[k]) / np.float32(-8.0)) == np.float16(d[i])
        assert nib[i, k] == 0
        # every element sits on the level nearest to it under the fp32 scale (clamped at 15), i.e. within half a step
        d32 = np.float64(np.float32(xi[k]) / np.float32(-8.0))
        t = xi / d32 + 8.0
        assert np.all(np.abs(np.minimum(t, 15.0) - nib[i]) <= 0.5 + 1e-6)


def test_quantize_q4_0_first_of_equal_magnitudes():
    x = np.zeros((1, 32), np.float32)
    x[0, 3] = -0.25
    x[0, 9] = 0.25  # same magnitude, later: the earlier (negative) one sets the sign of d
    q = O.quantize_q4_0(x).reshape(18)
    d = q[:2].copy().view(np.float16)[0]
    assert float(d) == 0.25 / 8
    nib = np.concatenate([q[2:] & 15, q[2:] >> 4])
    assert nib[3] == 0 and nib[9] == 15  # +0.25 / (0.25/8) + 8.5 = 16.5 -> clamped to 15


def test_quantize_q4_0_half_steps_round_up():
    """ggml's quantize_row_q4_0_ref truncates x * id + 8.5 toward zero, so a value exactly half-way between two levels
    takes the upper one (7.5 -> 8 would be 8 under round-half-even: these cases tell the rules apart), clamped at 15."""
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = -8.0  # the extreme element: d = -8 / -8 = 1, id = 1 (exact)
    vals = [0.5, 2.5, -1.5, 4.5, -3.5, 6.5, -5.5, 1.5, -0.5, 7.5, -7.5, 3.0, -6.0]
    x[0, 1:1 + len(vals)] = vals
    q = O.quantize_q4_0(x).reshape(18)
    assert float(q[:2].copy().view(np.float16)[0]) == 1.0
    nib = np.concatenate([q[2:] & 15, q[2:] >> 4]).astype(np.int64)
    want = [min(15, int(np.floor(v + 8.5))) for v in vals]
    assert want[:3] == [9, 11, 7]  # (half-even would give 8, 10, 6)
    assert list(nib[1:1 + len(vals)]) == want, (list(nib[1:1 + len(vals)]), want)
    assert nib[0] == 0 and np.all(nib[1 + len(vals):] == 8)


# ---- Q8_0 and the integer dot -------------------------------------------------------------------------------------------
def test_quantize_q8_0_invariants():
    r = rng(3)
    x = r.normal(0, 1, (8, 256)).astype(np.float32)
    x[1, :32] = 0.0
    q = O.quantize_q8_0(x).reshape(-1, 34)
    xb = x.reshape(-1, 32).astype(np.float64)
    for i in range(len(q)):
        d = float(q[i, :2].copy().view(np.float16)[0])
        qi = q[i, 2:].view(np.int8).astype(np.int64)
        amax = np.abs(xb[i]).max()
        if amax == 0:
            assert d == 0 and np.all(qi == 0)
            continue
        assert np.float16(np.float32(amax) / np.float32(127)) == np.float16(d)
        assert np.abs(qi).max() == 127 and qi[np.argmax(np.abs(xb[i]))] == np.sign(xb[i][np.argmax(np.abs(xb[i]))]) * 127
        # nearest level of x * 127 / amax
        assert np.all(np.abs(xb[i] * 127.0 / amax - qi) <= 0.5 + 1e-5)


def test_quantize_q8_0_rounds_half_to_even():
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1] = 2.5
    x[0, 2] = 3.5
    x[0, 3] = -2.5
    q = O.quantize_q8_0(x).reshape(34)[2:].view(np.int8)
    assert list(q[:4]) == [127, 2, 4, -2]


def test_vec_dot_is_integer_block_sum():
    r = rng(4)
    K = 512
    w = O.quantize_q4_0(r.normal(0, 0.02, (1, K)).astype(np.float32)).reshape(-1, 18)
    x = O.quantize_q8_0(r.normal(0, 1, (1, K)).astype(np.float32)).reshape(-1, 34)
    tot = 0.0
    for b in range(K // 32):
        q4 = np.concatenate([w[b, 2:] & 15, w[b, 2:] >> 4]).astype(np.int64) - 8
        q8 = x[b, 2:].view(np.int8).astype(np.int64)
        tot += int((q4 * q8).sum()) * float(w[b, :2].copy().view(np.float16)[0]) * float(x[b, :2].copy().view(np.float16)[0])
    got = O.lib().or_vec_dot_q4_0_q8_0(K, O._p(w), O._p(x))
    assert abs(got - tot) <= 1e-5 * max(1.0, abs(tot))


def test_mul_mat_vs_f64():
    r = rng(5)
    N, K, M = 96, 512, 8
    W = O.quantize_q4_0(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    Y = O.mul_mat_q4_0(W, K, X)
    # against fp64 over the Q8_0-dequantized activations: only fp32 rounding differs
    Xq = O.dequantize_q8_0(O.quantize_q8_0(X), K)
    Yq = O.mul_mat_q4_0_f64(W, K, Xq)
    assert np.max(np.abs(Y - Yq)) <= 1e-5 * np.max(np.abs(Yq))
    # against fp64 over the fp32 activations: the Q8_0 activation error only (~0.5% rms for N(0,1) blocks)
    Yf = O.mul_mat_q4_0_f64(W, K, X)
    rel_rms = np.sqrt(np.mean((Y - Yf) ** 2) / np.mean(Yf ** 2))
    assert rel_rms < 1e-2
    # and the fp64 product itself is the dequantized matrix times X
    Wd = O.dequantize_q4_0(W, K).astype(np.float64)
    assert np.allclose(Yf, X.astype(np.float64) @ Wd.T, rtol=1e-12, atol=1e-12)


# ---- Q8_0 weights (block_q8_0: kernels.metal:9; ggml quantize_row_q8_0_ref, dequantize_row_q8_0, vec_dot_q8_0_q8_0) -----
def test_quantize_q8_0_ref_invariants():
    r = rng(21)
    w = r.normal(0, 0.02, (6, 256)).astype(np.float32)
    w[2, :32] = 0.0
    q = O.quantize_q8_0_ref(w).reshape(-1, 34)
    wb = w.reshape(-1, 32).astype(np.float64)
    for i in range(len(q)):
        d = float(q[i, :2].copy().view(np.float16)[0])
        qi = q[i, 2:].view(np.int8).astype(np.int64)
        amax = np.abs(wb[i]).max()
        if amax == 0:
            assert d == 0 and np.all(qi == 0)
            continue
        d32 = np.float32(amax) / np.float32(127)
        assert np.float16(d32) == np.float16(d)
        j = np.argmax(np.abs(wb[i]))
        assert qi[j] == np.sign(wb[i][j]) * 127 and np.abs(qi).max() == 127
        # q is the nearest integer to x / d (d in fp32 before its fp16 rounding), so d * q is within d / 2 + the fp16
        # rounding of d times 127
        assert np.all(np.abs(wb[i] / float(d32) - qi) <= 0.5 + 1e-5)
    # dequantize_row_q8_0 is d * q exactly
    deq = O.dequantize_q8_0(q.reshape(6, -1), 256).reshape(-1, 32)
    want = q[:, 2:].view(np.int8).astype(np.float32) * q[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(deq, want)


def test_quantize_q8_0_ref_rounds_half_away_from_zero():
    # d = 127 / 127 = 1 exactly, id = 1: x = k + 0.5 lands on a tie; the weights' quantizer (roundf) goes away from zero,
    # where the activations' x86 quantizer (round-half-even) goes to the even neighbour
    x = np.zeros((1, 32), np.float32)
    x[0, :5] = [127.0, 2.5, 3.5, -2.5, -0.5]
    qw = O.quantize_q8_0_ref(x).reshape(34)[2:].view(np.int8)
    qa = O.quantize_q8_0(x).reshape(34)[2:].view(np.int8)
    assert list(qw[:5]) == [127, 3, 4, -3, -1]
    assert list(qa[:5]) == [127, 2, 4, -2, 0]


def test_vec_dot_q8_0_is_integer_block_sum_bitwise():
    r = rng(22)
    K = 1024
    w = O.quantize_q8_0_ref(r.normal(0, 0.02, (1, K)).astype(np.float32)).reshape(-1, 34)
    x = O.quantize_q8_0(r.normal(0, 1, (1, K)).astype(np.float32)).reshape(-1, 34)
    # ggml's generic loop restated in float32: sumf += float(sumi) * (dw * dx), block by block
    sumf = np.float32(0.0)
    for b in range(K // 32):
        sumi = int((w[b, 2:].view(np.int8).astype(np.int64) * x[b, 2:].view(np.int8).astype(np.int64)).sum())
        dw = np.float32(w[b, :2].copy().view(np.float16)[0])
        dx = np.float32(x[b, :2].copy().view(np.float16)[0])
        sumf = np.float32(sumf + np.float32(sumi) * np.float32(dw * dx))
    got = np.float32(O.lib().or_vec_dot_q8_0_q8_0(K, O._p(w), O._p(x)))
    assert got.view(np.uint32) == sumf.view(np.uint32)


def test_mul_mat_q8_0_vs_f64():
    r = rng(23)
    N, K, M = 80, 512, 6
    W = O.quantize_q8_0_ref(r.normal(0, 0.02, (N, K)).astype(np.float32))
    X = r.normal(0, 1, (M, K)).astype(np.float32)
    Y = O.mul_mat_q8_0(W, K, X)
    Wd = O.dequantize_q8_0(W, K).astype(np.float64)
    Xq = O.dequantize_q8_0(O.quantize_q8_0(X), K).astype(np.float64)
    assert np.max(np.abs(Y - Xq @ Wd.T)) <= 1e-5 * np.max(np.abs(Y))


# ---- row math -----------------------------------------------------------------------------------------------------------
def test_rmsnorm_closed_form():
    r = rng(6)
    x = r.normal(0, 3, (4, 2560)).astype(np.float32)
    w = r.normal(1, 0.1, 2560).astype(np.float32)
    y = O.rmsnorm(x, w, 1e-6)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6) * w
    assert np.allclose(y, ref, rtol=2e-6, atol=1e-7)


def test_rope_invariants():
    D, base = 128, 1e6
    s = np.float32(base) ** np.float32(-2.0 / D)
    r = rng(7)
    x = r.normal(0, 1, D).astype(np.float32)
    w = np.ones(D, np.float32)
    # position 0 is the identity (after the norm)
    cs0 = O.rope_cache(0, s, D)
    assert np.array_equal(cs0[0::2], np.ones(D // 2, np.float32)) and np.array_equal(cs0[1::2], np.zeros(D // 2, np.float32))
    for p in (1, 17, 1000, 4095):
        cs = O.rope_cache(p, s, D)
        ang = np.arctan2(cs[1::2], cs[0::2]).astype(np.float64)
        want = np.mod(p * base ** (-2.0 * np.arange(D // 2) / D) + np.pi, 2 * np.pi) - np.pi
        diff = np.abs(np.mod(ang - want + np.pi, 2 * np.pi) - np.pi)
        assert diff.max() < 2e-3 * max(1, p / 1000)  # fp32 iterated theta
        y = O.qk_norm_rope(x, w, 1e-6, cs)
        xn = O.rmsnorm(x[None], w, 1e-6)[0]
        # each (i, i + 64) pair keeps its length
        assert np.allclose(y[:64] ** 2 + y[64:] ** 2, xn[:64] ** 2 + xn[64:] ** 2, rtol=1e-5, atol=1e-6)
    # relative position: <rope(q, p1), rope(k, p2)> depends on p1 - p2 only
    q = r.normal(0, 1, D).astype(np.float32)
    k = r.normal(0, 1, D).astype(np.float32)
    dots = []
    for p in (10, 200, 3000):
        dots.append(float(np.dot(O.qk_norm_rope(q, w, 1e-6, O.rope_cache(p + 5, s, D)),
                                 O.qk_norm_rope(k, w, 1e-6, O.rope_cache(p, s, D)))))
    assert max(dots) - min(dots) < 5e-3


def test_argmax_ties_and_bans():
    x = np.array([1.0, 3.0, 3.0, -1.0, 3.0], np.float32)
    assert O.argmax(x) == 1
    assert O.argmax(x, ban=[1]) == 2
    assert O.argmax(x, ban=[1, 2, 4]) == 0
    r = rng(8)
    for _ in range(50):
        y = r.integers(-3, 3, 1000).astype(np.float32)
        assert O.argmax(y) == int(np.argmax(y))  # numpy: the first occurrence of the maximum
    i1, v1, i2, v2, lse = O.top2(np.array([0.5, 2.0, 2.0, 1.0], np.float32))
    assert (i1, i2) == (1, 2) and v1 == v2 == 2.0
    assert abs(lse - math.log(math.exp(0.5) + 2 * math.exp(2.0) + math.exp(1.0))) < 1e-5
    # a row with no finite score: no pair, log-sum-exp -inf (kernels.metal:436), the first unbanned id chosen
    i1, v1, i2, v2, lse = O.top2(np.full(7, -np.inf, np.float32))
    assert (i1, i2) == (0x7FFFFFFF, 0x7FFFFFFF) and v1 == v2 == lse == -np.inf
    assert O.argmax(np.full(7, -np.inf, np.float32), ban=[0, 1]) == 2
    # the log-sum-exp against scipy's, on a wide row
    from scipy.special import logsumexp
    y = (r.standard_normal(151936) * 5).astype(np.float32)
    assert abs(O.top2(y)[4] - logsumexp(y.astype(np.float64))) < 1e-5


# ---- paged attention ----------------------------------------------------------------------------------------------------
def _paged_case(seed, S=5, H=8, KVH=2, D=128, page=32, ctx_lo=1, ctx_hi=300, share=0):
    r = rng(seed)
    ctx = r.integers(ctx_lo, ctx_hi + 1, S)
    maxp = int(np.ceil(ctx.max() / page))
    n_pages = int(sum(np.ceil(ctx / page))) + 4
    perm = r.permutation(n_pages)
    pt = np.full((S, maxp), -1, np.int32)
    k = 0
    for s in range(S):
        for c in range(int(np.ceil(ctx[s] / page))):
            if share and s < share and c < 2 and s > 0:
                pt[s, c] = pt[0, c]  # a shared prefix of two pages
            else:
                pt[s, c] = perm[k]
                k += 1
    kpool = r.normal(0, 1, (n_pages, KVH, page, D)).astype(np.float16).view(np.uint16)
    vpool = r.normal(0, 1, (n_pages, KVH, page, D)).astype(np.float16).view(np.uint16)
    q = r.normal(0, 1, (S, H, D)).astype(np.float32)
    return q, np.arange(S, dtype=np.int32), (ctx - 1).astype(np.int32), kpool, vpool, pt, page


def test_paged_attention_vs_dense_brute_force():
    q, seq, pos, kp, vp, pt, page = _paged_case(9)
    S, H, D = q.shape
    KVH = kp.shape[1]
    scale = 1 / math.sqrt(D)
    out = O.paged_attn(q, seq, pos, KVH, kp, vp, page, pt, scale)
    K = kp.view(np.float16).astype(np.float64)
    V = vp.view(np.float16).astype(np.float64)
    for s in range(S):
        n = pos[s] + 1
        cells = [(pt[s, c // page], c % page) for c in range(n)]
        for h in range(H):
            kh = h // (H // KVH)
            Kd = np.stack([K[p, kh, o] for p, o in cells])
            Vd = np.stack([V[p, kh, o] for p, o in cells])
            sc = Kd @ q[s, h].astype(np.float64) * scale
            p = np.exp(sc - sc.max())
            ref = (p / p.sum()) @ Vd
            assert np.allclose(out[s, h], ref, rtol=1e-4, atol=2e-6)
    out64 = O.paged_attn(q, seq, pos, KVH, kp, vp, page, pt, scale, f64=True)
    assert np.allclose(out, out64, rtol=1e-4, atol=2e-6)


def test_paged_attention_chunked_equals_monolithic():
    q, seq, pos, kp, vp, pt, page = _paged_case(10, ctx_hi=900)
    scale = 1 / math.sqrt(128)
    a = O.paged_attn(q, seq, pos, kp.shape[1], kp, vp, page, pt, scale)
    for chunk in (32, 64, 256):
        b = O.paged_attn_chunked(q, seq, pos, kp.shape[1], kp, vp, page, pt, scale, chunk)
        assert np.allclose(a, b, rtol=1e-4, atol=1e-6)


def test_paged_attention_page_permutation_and_shared_prefix():
    q, seq, pos, kp, vp, pt, page = _paged_case(11, S=3, ctx_lo=100, ctx_hi=200, share=3)
    scale = 1 / math.sqrt(128)
    q[:] = q[0]  # same query everywhere
    pos[:] = pos[0]
    # sequences 1, 2 share sequence 0's first two pages; give them sequence 0's remaining pages' contents too
    for s in (1, 2):
        for c in range(2, pt.shape[1]):
            if pt[0, c] >= 0:
                kp[pt[s, c]] = kp[pt[0, c]]
                vp[pt[s, c]] = vp[pt[0, c]]
    out = O.paged_attn(q, seq, pos, kp.shape[1], kp, vp, page, pt, scale)
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[0], out[2])


# ---- MoE routing and acceptance -----------------------------------------------------------------------------------------
def test_moe_route_brute_force():
    r = rng(12)
    for trial in range(20):
        lg = r.normal(0, 1, 128).astype(np.float32)
        if trial % 5 == 0:
            lg[10] = lg[20] = lg.max() + 1  # a tie: the lower id first
        ids, w = O.moe_route(lg, 8)
        order = sorted(range(128), key=lambda i: (-float(lg[i]), i))[:8]
        assert list(ids) == order
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        sel = p[order]
        assert np.allclose(w, sel / max(sel.sum(), 6.103515625e-5), rtol=1e-5)
    # the floor: tiny probabilities are not blown up past their share
    lg = np.full(128, -100.0, np.float32)
    lg[0] = 0.0
    ids, w = O.moe_route(lg, 2)
    assert ids[0] == 0 and abs(w[0] - 1.0) < 1e-6


def test_accept_rule_brute_force():
    for k in range(0, 4):
        for d in itertools.product(range(2), repeat=k):
            for t in itertools.product(range(2), repeat=k + 1):
                a = O.accept(np.array(d, np.int32), np.array(t, np.int32))
                # take.rs:339-357: row i is taken while its draft is the target's token; then the target's next
                want = 0
                while want < k and d[want] == t[want]:
                    want += 1
                assert a == want


# ---- Q6_K / Q8_K (ggml k-quants) ------------------------------------------------------------------------------------
def pack_q6_K(q: np.ndarray, sc: np.ndarray, d: np.ndarray) -> np.ndarray:
    """block_q6_K bytes from explicit values: q [nb][256] in 0..63 (value q - 32), sc [nb][16] int8, d [nb] fp16. Element
    e: half h = e // 128, quarter c = (e % 128) // 32, l = e % 32; low 4 bits in ql[64h + 32(c & 1) + l] (low nibble
    for c < 2, high for c >= 2), high 2 bits at bit 2c of qh[32h + l]."""
    nb = q.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    for b in range(nb):
        ql = np.zeros(128, np.int64)
        qh = np.zeros(64, np.int64)
        for e in range(256):
            h, c, l = e // 128, (e % 128) // 32, e % 32
            v = int(q[b, e])
            i = 64 * h + 32 * (c & 1) + l
            ql[i] |= (v & 15) << (4 if c >= 2 else 0)
            qh[32 * h + l] |= (v >> 4) << (2 * c)
        out[b, :128] = ql
        out[b, 128:192] = qh
        out[b, 192:208] = sc[b].astype(np.int8).view(np.uint8)
        out[b, 208:210] = np.array([d[b]], np.float16).view(np.uint8)
    return out


def test_q6_K_dequant_closed_form():
    r = rng(60)
    nb = 3
    q = r.integers(0, 64, (nb, 256))
    q[0] = np.arange(256) % 64  # every value in every position class
    sc = r.integers(-128, 128, (nb, 16))
    sc[1, :2] = (-128, 127)
    d = np.array([0.0123, -3.5e-5, 6.1e-5], np.float16)  # normal, small negative, near the subnormal edge
    blocks = pack_q6_K(q, sc, d)
    got = O.dequantize_q6_K(blocks.reshape(-1), 256 * nb).reshape(nb, 256)
    want = (d.astype(np.float32)[:, None] * sc.astype(np.float32)[:, np.arange(256) // 16]) * (q - 32).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_quantize_q8_K_invariants():
    r = rng(61)
    x = (r.standard_normal((4, 512)) * 3).astype(np.float32)
    x[1, 7] = -9.0  # a negative extreme
    x[2, 300], x[2, 301] = 5.0, -5.0  # equal |x|: the first is the extreme
    x[3, 256:] = 0.0  # an all-zero block
    xq = O.quantize_q8_K(x).reshape(4, 2, 292)
    for m in range(4):
        for b in range(2):
            blk = xq[m, b]
            d = blk[:4].copy().view(np.float32)[0]
            qs = blk[4:260].copy().view(np.int8).astype(np.int64)
            bs = blk[260:292].copy().view(np.int16).astype(np.int64)
            xs = x[m, 256 * b:256 * (b + 1)]
            if not np.any(xs):
                assert d == 0 and not qs.any() and not bs.any()
                continue
            j = int(np.argmax(np.abs(xs)))  # numpy: the first of equal maxima
            assert qs[j] == -127  # iscale = -127 / max sends the extreme to -127
            assert np.all(qs >= -127) and np.all(qs <= 127)
            assert np.array_equal(bs, qs.reshape(16, 16).sum(1))
            assert abs(d * -127 - xs[j]) <= 1e-6 * abs(xs[j])
            assert np.all(np.abs(d * qs - xs) <= abs(d) * 0.5 + 1e-6 * abs(xs[j]))


def test_vec_dot_q6_K_is_the_integer_block_sum():
    r = rng(62)
    nb, K = 4, 1024
    q = r.integers(0, 64, (nb, 256))
    sc = r.integers(-128, 128, (nb, 16))
    d = (r.random(nb) * 1e-3 + 1e-4).astype(np.float16)
    w = pack_q6_K(q, sc, d).reshape(-1)
    x = r.standard_normal((1, K)).astype(np.float32)
    xq = O.quantize_q8_K(x).reshape(nb, 292)
    got = O.vec_dot_q6_K_q8_K(w, xq.reshape(-1), K)
    want = 0.0
    for b in range(nb):
        q8 = xq[b, 4:260].copy().view(np.int8).astype(np.int64)
        isum = int(np.sum(sc[b][np.arange(256) // 16] * (q[b] - 32) * q8))
        want += float(np.float32(np.float32(d[b]) * xq[b, :4].copy().view(np.float32)[0])) * isum
    assert abs(got - want) <= 1e-5 * max(1.0, abs(want))
    # and the f64 product of the dequantized operands (the same numbers)
    wd = O.dequantize_q6_K(w, K).astype(np.float64)
    xd = np.concatenate([xq[b, :4].copy().view(np.float32)[0] * xq[b, 4:260].copy().view(np.int8).astype(np.float64)
                         for b in range(nb)])
    assert abs(got - float(wd[0] @ xd)) <= 1e-5 * max(1.0, abs(want))
    Y = O.mul_mat_q6_K(w.reshape(1, -1), K, x)
    assert Y.shape == (1, 1) and Y[0, 0] == np.float32(got)
