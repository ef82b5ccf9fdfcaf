"""Qwen3-MoE layers on the GPU (moe_ffn, sn_layers.inc.h:129-144; moe_topk1 / moe_lists / qmm_grouped / moe_out,
kernels.metal:3419-3538) against the oracle's MoE step (softmax -> top-k with ties to the lower id -> renormalised
weights, Q4_0 expert matmuls with ggml's Q8_0 activations, the weighted sum in slot order): greedy tokens wherever the
oracle's top-2 gap exceeds the model's logit bound. A row's expert grouping depends on the other rows of the step (which
rows share an expert, where its tile falls); its logits must not: row invariance is checked bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

TINY_MOE = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=0, n_vocab=1000, n_expert=16, n_expert_used=4,
                n_ff_exp=128)
MODEL_ATOL = 3e-2


def setup_module(module):
    U.torch().cuda.init()


@pytest.fixture(scope="module")
def moe_model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "moe.gguf")
    S.write_model(path, S.model_cfg(**TINY_MOE), seed=31)
    return path


def test_moe_matches_oracle(moe_model):
    rng = np.random.default_rng(7)
    n_seq = 4
    lens = rng.integers(4, 12, n_seq)
    ref = O.Qwen3(GGUF(moe_model), n_seq=n_seq, ctx=64)
    stats = {"rows": 0, "checked": 0, "same": 0}
    with S.Engine(moe_model, slots=n_seq, ctx=64, max_rows=64) as eng:
        tok = rng.integers(0, TINY_MOE["n_vocab"], int(lens.sum())).astype(np.int32)
        seq = np.repeat(np.arange(n_seq, dtype=np.int32), lens)
        pos = np.concatenate([np.arange(n) for n in lens]).astype(np.int32)
        outs = (np.cumsum(lens) - 1).astype(np.int32)
        got = eng.step(tok, seq, pos, outs, n_write=0)
        want, lg, _ = ref.step(tok, seq, pos, outs)
        glg = eng.logits(np.arange(n_seq))
        np.testing.assert_allclose(glg, lg, rtol=0, atol=MODEL_ATOL)
        for step in range(4):
            for j in range(n_seq):
                i1, v1, i2, v2, _ = O.top2(lg[j])
                stats["rows"] += 1
                if v1 - v2 > 2 * MODEL_ATOL:
                    stats["checked"] += 1
                    assert got[j] == want[j], (step, j)
                stats["same"] += int(got[j] == want[j])
            # decode on from the oracle's tokens
            dpos = (lens + step).astype(np.int32)
            got = eng.step(want, np.arange(n_seq, dtype=np.int32), dpos, np.arange(n_seq, dtype=np.int32))
            want, lg, _ = ref.step(want, np.arange(n_seq, dtype=np.int32), dpos, np.arange(n_seq, dtype=np.int32))
            np.testing.assert_allclose(eng.logits(np.arange(n_seq)), lg, rtol=0, atol=MODEL_ATOL)
    print(f"moe end to end: {stats}")
    assert stats["checked"] >= 4


def test_moe_row_invariance(moe_model):
    """a row's logits are the same alone and in a batch whose rows share its experts differently"""
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, 1000, 9).astype(np.int32)
    others = rng.integers(0, 1000, (5, 9)).astype(np.int32)
    res = []
    for n_other in (0, 5):
        with S.Engine(moe_model, slots=6, ctx=64, max_rows=96) as eng:
            rows = [prompt] + [others[i] for i in range(n_other)]
            tok = np.concatenate(rows)
            seq = np.repeat(np.arange(len(rows), dtype=np.int32), 9)
            pos = np.tile(np.arange(9, dtype=np.int32), len(rows))
            t = eng.step(tok, seq, pos, np.array([8], np.int32), n_write=0)
            lg = eng.logits(np.array([0]))
            t2 = eng.step(t, np.zeros(1, np.int32), np.array([9], np.int32), np.zeros(1, np.int32))
            res.append((t, t2, lg, eng.logits(np.array([0]))))
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


# ---- the MoE kernels through the C ABI (include/sn_kernels.h) ---------------------------------------------------------
RTOL, ATOL = 1e-3, 2e-3  # per-op tolerance of the expert matmuls


def dptr(t, off=0):
    import ctypes as C
    return C.c_void_p(t.data_ptr() + off)


def grouping(ids, NE, k, P):
    """The expert-major tile layout a routing must give (moe_lists, kernels.metal:3468-3497), by counting."""
    flat = ids.reshape(-1)
    cnt = np.bincount(flat, minlength=NE)
    toff = np.concatenate([[0], np.cumsum((cnt + 15) // 16)])
    prow = np.empty(flat.size, np.int32)
    rsrc = np.full(P, -1, np.int32)
    fill = np.zeros(NE, np.int64)
    for u, x in enumerate(flat):
        p = toff[x] * 16 + fill[x]
        fill[x] += 1
        prow[u] = p
        rsrc[p] = u // k
    items = np.array([(x, i) for x in range(NE) for i in range(toff[x], toff[x + 1])], np.int32).reshape(-1, 2)
    return prow.reshape(ids.shape), rsrc, items, int(toff[NE])


def select_gpu(lg, k):
    L = S.lib()
    R, NE = lg.shape
    P = L.snk_moe_tile_rows(R, NE, k)
    ids, w, prow = U.empty(R * k * 4), U.empty(R * k * 4), U.empty(R * k * 4)
    rsrc, items, cnt = U.empty(P * 4), U.empty(P // 16 * 8), U.empty(4)
    assert L.snk_moe_select(U.ptr(U.dev(lg.astype(np.float32))), R, NE, k, U.ptr(ids), U.ptr(w), U.ptr(prow),
                            U.ptr(rsrc), U.ptr(items), U.ptr(cnt), U.stream()) == 0
    n = int(U.host(cnt, np.int32)[0])
    return (U.host(ids, np.int32)[:R * k].reshape(R, k), U.host(w, np.float32)[:R * k].reshape(R, k),
            U.host(prow, np.int32)[:R * k].reshape(R, k), U.host(rsrc, np.int32)[:P],
            U.host(items, np.int32)[:2 * n].reshape(n, 2), n, P, (rsrc, items, cnt))


def test_moe_graphs_and_chained_steps_are_bitwise_eager(moe_model):
    """MoE decode through HIP-graph replay and through sn_step's queued successor (chain) against eager, unchained
    steps of a second engine: the same tokens and logits bit for bit (the expert grouping and the weighted sum folded
    into the next layer's residual kernel run inside captured and queued steps alike)."""
    n, steps = 4, 6
    r = np.random.default_rng(17)
    prompts = [r.integers(0, TINY_MOE["n_vocab"], int(r.integers(5, 20))).astype(np.int32) for _ in range(n)]
    runs = []
    for graphs, chain in ((True, 1), (False, 0)):
        with S.Engine(moe_model, slots=n, ctx=128, max_rows=96) as eng:
            eng.graphs(graphs)
            tok = np.concatenate(prompts)
            seq = np.concatenate([np.full(len(p), s, np.int32) for s, p in enumerate(prompts)])
            pos = np.concatenate([np.arange(len(p), dtype=np.int32) for p in prompts])
            last = eng.step(tok, seq, pos, np.cumsum([len(p) for p in prompts]).astype(np.int32) - 1, n_write=0)
            p = np.array([len(x) for x in prompts], np.int32)
            trace = []
            for i in range(steps):
                last = eng.step(last, np.arange(n, dtype=np.int32), p, np.arange(n, dtype=np.int32),
                                chain=chain if i + 1 < steps else 0)
                trace.append((last.copy(), eng.logits(np.arange(n)).copy()))
                p += 1
            if chain:
                taken, _ = eng.chain_count()
                assert taken == steps - 1
            runs.append(trace)
    for (ta, la), (tb, lb) in zip(*runs):
        assert np.array_equal(ta, tb)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_moe_router_matches_f64_and_is_row_invariant():
    L = S.lib()
    r = np.random.default_rng(40)
    for R, E, NE in ((32, 2048, 128), (5, 256, 16), (37, 96, 10)):
        hn = r.standard_normal((R, E)).astype(np.float32)
        rw = (r.standard_normal((NE, E)) * 0.05).astype(np.float32)
        lg = U.empty(R * NE * 4)
        assert L.snk_moe_router(U.ptr(U.dev(hn)), R, E, U.ptr(U.dev(rw)), NE, U.ptr(lg), U.stream()) == 0
        got = U.host(lg, np.float32)[:R * NE].reshape(R, NE)
        want = hn.astype(np.float64) @ rw.astype(np.float64).T
        bound = 1e-5 * (np.abs(hn).astype(np.float64) @ np.abs(rw).astype(np.float64).T)
        assert np.all(np.abs(got - want) <= bound), np.abs(got - want).max()
        one = U.empty(NE * 4)  # the last row alone: the same bits
        assert L.snk_moe_router(U.ptr(U.dev(hn[-1:])), 1, E, U.ptr(U.dev(rw)), NE, U.ptr(one), U.stream()) == 0
        assert np.array_equal(U.host(one, np.float32)[:NE].view(np.uint32), got[-1].view(np.uint32))


@pytest.mark.parametrize("R,NE,k", [(32, 128, 8), (5, 16, 4), (100, 64, 8), (3, 8, 8), (40, 6, 2)])
def test_moe_select_matches_oracle(R, NE, k):
    r = np.random.default_rng(R * 1000 + NE)
    lg = (r.standard_normal((R, NE)) * 2).astype(np.float32)
    if NE >= 8:  # ties: equal logits pick the lower id
        lg[0, :] = 1.0
        lg[1 % R, 3:7] = 9.0
    ids, w, prow, rsrc, items, n, P, _ = select_gpu(lg, k)
    for i in range(R):
        oid, ow = O.moe_route(lg[i], k)
        assert np.array_equal(ids[i], oid), (i, ids[i], oid)
        np.testing.assert_allclose(w[i], ow, rtol=1e-5, atol=1e-7)
    wp, wr, wi, wn = grouping(ids, NE, k, P)
    assert n == wn and np.array_equal(prow, wp) and np.array_equal(rsrc, wr) and np.array_equal(items, wi)


@pytest.mark.parametrize("R,E,NE,k", [(32, 2048, 128, 8), (5, 256, 16, 4), (100, 96, 64, 8), (3, 64, 8, 8),
                                      (40, 32, 6, 2), (1, 2048, 128, 8)])
def test_moe_route_one_launch_equals_router_and_select(R, E, NE, k):
    """The one-launch routing (the row blocks' logits, each block routed by its last workgroup through its XCD's L2,
    the grouping by the last block) against snk_moe_router + snk_moe_select: logits, ids, weights and the tile layout
    bit for bit, with no row block's workgroups found on two XCDs."""
    L = S.lib()
    r = np.random.default_rng(R * 7 + NE)
    hn = r.standard_normal((R, E)).astype(np.float32)
    rw = (r.standard_normal((NE, E)) * 0.05).astype(np.float32)
    if NE >= 8:
        rw[3:7] = rw[3]  # ties among the logits
    dh, dr = U.dev(hn), U.dev(rw)
    lg = U.empty(R * NE * 4)
    assert L.snk_moe_router(U.ptr(dh), R, E, U.ptr(dr), NE, U.ptr(lg), U.stream()) == 0
    want = select_gpu(U.host(lg, np.float32)[:R * NE].reshape(R, NE), k)
    P = L.snk_moe_tile_rows(R, NE, k)
    for rep in range(3):  # (the counters return to zero: later launches alike)
        lg2 = U.empty(R * NE * 4)
        ids, w, prow = U.empty(R * k * 4), U.empty(R * k * 4), U.empty(R * k * 4)
        rsrc, items, cnt = U.empty(P * 4), U.empty(P // 16 * 8), U.empty(4)
        xerr = C.c_int(-1)
        assert L.snk_moe_route(U.ptr(dh), R, E, U.ptr(dr), NE, k, U.ptr(lg2), U.ptr(ids), U.ptr(w), U.ptr(prow),
                               U.ptr(rsrc), U.ptr(items), U.ptr(cnt), C.byref(xerr), U.stream()) == 0
        assert xerr.value == 0
        assert np.array_equal(U.host(lg2, np.uint32)[:R * NE], U.host(lg, np.uint32)[:R * NE])
        n = int(U.host(cnt, np.int32)[0])
        got = (U.host(ids, np.int32)[:R * k].reshape(R, k), U.host(w, np.float32)[:R * k].reshape(R, k),
               U.host(prow, np.int32)[:R * k].reshape(R, k), U.host(rsrc, np.int32)[:P],
               U.host(items, np.int32)[:2 * n].reshape(n, 2), n)
        for a, b in zip(got, want[:6]):
            a, b = np.asarray(a), np.asarray(b)
            assert a.shape == b.shape and np.array_equal(a.view(np.uint8) if a.ndim else a, b.view(np.uint8) if b.ndim else b)


def test_moe_select_rejects_bad_shapes():
    L = S.lib()
    b = U.empty(1 << 16)
    for R, NE, k in ((4, 300, 2), (4, 8, 9), (4, 4, 5), (600, 8, 8)):
        assert L.snk_moe_select(U.ptr(b), R, NE, k, U.ptr(b), U.ptr(b), U.ptr(b), U.ptr(b), U.ptr(b), U.ptr(b),
                                U.stream()) == -1


@pytest.mark.parametrize("wt", [2, 8])
def test_grouped_expert_matmul_matches_oracle(wt):
    """Every real row of every tile against the oracle's matmul of its expert; padding rows are left as they were."""
    L = S.lib()
    r = np.random.default_rng(50 + wt)
    NE, k, R, N, K = 6, 2, 20, 160, 384
    lg = r.standard_normal((R, NE)).astype(np.float32)
    lg[:, 2] += 10.0  # expert 2 in every row: two tiles
    ids, w, prow, rsrc, items, n, P, (d_rsrc, d_items, d_cnt) = select_gpu(lg, k)
    assert (ids == 2).sum() == R and (items[:, 0] == 2).sum() == 2
    hn = r.standard_normal((R, K)).astype(np.float32)
    Ws = [(r.standard_normal((N, K)) * 0.1).astype(np.float32) for _ in range(NE)]
    if wt == 2:
        Wq = [O.quantize_q4_0(W) for W in Ws]
        stride, repack, mm = L.snk_q4_stripes_bytes(N, K), L.snk_q4_repack, O.mul_mat_q4_0
    else:
        Wq = [O.quantize_q8_0_ref(W) for W in Ws]
        stride, repack, mm = L.snk_q8_tiles_bytes(N, K), L.snk_q8_repack, O.mul_mat_q8_0
    wbuf = U.empty(NE * stride)
    for x in range(NE):
        assert repack(U.ptr(U.dev(Wq[x])), N, K, dptr(wbuf, x * stride), U.stream()) == 0
    X = np.zeros((P, K), np.float32)
    X[rsrc >= 0] = hn[rsrc[rsrc >= 0]]
    xa = U.empty(L.snk_xa_bytes(P, K))
    assert L.snk_quant_act(U.ptr(U.dev(X)), P, K, K, None, 0.0, U.ptr(xa), U.stream()) == 0
    part = U.dev(np.full((P, N), np.nan, np.float32))
    assert L.snk_gemm_grouped(wt, U.ptr(wbuf), stride, U.ptr(d_items), U.ptr(d_cnt), P // 16, U.ptr(xa), P, N, K,
                              U.ptr(part), P * N * 4, U.ptr(d_rsrc), U.stream()) == 0
    got = U.host(part, np.float32)[:P * N].reshape(P, N)
    assert np.all(np.isnan(got[rsrc < 0]))
    for x in range(NE):
        rows = [p for p in range(P) if rsrc[p] >= 0 and any(items[i, 0] == x and items[i, 1] == p // 16 for i in range(n))]
        if not rows:
            continue
        want = mm(Wq[x], K, hn[rsrc[rows]])
        np.testing.assert_allclose(got[rows], want, rtol=RTOL, atol=ATOL)
