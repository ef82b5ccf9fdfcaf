"""Greedy argmax of logit rows (argmax / argmax_p, kernels.metal:327-442) on the GPU against the oracle's or_argmax and
or_top2, through the C ABI (include/sn_kernels.h snk_argmax).

Bar: chosen ids, best/second ids and their scores bit-exact (a selection, no arithmetic); the log-sum-exp within 2e-6
relative of the oracle's double-precision sum (the kernel sums exp in fp32 per chunk, then rescales chunk sums).
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

LSE_RTOL = 2e-6


def setup_module(module):
    U.torch().cuda.init()


def run(x, ban=(), skip=None, rec=True):
    L = S.lib()
    n, V = x.shape
    ws = U.empty(L.snk_argmax_workspace_bytes(n, V))
    out = U.empty(n * 4)
    rb = U.empty(n * 32)
    b = U.dev(np.array(ban, np.int32)) if len(ban) else None
    sk = U.dev(np.array(skip, np.uint8)) if skip is not None else None
    rc = L.snk_argmax(U.ptr(U.dev(x.astype(np.float32))), V, n, U.ptr(b) if b is not None else None, len(ban),
                      U.ptr(sk) if sk is not None else None, U.ptr(out), U.ptr(rb) if rec else None, U.ptr(ws),
                      ws.numel(), U.stream())
    assert rc == 0
    return U.host(out, np.int32)[:n].copy(), U.host(rb, np.float32)[:n * 8].reshape(n, 8).copy()


def check(x, ban=(), skip=None):
    got, rec = run(x, ban, skip)
    for r in range(x.shape[0]):
        banned = ban if (skip is not None and skip[r]) else ()
        want = O.argmax(x[r], banned)
        assert got[r] == want, (r, got[r], want)
        i1, v1, i2, v2, lse = O.top2(x[r])
        rr = rec[r]
        assert rr[0:1].view(np.int32)[0] == want
        if want >= 0:
            assert rr[1] == x[r, want]
        assert rr[2:3].view(np.int32)[0] == i1 and rr[3] == v1
        assert rr[4:5].view(np.int32)[0] == i2 and rr[5] == v2
        if np.isfinite(lse):
            assert abs(rr[6] - lse) <= LSE_RTOL * max(1.0, abs(lse)), (r, rr[6], lse)
        else:
            assert rr[6] == lse
        assert rr[7] == 0.0


@pytest.mark.parametrize("n,V", [(1, 1000), (5, 4096), (3, 4097), (7, 8193), (32, 151936)])
def test_argmax_random_rows(n, V):
    r = np.random.default_rng(V + n)
    x = (r.standard_normal((n, V)) * 4).astype(np.float32)
    check(x)


def test_argmax_ties_take_the_lowest_id():
    V = 3 * 4096 + 17
    x = np.random.default_rng(1).standard_normal((6, V)).astype(np.float32)
    # ties inside a thread's ids, across threads of a chunk, across chunk boundaries, and a three-way tie for second
    for r, ids in enumerate([(5, 261), (300, 301), (4095, 4096), (8191, 12288), (V - 1, 0), (4096 * 2 + 7, 33)]):
        for i in ids:
            x[r, i] = 50.0
    x[5, [40, 4100, 9000]] = 49.0
    x[5, 4096 * 2 + 7] = 49.0  # now 33 is the unique max and three ids (40 < 4100 < 8199 < 9000) tie for second
    check(x)


def test_argmax_bans_only_skip_rows():
    V = 10000
    x = np.random.default_rng(2).standard_normal((4, V)).astype(np.float32)
    top = int(np.argmax(x[0]))
    for r in range(4):
        x[r, top] = 100.0
        x[r, 7] = 99.0
    ban = (top, 3, 9999)
    check(x, ban, skip=[1, 0, 1, 0])
    got, _ = run(x, ban, skip=[1, 0, 1, 0], rec=False)
    assert list(got) == [7, top, 7, top]


def test_argmax_all_minus_inf_and_all_banned():
    x = np.full((3, 4100), -np.inf, np.float32)
    # every score -inf: the first id that is not banned (or_argmax), row 1 with ids 0 and 1 banned
    check(x, ban=(0, 1), skip=[0, 1, 0])
    got, _ = run(x, ban=(0, 1), skip=[0, 1, 0])
    assert list(got) == [0, 2, 0]
    # every id banned: -1
    y = np.random.default_rng(3).standard_normal((2, 5)).astype(np.float32)
    check(y, ban=(0, 1, 2, 3, 4), skip=[1, 0])
    got, _ = run(y, ban=(0, 1, 2, 3, 4), skip=[1, 0])
    assert got[0] == -1


def test_argmax_rejects_small_workspace():
    L = S.lib()
    x = U.dev(np.zeros((2, 5000), np.float32))
    out = U.empty(8)
    ws = U.empty(L.snk_argmax_workspace_bytes(2, 5000) - 32)
    assert L.snk_argmax(U.ptr(x), 5000, 2, None, 0, None, U.ptr(out), None, U.ptr(ws),
                        L.snk_argmax_workspace_bytes(2, 5000) - 32, U.stream()) == -1
