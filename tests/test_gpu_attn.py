"""Paged GQA attention on the GPU against the oracle, through the C ABI (include/sn_kernels.h).

Tolerance: within 1e-3 relative / 2e-3 absolute of the fp32 oracle (different reduction
order); also checked against the fp64 closed form. Invariants: a verify row (grouped with its sequence's other draft
rows) gives bitwise the output of the same row run alone (draft_test.m:45-67), and the result does not depend on where
the pages sit in the pool.
"""
import math

import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-3
H, KVH, D = 32, 8, 128


def setup_module(module):
    U.torch().cuda.init()


def config2_case(seed=2, S_=32, page=32, lo=256, hi=4096, n_share=8, share_cells=1024, kvh=KVH):
    """32 sequences, ctx ~ U[256, 4096], 32-token pages from a seeded permutation of one pool;
    sequences 0..7 share their first 1024 cells (their own ctx drawn from [1024, 4096] so each holds the prefix)."""
    r = np.random.default_rng(seed)
    ctx = r.integers(lo, hi + 1, S_)
    ctx[:n_share] = r.integers(share_cells, hi + 1, n_share)
    maxp = (hi + page - 1) // page
    sp = share_cells // page
    need = sum((c + page - 1) // page for c in ctx) - (n_share - 1) * sp
    perm = r.permutation(need).astype(np.int32)
    pt = np.full((S_, maxp), -1, np.int32)
    k = 0
    for s in range(S_):
        for c in range((ctx[s] + page - 1) // page):
            if 0 < s < n_share and c < sp:
                pt[s, c] = pt[0, c]
            else:
                pt[s, c] = perm[k]
                k += 1
    kpool = r.standard_normal((need, kvh, page, D), dtype=np.float32).astype(np.float16).view(np.uint16)
    vpool = r.standard_normal((need, kvh, page, D), dtype=np.float32).astype(np.float16).view(np.uint16)
    q = r.standard_normal((S_, H, D), dtype=np.float32)
    return q, np.arange(S_, dtype=np.int32), (ctx - 1).astype(np.int32), kpool, vpool, pt, page


def attn_gpu(q, seq, pos, kpool, vpool, pt, page, scale, bufs=None, whole=None, mode=-1, share=False, runs=None,
             fold=None):
    """whole: when given, the work list's form the planner chose (whole groups, or per-chunk items and the merge) is
    checked too; mode: the form forced (snk_attn_new_mode), -1 the planner's; share: the planner sees the page table
    (snk_attn_new_pt) and reads shared chunks once for their rows; runs: when given, the number of run items the list
    holds; fold: when given, the chunk items and their merge in one launch (True: the list must take it, and no unit
    may have run on two XCDs) or in two (False). The KV head count is the pools'."""
    L = S.lib()
    kvh = kpool.shape[1]
    err = __import__("ctypes").create_string_buffer(256)
    seq = np.ascontiguousarray(seq, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    for s_, p_ in zip(seq, pos):  # every cell a row reads has a page (host-side check before the launch)
        assert np.all(pt[s_, :p_ // page + 1] >= 0)
    if share:
        ptc = np.ascontiguousarray(pt, np.int32)
        plan = L.snk_attn_new_pt(len(seq), seq.ctypes.data, pos.ctypes.data, H, kvh, pt.shape[1], page, mode,
                                 ptc.ctypes.data, err, 256)
    else:
        plan = L.snk_attn_new_mode(len(seq), seq.ctypes.data, pos.ctypes.data, H, kvh, pt.shape[1], page, mode, err,
                                   256)
    assert plan, err.value
    if whole is not None:
        assert L.snk_attn_whole(plan) == int(whole)
    if runs is not None:
        assert L.snk_attn_runs(plan) == runs, (L.snk_attn_runs(plan), runs)
    if bufs is None:
        bufs = (U.dev(U.k_pages(kpool)), U.dev(vpool), U.dev(pt))
    if fold is not None:
        assert L.snk_attn_fold(plan, int(fold)) == int(fold)
    dq = U.dev(q)
    out = U.empty(q.size * 4)
    rc = L.snk_attn_run(plan, U.ptr(dq), H * D, U.ptr(bufs[0]), U.ptr(bufs[1]), U.ptr(bufs[2]), scale, U.ptr(out),
                        H * D, U.stream())
    faults = L.snk_attn_xcd_faults(plan) if fold else 0
    L.snk_attn_free(plan)
    assert rc == 0
    assert faults == 0
    return U.host(out, np.float32)[:q.size].reshape(q.shape)


def test_config2_paged_attention():
    q, seq, pos, kp, vp, pt, page = config2_case()
    scale = 1 / math.sqrt(D)
    got = attn_gpu(q, seq, pos, kp, vp, pt, page, scale)
    ref = O.paged_attn(q, seq, pos, KVH, kp, vp, page, pt, scale)
    err = np.abs(got - ref)
    print(f"config 2: max abs err {err.max():.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref))
    ref64 = O.paged_attn(q, seq, pos, KVH, kp, vp, page, pt, scale, f64=True)
    assert np.max(np.abs(got - ref64)) < 1e-4


@pytest.mark.parametrize("kvh,n_share", [(8, 8), (8, 6), (4, 5)])
def test_shared_prefix_read_once(kvh, n_share):
    """Rows of sequences whose first 1024 cells are the same pages (config 2's sharers): the planner given the page
    table serves each shared 256-cell chunk of up to 16 / G rows with one work item, so its K/V is read once for them.
    Each row's output equals the unshared plan's bit for bit (a query's chunk partial depends on its own column only),
    with groups of sharers split into items of up to 4 (G = 4) or 2 (G = 8) rows and a lone last sharer on its own
    item; and it matches the oracle."""
    q, seq, pos, kp, vp, pt, page = config2_case(n_share=n_share, kvh=kvh)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    a = attn_gpu(q, seq, pos, kp, vp, pt, page, scale, bufs=bufs, mode=0)
    b = attn_gpu(q, seq, pos, kp, vp, pt, page, scale, bufs=bufs, mode=0, share=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = O.paged_attn(q, seq, pos, kvh, kp, vp, page, pt, scale)
    assert np.all(np.abs(b - ref) <= ATOL + RTOL * np.abs(ref))


@pytest.mark.parametrize("page", [32, 64])
def test_short_and_ragged_contexts(page):
    # contexts of 1 cell, chunk and page edges
    ctxs = np.array([1, 2, 31, 32, 33, 63, 64, 65, 255, 256, 257, 511, 512, 513, 1000], np.int32)
    r = np.random.default_rng(5)
    S_ = len(ctxs)
    maxp = (ctxs.max() + page - 1) // page
    npg = int(sum((c + page - 1) // page for c in ctxs))
    perm = r.permutation(npg).astype(np.int32)
    pt = np.full((S_, maxp), -1, np.int32)
    k = 0
    for s in range(S_):
        for c in range((ctxs[s] + page - 1) // page):
            pt[s, c] = perm[k]
            k += 1
    kp = r.standard_normal((npg, KVH, page, D), dtype=np.float32).astype(np.float16).view(np.uint16)
    vp = r.standard_normal((npg, KVH, page, D), dtype=np.float32).astype(np.float16).view(np.uint16)
    q = r.standard_normal((S_, H, D), dtype=np.float32) * 3
    seq = np.arange(S_, dtype=np.int32)
    pos = ctxs - 1
    scale = 1 / math.sqrt(D)
    got = attn_gpu(q, seq, pos, kp, vp, pt, page, scale)
    ref = O.paged_attn(q, seq, pos, KVH, kp, vp, page, pt, scale)
    assert np.all(np.abs(got - ref) <= ATOL + RTOL * np.abs(ref))


def test_verify_rows_equal_single_rows_bitwise():
    q, seq, pos, kp, vp, pt, page = config2_case(seed=7, S_=4, lo=300, hi=800, n_share=0)
    scale = 1 / math.sqrt(D)
    # 4 draft rows of each sequence at positions p0 .. p0 + 3 (causal within the draft)
    rows_seq = np.repeat(seq, 4).astype(np.int32)
    p0 = pos - 3
    rows_pos = (np.repeat(p0, 4) + np.tile(np.arange(4), len(seq))).astype(np.int32)
    r = np.random.default_rng(8)
    qv = r.standard_normal((len(rows_seq), H, D), dtype=np.float32)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    grouped = attn_gpu(qv, rows_seq, rows_pos, kp, vp, pt, page, scale, bufs)
    for i in range(len(rows_seq)):
        one = attn_gpu(qv[i:i + 1].copy(), rows_seq[i:i + 1].copy(), rows_pos[i:i + 1].copy(), kp, vp, pt, page,
                       scale, bufs)
        assert np.array_equal(one[0].view(np.uint32), grouped[i].view(np.uint32)), i
    ref = O.paged_attn(qv, rows_seq, rows_pos, KVH, kp, vp, page, pt, scale)
    assert np.all(np.abs(grouped - ref) <= ATOL + RTOL * np.abs(ref))


def test_page_placement_does_not_matter():
    q, seq, pos, kp, vp, pt, page = config2_case(seed=9, S_=6, lo=200, hi=1500, n_share=0)
    scale = 1 / math.sqrt(D)
    a = attn_gpu(q, seq, pos, kp, vp, pt, page, scale)
    r = np.random.default_rng(10)
    perm = r.permutation(kp.shape[0]).astype(np.int32)  # move page p to perm[p]
    kp2 = np.empty_like(kp)
    vp2 = np.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    pt2 = np.where(pt >= 0, perm[np.maximum(pt, 0)], -1).astype(np.int32)
    b = attn_gpu(q, seq, pos, kp2, vp2, pt2, page, scale)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("page,lo,hi,auto", [(32, 256, 4096, False), (64, 200, 700, False), (32, 1, 300, False),
                                            (64, 2560, 4096, False), (32, 3000, 3100, True), (64, 2560, 2600, True)])
def test_whole_group_list_equals_chunk_list_bitwise(page, lo, hi, auto):
    """The two forms of the work list on the same 32 rows: whole groups (one workgroup walks a row's whole context and
    writes its output, no merge) and per-chunk items with the merge. The outputs are the same bits (the chunk partials
    are folded in the same order with the same arithmetic), they match the oracle, and the planner picks whole groups
    for these 32 x 8 workgroups exactly when the contexts are long and alike (auto)."""
    q, seq, pos, kp, vp, pt, pg = config2_case(seed=11 + lo, S_=32, page=page, lo=lo, hi=hi, n_share=0)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    whole = attn_gpu(q, seq, pos, kp, vp, pt, pg, scale, bufs, mode=1)
    split = attn_gpu(q, seq, pos, kp, vp, pt, pg, scale, bufs, mode=0)
    assert np.array_equal(whole.view(np.uint32), split.view(np.uint32))
    attn_gpu(q[:1], seq[:1], pos[:1], kp, vp, pt, pg, scale, bufs, whole=False)  # 8 workgroups: never whole
    auto_out = attn_gpu(q, seq, pos, kp, vp, pt, pg, scale, bufs, whole=auto)
    assert np.array_equal(auto_out.view(np.uint32), whole.view(np.uint32))
    ref = O.paged_attn(q, seq, pos, KVH, kp, vp, pg, pt, scale)
    assert np.all(np.abs(whole - ref) <= ATOL + RTOL * np.abs(ref))


@pytest.mark.parametrize("kvh", [4, 2, 16])
def test_gqa_group_sizes(kvh):
    """Other query-group sizes G = H / KVH: 8 (configs[4], Qwen3-30B-A3B: 32 query heads on 4 KV heads, so a query
    group holds 2 rows of a sequence), 16 (one row a group) and 2 (up to 8 rows). Decode rows of 32 sequences with
    C5-like contexts (about 2048 cells, 4 sharers of a 1024-cell prefix), then 4 verify rows of 8 sequences each
    (split into groups of 16 / G rows): against the fp32 and fp64 oracle, verify rows bit for bit equal to the same
    rows alone, and both work-list forms bit for bit equal (the kernels index rows and heads by G; attn_part, any G,
    kernels.metal:1135-1200; fa2_128_g8, kernels.metal:2674-2770)."""
    q, seq, pos, kp, vp, pt, page = config2_case(seed=31 + kvh, S_=32, page=64, lo=1500, hi=2600, n_share=4,
                                                 kvh=kvh)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    got = attn_gpu(q, seq, pos, kp, vp, pt, page, scale, bufs)
    ref = O.paged_attn(q, seq, pos, kvh, kp, vp, page, pt, scale)
    err = np.abs(got - ref)
    print(f"G={H // kvh} decode: max abs err {err.max():.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref))
    ref64 = O.paged_attn(q, seq, pos, kvh, kp, vp, page, pt, scale, f64=True)
    assert np.max(np.abs(got - ref64)) < 1e-4
    for mode in (0, 1):
        forced = attn_gpu(q, seq, pos, kp, vp, pt, page, scale, bufs, mode=mode)
        assert np.array_equal(forced.view(np.uint32), got.view(np.uint32)), mode
    # verify rows: 4 consecutive positions of each of 8 sequences
    vseq = np.repeat(seq[:8], 4).astype(np.int32)
    vpos = (np.repeat(pos[:8] - 3, 4) + np.tile(np.arange(4), 8)).astype(np.int32)
    qv = np.random.default_rng(kvh).standard_normal((32, H, D), dtype=np.float32)
    grouped = attn_gpu(qv, vseq, vpos, kp, vp, pt, page, scale, bufs)
    ref = O.paged_attn(qv, vseq, vpos, kvh, kp, vp, page, pt, scale)
    assert np.all(np.abs(grouped - ref) <= ATOL + RTOL * np.abs(ref))
    for i in (0, 1, 2, 3, 13, 31):
        one = attn_gpu(qv[i:i + 1].copy(), vseq[i:i + 1].copy(), vpos[i:i + 1].copy(), kp, vp, pt, page, scale, bufs)
        assert np.array_equal(one[0].view(np.uint32), grouped[i].view(np.uint32)), i


@pytest.mark.parametrize("kvh,page", [(8, 32), (8, 64), (4, 64)])
def test_prompt_runs_equal_chunk_items_bitwise(kvh, page):
    """Prompt rows as run items: up to 4 consecutive query groups of one sequence (16 rows at G = 4, 8 at G = 8) walked
    over their context by one workgroup per (item, KV head), K/V cells read once for all of them, outputs written
    directly (the prompt attention of attn_pre, kernels.metal:1201-1306). Rows of four sequences: 64 prompt rows
    across the 256-cell chunk edge, 41 rows (a run whose last group is short and a lone row after it), a decode row
    and 6 rows from position 0. Run items (mode 2), per-chunk items with the merge (mode 0) and whole groups (mode 1)
    give the same bits for every row; the planner's own choice (-1: too few workgroups for run items) too; and the
    rows match the fp32 oracle."""
    q, seq, pos, kp, vp, pt, pg = config2_case(seed=40 + kvh + page, S_=4, page=page, lo=1100, hi=1500, n_share=0,
                                               kvh=kvh)
    G = H // kvh
    spans = [(0, 230, 64), (1, 1000, 41), (2, int(pos[2]), 1), (3, 0, 6)]
    rseq = np.concatenate([np.full(n, s_, np.int32) for s_, _, n in spans])
    rpos = np.concatenate([np.arange(p0, p0 + n, dtype=np.int32) for _, p0, n in spans])
    r = np.random.default_rng(kvh * page)
    qr = r.standard_normal((len(rseq), H, D), dtype=np.float32)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    # run items of up to 4 groups: 64 rows in groups of 16 / G rows; 41 rows in 10 (G = 4) or 20 (G = 8) full groups
    # and a short last one, which joins the run; the 6 rows from position 0 in 2 (G = 4) or 3 groups; the decode row
    # stays a group of its own
    gmax = 16 // G
    n_runs = sum(-(-(-(-n // gmax)) // 4) for n in (64, 41, 6))
    runs = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, mode=2, runs=n_runs)
    chunks = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, mode=0, runs=0)
    whole = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, mode=1, runs=0)
    auto = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, runs=0)
    assert np.array_equal(runs.view(np.uint32), chunks.view(np.uint32))
    assert np.array_equal(runs.view(np.uint32), whole.view(np.uint32))
    assert np.array_equal(runs.view(np.uint32), auto.view(np.uint32))
    ref = O.paged_attn(qr, rseq, rpos, kvh, kp, vp, pg, pt, scale)
    err = np.abs(runs - ref)
    print(f"G={G} page {pg}: {len(rseq)} rows, max abs err {err.max():.3g}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref))


def test_prompt_runs_chosen_for_prompt_steps():
    """The planner takes run items by itself when they make at least 128 workgroups: one sequence's 512 prompt rows
    at positions 1536 .. 2047 (128 groups of 4 rows: 32 run items x 8 KV heads), bit for bit the chunk items' output
    and the oracle's within tolerance."""
    q, seq, pos, kp, vp, pt, pg = config2_case(seed=50, S_=1, page=64, lo=2048, hi=2048, n_share=0)
    rseq = np.zeros(512, np.int32)
    rpos = np.arange(1536, 2048, dtype=np.int32)
    qr = np.random.default_rng(51).standard_normal((512, H, D), dtype=np.float32)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    auto = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, runs=32)
    chunks = attn_gpu(qr, rseq, rpos, kp, vp, pt, pg, scale, bufs, mode=0, runs=0)
    assert np.array_equal(auto.view(np.uint32), chunks.view(np.uint32))
    sel = np.r_[0:8, 250:262, 504:512]  # rows at the first, middle and last chunk edges (the oracle is slow)
    ref = O.paged_attn(qr[sel], rseq[sel], rpos[sel], KVH, kp, vp, pg, pt, scale)
    assert np.all(np.abs(auto[sel] - ref) <= ATOL + RTOL * np.abs(ref))


@pytest.mark.skip(reason="k_attn_fold withdrawn: one run of this test differed (kvh 16, 64-cell pages, contexts "
                         "300..1200) on one MI355X, 45 repeats on another box were equal and no cause was found by "
                         "reading the handoff; snk_attn_fold now refuses the form")
@pytest.mark.parametrize("kvh,page,lo,hi,verify", [(8, 32, 256, 4096, False), (8, 64, 2040, 2100, False),
                                                   (4, 64, 1500, 2600, True), (8, 32, 1, 300, True),
                                                   (16, 64, 300, 1200, False), (2, 64, 500, 900, True)])
def test_fold_equals_two_launches_bitwise(kvh, page, lo, hi, verify):
    """The chunk items and their merge in one launch (k_attn_fold: a (group, KV head)'s chunk workgroups dealt to one
    XCD, the last of them folding the group's rows through its L2) against the partial kernel and the merge kernel:
    the same bits on decode rows and on 4-row verify groups, at G = 2 .. 16 and both page sizes, against the oracle,
    and no unit found on two XCDs."""
    q, seq, pos, kp, vp, pt, pg = config2_case(seed=50 + kvh + lo, S_=32, page=page, lo=lo, hi=hi, n_share=0, kvh=kvh)
    if verify:  # 4 consecutive positions of each of 8 sequences
        seq = np.repeat(seq[:8], 4).astype(np.int32)
        pos = (np.repeat(np.maximum(pos[:8], 3) - 3, 4) + np.tile(np.arange(4), 8)).astype(np.int32)
        q = np.random.default_rng(kvh + 1).standard_normal((32, H, D), dtype=np.float32)
    scale = 1 / math.sqrt(D)
    bufs = (U.dev(U.k_pages(kp)), U.dev(vp), U.dev(pt))
    one = attn_gpu(q, seq, pos, kp, vp, pt, pg, scale, bufs, mode=0, fold=True)
    two = attn_gpu(q, seq, pos, kp, vp, pt, pg, scale, bufs, mode=0, fold=False)
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))
    ref = O.paged_attn(q, seq, pos, kvh, kp, vp, pg, pt, scale)
    assert np.all(np.abs(one - ref) <= ATOL + RTOL * np.abs(ref))
