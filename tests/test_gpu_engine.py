"""The engine behind sn.h on the GPU against the oracle's Qwen3 step (a small random-init model written by
snx_write_model), plus the step-level invariants of the reference's benches: a row's tokens do not depend on the
other rows (qbench.m:158-168), copied prefixes equal their source, cut-back cells are rebuilt bit for bit
(draft_test.m:45-67), and the cache error paths (-2 out of pages, bad shapes).

Two levels of parity:
  * stage by stage: each stage of a layer fed the engine's own previous stage agrees with the oracle's stage to the
    per-op tolerance (1e-3 relative / 2e-3 absolute), in practice to ~1e-7;
  * end to end: the GPU and the oracle sum in different fp32 orders, so now and then a value lands on the other side of
    an fp16 (K/V cache) or Q8_0 (activation) rounding boundary and moves by a whole step; over layers this leaves the
    logits apart by the activations' Q8_0 noise (~1e-2 for this model). Greedy tokens are compared wherever the
    oracle's top-2 gap exceeds that bound (MODEL_ATOL); the north star's 1e-4 gap cannot be held by any implementation
    whose summation order differs from ggml's, and the fraction of rows under the bound is printed.
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000)


def setup_module(module):
    U.torch().cuda.init()


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "tiny.gguf")
    S.write_model(path, S.model_cfg(**TINY), seed=11)
    return path


MODEL_ATOL = 3e-2  # end-to-end logit bound of this 2-layer model (Q8_0 activation noise; measured 1.1e-2)
RTOL, ATOL = 1e-3, 2e-3  # per-op tolerance


def check_tokens(got, ref_tok, ref_logits, stats):
    for j in range(len(got)):
        i1, v1, i2, v2, _ = O.top2(ref_logits[j])
        stats["rows"] += 1
        if v1 - v2 > 2 * MODEL_ATOL:
            stats["checked"] += 1
            assert got[j] == ref_tok[j], (j, got[j], ref_tok[j], v1 - v2)
        stats["same"] += int(got[j] == ref_tok[j])


def test_prefill_and_decode_match_oracle(tiny):
    prefill_and_decode(tiny)


@pytest.mark.parametrize("embd_type,tied,wtype", [(14, 1, 2), (14, 0, 8), (8, 1, 8), (2, 1, 2), (8, 0, 2)])
def test_token_tables_and_tied_heads(tmp_path, embd_type, tied, wtype):
    """Quantized token tables (Q4_0, Q8_0, Q6_K: dequantized at load, ggml's dequantize_row_* element for element) and
    the LM head tied to them (sn_load.inc.h:341-352): Q6_K heads take Q8_K activations, as ggml's CPU path does."""
    path = str(tmp_path / "t.gguf")
    S.write_model(path, S.model_cfg(**TINY, embd_type=embd_type, tied=tied, wtype=wtype), seed=12)
    g = GGUF(path)
    assert ("output.weight" in g.tinfo) == (not tied)
    prefill_and_decode(path)


@pytest.mark.parametrize("n_ff", [17408, 25600])
def test_deep_down_projection_matches_oracle(tmp_path, n_ff):
    """FFN widths of Qwen3-14B (17408) and Qwen3-32B (25600): the down projection's plan takes slices of 10 and 14
    groups (the ring kernel at decode row counts) so that the row kernels add at most 16 k-slices; prefill and decode
    against the oracle (its reversed-order drift on these models: 0.011)."""
    path = str(tmp_path / "deep.gguf")
    S.write_model(path, S.model_cfg(**dict(TINY, n_ff=n_ff)), seed=14)
    assert S.q4_plan(TINY["n_embd"], n_ff)[1] <= 16
    prefill_and_decode(path)


def prefill_and_decode(path):
    ref = O.Qwen3(GGUF(path), n_seq=4, ctx=256)
    r = np.random.default_rng(0)
    lens = [40, 23]
    toks = [r.integers(0, TINY["n_vocab"], n).astype(np.int32) for n in lens]
    with S.Engine(path, slots=4, ctx=256, max_rows=64) as eng:
        # one step of prompt rows for both sequences, outputs at their last rows
        tok = np.concatenate(toks)
        seq = np.concatenate([np.full(n, s, np.int32) for s, n in enumerate(lens)])
        pos = np.concatenate([np.arange(n, dtype=np.int32) for n in lens])
        outs = np.array([lens[0] - 1, sum(lens) - 1], np.int32)
        got = eng.step(tok, seq, pos, outs, n_write=0)
        rt, rl, _ = ref.step(tok, seq, pos, outs)
        gl = eng.logits([0, 1])
        print("prefill max |logit diff|", np.abs(gl - rl).max())
        assert np.abs(gl - rl).max() <= MODEL_ATOL
        stats = {"rows": 0, "checked": 0, "same": 0}
        check_tokens(got, rt, rl, stats)
        # greedy decode, both sequences each step, fed the oracle's tokens
        cur = rt.copy()
        p = np.array(lens, np.int32)
        for step in range(6):
            got = eng.step(cur, np.array([0, 1], np.int32), p, np.array([0, 1], np.int32))
            rt, rl, _ = ref.step(cur, np.array([0, 1], np.int32), p, np.array([0, 1], np.int32))
            gl = eng.logits([0, 1])
            assert np.abs(gl - rl).max() <= MODEL_ATOL, step
            check_tokens(got, rt, rl, stats)
            cur = rt.copy()
            p += 1
        print("end to end:", stats)
        assert stats["same"] == stats["rows"]


def test_32_cell_pages_match_oracle(tiny, monkeypatch):
    """SN_PAGE=32 (config 2's page size, sn.h:13 keeps 64 by default): the same prefill and decode against the oracle,
    with a 40-row prompt taking two pages."""
    monkeypatch.setenv("SN_PAGE", "32")
    with S.Engine(tiny, slots=2, ctx=256, max_rows=64) as eng:
        eng.step(np.arange(40, dtype=np.int32), np.zeros(40, np.int32), np.arange(40, dtype=np.int32),
                 np.array([39], np.int32), n_write=0)
        assert eng.seq_pages(0)[0] == 2
    prefill_and_decode(tiny)


def test_large_prompt_step_matches_oracle(tiny):
    """One step of 500 prompt rows of one sequence (32 row tiles, 125 attention query groups over up to 2 chunks) and a
    second sequence's 37, then decode steps of both: logits and tokens against the oracle as above."""
    ref = O.Qwen3(GGUF(tiny), n_seq=2, ctx=1024)
    r = np.random.default_rng(41)
    lens = [500, 37]
    toks = [r.integers(0, TINY["n_vocab"], n).astype(np.int32) for n in lens]
    tok = np.concatenate(toks)
    seq = np.concatenate([np.full(n, s, np.int32) for s, n in enumerate(lens)])
    pos = np.concatenate([np.arange(n, dtype=np.int32) for n in lens])
    outs = np.array([lens[0] - 1, sum(lens) - 1], np.int32)
    stats = {"rows": 0, "checked": 0, "same": 0}
    with S.Engine(tiny, slots=2, ctx=1024, max_rows=544) as eng:
        got = eng.step(tok, seq, pos, outs, n_write=0)
        rt, rl, _ = ref.step(tok, seq, pos, outs)
        gl = eng.logits([0, 1])
        print("500-row prompt max |logit diff|", np.abs(gl - rl).max())
        assert np.abs(gl - rl).max() <= MODEL_ATOL
        check_tokens(got, rt, rl, stats)
        cur = rt.copy()
        p = np.array(lens, np.int32)
        for _ in range(3):
            got = eng.step(cur, np.array([0, 1], np.int32), p, np.array([0, 1], np.int32))
            rt, rl, _ = ref.step(cur, np.array([0, 1], np.int32), p, np.array([0, 1], np.int32))
            assert np.abs(eng.logits([0, 1]) - rl).max() <= MODEL_ATOL
            check_tokens(got, rt, rl, stats)
            cur = rt.copy()
            p += 1
    print("end to end:", stats)  # tokens are compared where the oracle's top-2 gap clears the bound (check_tokens)
    assert stats["checked"] >= 4


def test_stagewise_parity(tmp_path):
    """One layer, 40 prompt rows of one sequence: each stage against the oracle given the engine's previous stage."""
    import ctypes as C
    import math
    path = str(tmp_path / "one.gguf")
    S.write_model(path, S.model_cfg(**dict(TINY, n_layer=1)), seed=11)
    g = GGUF(path)
    E, H, KVH, D, F, V = 256, 8, 2, 128, 512, 1000
    QD, KD = H * D, KVH * D
    r = np.random.default_rng(0)
    T = 40
    tok = r.integers(0, V, T).astype(np.int32)
    eps = float(g.kv["qwen3.attention.layer_norm_rms_epsilon"])
    ts = np.float32(np.power(np.float32(1e6), np.float32(-2.0 / D)))
    L = S.lib()
    L.snx_debug_read.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]
    with S.Engine(path, slots=2, ctx=256, max_rows=64) as eng:
        eng.step(tok, np.zeros(T, np.int32), np.arange(T, dtype=np.int32), np.array([T - 1], np.int32), n_write=0)

        def rd(which, cols):
            out = np.empty((T, cols), np.float32)
            assert L.snx_debug_read(eng.e, which, out.ctypes.data, out.size) == 0
            return out
        gx, gq, gao, ghb = rd(0, E), rd(1, QD + 2 * KD), rd(2, QD), rd(3, F)
    t = g.tensor
    x0 = t("token_embd.weight")[tok].astype(np.float32)
    h = O.rmsnorm(x0, t("blk.0.attn_norm.weight"), eps)
    q = O.mul_mat_q4_0(t("blk.0.attn_q.weight"), E, h)
    k = O.mul_mat_q4_0(t("blk.0.attn_k.weight"), E, h)
    v = O.mul_mat_q4_0(t("blk.0.attn_v.weight"), E, h)
    assert np.allclose(gq[:, QD:], np.concatenate([k, v], 1), rtol=RTOL, atol=ATOL)  # k, v stay raw in the buffer
    qn, kn = t("blk.0.attn_q_norm.weight"), t("blk.0.attn_k_norm.weight")
    kr = gq[:, QD:QD + KD].copy()
    qr = gq[:, :QD].copy()
    for i in range(T):
        cs = O.rope_cache(i, ts, D)
        for hh in range(H):
            want = O.qk_norm_rope(q[i, hh * D:(hh + 1) * D], qn, eps, cs)
            assert np.allclose(qr[i, hh * D:(hh + 1) * D], want, rtol=RTOL, atol=ATOL)
        for hh in range(KVH):
            kr[i, hh * D:(hh + 1) * D] = O.qk_norm_rope(gq[i, QD + hh * D:QD + (hh + 1) * D], kn, eps, cs)
    # attention over the engine's q and its k, v (fp16 cells), one page table for the 40 cells
    kp = kr.reshape(T, KVH, D).transpose(1, 0, 2)[None].astype(np.float16).view(np.uint16).copy()
    vp = gq[:, QD + KD:].reshape(T, KVH, D).transpose(1, 0, 2)[None].astype(np.float16).view(np.uint16).copy()
    kp = np.concatenate([kp, np.zeros((1, KVH, 64 - T, D), np.uint16)], 2)
    vp = np.concatenate([vp, np.zeros((1, KVH, 64 - T, D), np.uint16)], 2)
    ao = O.paged_attn(qr.reshape(T, H, D), np.zeros(T, np.int32), np.arange(T, dtype=np.int32), KVH, kp, vp, 64,
                      np.zeros((1, 1), np.int32), 1 / math.sqrt(D)).reshape(T, QD)
    assert np.allclose(gao, ao, rtol=RTOL, atol=ATOL)
    # the FFN and both residual adds on the engine's attention output
    x1 = x0 + O.mul_mat_q4_0(t("blk.0.attn_output.weight"), QD, gao)
    h2 = O.rmsnorm(x1, t("blk.0.ffn_norm.weight"), eps)
    gg = O.mul_mat_q4_0(t("blk.0.ffn_gate.weight"), E, h2).astype(np.float64)
    uu = O.mul_mat_q4_0(t("blk.0.ffn_up.weight"), E, h2).astype(np.float64)
    assert np.allclose(ghb, gg / (1 + np.exp(-gg)) * uu, rtol=RTOL, atol=ATOL)
    x2 = x1 + O.mul_mat_q4_0(t("blk.0.ffn_down.weight"), F, ghb)
    assert np.allclose(gx, x2, rtol=RTOL, atol=ATOL)
    print("stage diffs: ao %.2g hb %.2g x %.2g" % (np.abs(gao - ao).max(), np.abs(ghb - gg / (1 + np.exp(-gg)) * uu).max(),
                                                  np.abs(gx - x2).max()))


def test_row_invariance_copy_and_cut(tiny):
    r = np.random.default_rng(1)
    with S.Engine(tiny, slots=4, ctx=256, max_rows=128) as eng:
        a = r.integers(0, 1000, 70).astype(np.int32)
        b = r.integers(0, 1000, 50).astype(np.int32)
        eng.step(a, np.zeros(70, np.int32), np.arange(70, dtype=np.int32), np.array([69], np.int32), n_write=0)
        eng.step(b, np.ones(50, np.int32), np.arange(50, dtype=np.int32), np.array([49], np.int32), n_write=0)
        eng.copy(0, 2, 70)  # a full page shared, the partial page copied
        # slot 0 in a 2-row step vs its copy alone
        eng.step(np.array([5, 6], np.int32), np.array([0, 1], np.int32), np.array([70, 50], np.int32),
                 np.array([0, 1], np.int32))
        l_pair = eng.logits([0])
        eng.step(np.array([5], np.int32), np.array([2], np.int32), np.array([70], np.int32), np.array([0], np.int32))
        l_alone = eng.logits([0])
        assert np.array_equal(l_pair.view(np.uint32), l_alone.view(np.uint32))
        # draft rows of one sequence (a verify step) vs the same rows one step each, with cut-backs
        toks = np.array([7, 8, 9, 10], np.int32)
        eng.step(toks, np.full(4, 2, np.int32), np.arange(71, 75, dtype=np.int32), np.arange(4, dtype=np.int32),
                 n_fast=-4)
        l_verify = eng.logits(np.arange(4))
        eng.clear(2, 71, 75)
        singles = []
        for i in range(4):
            eng.step(toks[i:i + 1], np.array([2], np.int32), np.array([71 + i], np.int32), np.array([0], np.int32))
            singles.append(eng.logits([0])[0])
        assert np.array_equal(np.stack(singles).view(np.uint32), l_verify.view(np.uint32))
        # save / load: slot 2's cells into slot 3 give the same next row
        kv = eng.kv_save(2, 75)
        eng.kv_load(3, 75, kv)
        eng.step(np.array([11], np.int32), np.array([2], np.int32), np.array([75], np.int32), np.array([0], np.int32))
        x = eng.logits([0])
        eng.step(np.array([11], np.int32), np.array([3], np.int32), np.array([75], np.int32), np.array([0], np.int32))
        y = eng.logits([0])
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_error_paths(tiny):
    with S.Engine(tiny, slots=2, ctx=256, max_rows=16, pages=3) as eng:
        # sn_cut_best (sn_cache.inc.h:448-452): a bad slot or n <= 0 gives 0, otherwise sn_cut_ok's n
        L = S.lib()
        assert (L.sn_cut_best(eng.e, -1, 5), L.sn_cut_best(eng.e, 2, 5), L.sn_cut_best(eng.e, 0, 0)) == (0, 0, 0)
        assert L.sn_cut_best(eng.e, 1, 10) == 10 and L.sn_cut_ok(eng.e, 1, 10) == 1
        with pytest.raises(S.SnError) as ei:
            eng.step(np.array([1], np.int32), np.array([5], np.int32), np.array([0], np.int32), np.array([0], np.int32))
        assert ei.value.rc == -1
        with pytest.raises(S.SnError) as ei:
            eng.step(np.zeros(17, np.int32), np.zeros(17, np.int32), np.arange(17, dtype=np.int32),
                     np.array([0], np.int32))
        assert ei.value.rc == -1
        eng.step(np.zeros(16, np.int32), np.zeros(16, np.int32), np.arange(16, dtype=np.int32), np.array([15], np.int32),
                 n_write=0)
        # slot 1 starts at cell 64: its unwritten first page is given too (zero cells)
        eng.step(np.zeros(1, np.int32), np.ones(1, np.int32), np.array([64], np.int32), np.array([0], np.int32))
        assert eng.pages_free() == 0 and eng.seq_pages(1)[0] == 2
        with pytest.raises(S.SnError) as ei:  # a third page: out of pages, nothing ran
            eng.step(np.zeros(1, np.int32), np.zeros(1, np.int32), np.array([64], np.int32), np.array([0], np.int32))
        assert ei.value.rc == -2
        assert eng.pages_free() == 0
        eng.clear(1, 0, 65)
        assert eng.pages_free() == 2
    # empty, ragged and out-of-range inputs are refused before anything runs (sn_step.inc.h:97-99); the engine then
    # steps normally
    V = TINY["n_vocab"]
    with S.Engine(tiny, slots=2, ctx=256, max_rows=16) as eng:
        one = lambda t, s_, p_, o, **kw: eng.step(np.array(t, np.int32), np.array(s_, np.int32), np.array(p_, np.int32),
                                                  np.array(o, np.int32), **kw)
        for args, kw in [(([], [], [], []), {}),                      # no rows
                         (([1], [0], [0], [0]), {"n_write": 2}),      # more write rows than rows
                         (([1, 2], [0, 0], [0, 1], [2]), {}),         # an output row outside the step
                         (([V], [0], [0], [0]), {}),                  # a token outside the vocabulary
                         (([1], [0], [-1], [0]), {}),                 # a negative position
                         (([1], [0], [256], [0]), {})]:               # a position past the context
            with pytest.raises(S.SnError) as ei:
                one(*args, **kw)
            assert ei.value.rc == -1, args
        assert eng.pages_free() == eng.pages_total()
        assert one([3, 4, 5], [0, 0, 0], [0, 1, 2], [], n_write=0).size == 0  # no outputs: the cells are written
        assert eng.seq_pages(0)[0] == 1
        t = one([6], [0], [3], [0])
        assert t.size == 1 and 0 <= t[0] < V


def test_graph_replay_matches_eager(tiny):
    """Steps replayed from the captured HIP graph give the same tokens and logits, bit for bit, as eager launches: over
    repeated shapes (replays), shape changes (rows, outputs, a new 256-cell attention chunk: recaptures), with eager
    cache operations (sn_copy, sn_clear) and host reads between the replays."""
    r = np.random.default_rng(5)
    V = TINY["n_vocab"]
    with S.Engine(tiny, slots=4, ctx=512, max_rows=256) as ge, S.Engine(tiny, slots=4, ctx=512, max_rows=256) as ee:
        ee.graphs(False)
        prompt = r.integers(0, V, 250).astype(np.int32)
        for eng in (ge, ee):  # a 250-cell prompt in slot 0 (one eager-equivalent step shape)
            eng.step(prompt, np.zeros(250, np.int32), np.arange(250, dtype=np.int32), np.array([249], np.int32), n_write=0)
        for eng in (ge, ee):
            eng.copy(0, 1, 250)
        pos = np.array([250, 250], np.int32)
        tok = r.integers(0, V, 2).astype(np.int32)
        n_steps = 0
        for it in range(14):  # 2 rows crossing the 256-cell chunk boundary at position 256
            seq = np.array([0, 1], np.int32)
            outs = np.arange(2, dtype=np.int32) if it % 5 != 3 else np.array([1], np.int32)
            tg = ge.step(tok, seq, pos, outs)
            te = ee.step(tok, seq, pos, outs)
            lg, le = ge.logits(list(range(len(outs)))), ee.logits(list(range(len(outs))))
            assert np.array_equal(tg, te), (it, tg, te)
            assert np.array_equal(lg.view(np.uint32), le.view(np.uint32)), it
            n_steps += 1
            if len(outs) == 2:
                tok = tg.astype(np.int32)
            pos = pos + 1
            if it == 6:  # eager cache work between replays: cut slot 1 back one cell and rebuild it
                for eng in (ge, ee):
                    eng.clear(1, int(pos[1]) - 1, int(pos[1]))
                pos[1] -= 1
        assert n_steps == 14
        caps, reps = ge.graph_count()
        assert reps >= 5 and caps >= 3, (caps, reps)  # replays happened, and shape changes recaptured
        assert ee.graph_count() == (0, 0)


def test_graph_key_separates_attention_forms(tmp_path):
    """Regression: a step whose attention the planner runs as whole groups must not replay the graph of a step with
    per-chunk items of the same row and item counts. 32 decode rows on an H = 32, KVH = 8 model: at position 100 every
    row is one chunk (32 items and a merge); at position 3000 the contexts are long and alike, so the auto plan takes
    whole groups (32 x 8 = 256 workgroups, 32 items, no merge). Both shapes are captured and replayed, in alternation,
    and every step equals an eager engine's bit for bit."""
    path = str(tmp_path / "g8.gguf")
    S.write_model(path, S.model_cfg(n_layer=1, n_embd=256, n_head=32, n_head_kv=8, n_ff=512, n_vocab=1000), seed=21)
    seq = np.arange(32, dtype=np.int32)
    assert S.step_key(32, 8, 64, -1, seq, np.full(32, 100, np.int32))[1] is False
    assert S.step_key(32, 8, 64, -1, seq, np.full(32, 3000, np.int32))[1] is True
    r = np.random.default_rng(6)
    with S.Engine(path, slots=32, ctx=3072, max_rows=32) as ge, S.Engine(path, slots=32, ctx=3072, max_rows=32) as ee:
        ee.graphs(False)
        for eng in (ge, ee):
            for s in range(32):
                eng.fill_kv(s, 3004, seed=77)
        for it, p in enumerate((100, 3000, 101, 3001, 102)):
            tok = r.integers(0, 1000, 32).astype(np.int32)
            pos = np.full(32, p, np.int32)
            tg, te = ge.step(tok, seq, pos, seq), ee.step(tok, seq, pos, seq)
            lg, le = ge.logits(seq), ee.logits(seq)
            assert np.array_equal(tg, te), (it, p)
            assert np.array_equal(lg.view(np.uint32), le.view(np.uint32)), (it, p)
        assert ge.graph_count() == (2, 3), ge.graph_count()  # two shapes captured, each replayed


def test_probs_records_and_end_ban(tiny):
    """sn_want_probs / sn_probs and sn_set_eog / sn_no_end through sn_step (argmax_p, kernels.metal:380-442): the
    records equal the oracle's top2 and log-sum-exp of the step's own logits; a slot under no_end never takes an
    end-of-generation id, other slots may."""
    V = TINY["n_vocab"]
    r = np.random.default_rng(9)
    with S.Engine(tiny, slots=2, ctx=256, max_rows=64) as eng:
        eng.want_probs(True)
        prompt = r.integers(0, V, 12).astype(np.int32)
        seq = np.array([0] * 6 + [1] * 6, np.int32)
        pos = np.array(list(range(6)) * 2, np.int32)
        got = eng.step(prompt, seq, pos, np.array([5, 11], np.int32), n_write=0)
        lg = eng.logits([0, 1])
        pr = eng.probs(2)
        for j in range(2):
            i1, v1, i2, v2, lse = O.top2(lg[j])
            assert got[j] == O.argmax(lg[j])
            assert pr[j, 0:1].view(np.int32)[0] == got[j] and pr[j, 1] == lg[j, got[j]]
            assert pr[j, 2:3].view(np.int32)[0] == i1 and pr[j, 3] == v1
            assert pr[j, 4:5].view(np.int32)[0] == i2 and pr[j, 5] == v2
            assert abs(pr[j, 6] - lse) <= 2e-6 * max(1.0, abs(lse))
        # make both rows' greedy choices end-of-generation ids; slot 1 refuses them
        eog = np.unique(got)
        eng.set_eog(eog)
        eng.no_end(1, True)
        got2 = eng.step(prompt, seq, pos, np.array([5, 11], np.int32), n_write=0)
        lg2 = eng.logits([0, 1])
        pr2 = eng.probs(2)
        assert got2[0] == O.argmax(lg2[0]) == got[0]
        assert got2[1] == O.argmax(lg2[1], list(eog)) and got2[1] not in eog
        assert pr2[1, 0:1].view(np.int32)[0] == got2[1]
        assert pr2[1, 2:3].view(np.int32)[0] == O.top2(lg2[1])[0]  # the pair still ranks every id
        with pytest.raises(S.SnError):
            eng.set_eog([V])


def test_attention_list_forms_give_the_same_steps(tiny):
    """snx_attn_mode: whole-group attention (its kernel writes the rows' outputs and the o-projection's Q8_0 operand
    itself), per-chunk attention with the merge and run items for the prompt rows (mode 2: up to 4 consecutive query
    groups a workgroup, writing their outputs and operand) give the same tokens and logits, bit for bit, over prompt
    and decode steps that cross 256-cell chunk boundaries."""
    V = TINY["n_vocab"]
    lens = [300, 40, 530]
    outs = []
    for mode in (0, 1, 2):
        with S.Engine(tiny, slots=3, ctx=640, max_rows=256) as eng:
            eng.attn_mode(mode)
            rr = np.random.default_rng(21)
            got = []
            for s, n in enumerate(lens):  # prompts in 256-row steps
                toks = rr.integers(0, V, n).astype(np.int32)
                for a in range(0, n, 256):
                    b = min(n, a + 256)
                    t = eng.step(toks[a:b], np.full(b - a, s, np.int32), np.arange(a, b, dtype=np.int32),
                                 np.array([b - a - 1], np.int32), n_write=0)
                got.append((t.copy(), eng.logits([0]).copy()))
            cur = rr.integers(0, V, 3).astype(np.int32)
            pos = np.array(lens, np.int32)
            for it in range(4):
                t = eng.step(cur, np.arange(3, dtype=np.int32), pos, np.arange(3, dtype=np.int32))
                got.append((t.copy(), eng.logits([0, 1, 2]).copy()))
                cur = t.astype(np.int32)
                pos = pos + 1
            outs.append(got)
    for other in outs[1:]:
        for (ta, la), (tb, lb) in zip(outs[0], other):
            assert np.array_equal(ta, tb)
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_prompt_chunking_does_not_change_the_next_row(tmp_path):
    """A prompt fed in one step or in several gives the same cells and so the same next row, bit for bit (qbench.m's
    read_chunks, qbench.m:124-130): 600 prompt rows in one step (the full-K matmul walk and run items at 600 rows),
    in 200-row steps (the split launches and chunk items; the workgroup-per-row QK-RoPE adding the k-slice sums), and
    in 64 + 536 (the 64 rows through the wavefront-per-head QK-RoPE), then the same decode row. The model's
    matrices all split K (n_embd 1024: 2 slices) and its gate|up is wide enough (n_ff 3072: 384 stripes) for the prompt
    SwiGLU epilogue."""
    path = str(tmp_path / "w.gguf")
    S.write_model(path, S.model_cfg(n_layer=2, n_embd=1024, n_head=8, n_head_kv=2, n_ff=3072, n_vocab=1000), seed=13)
    assert S.q4_plan(2 * 3072, 1024)[1] > 1 and S.q4_plan(1024, 3072)[1] > 1  # (k-slices: the full-K walk applies)
    r = np.random.default_rng(14)
    toks = r.integers(0, 1000, 600).astype(np.int32)
    nxt = np.array([int(r.integers(0, 1000))], np.int32)
    outs = []
    for cuts in ([0, 600], [0, 200, 400, 600], [0, 64, 600]):
        with S.Engine(path, slots=1, ctx=1024, max_rows=600) as eng:
            for a, b in zip(cuts[:-1], cuts[1:]):
                eng.step(toks[a:b], np.zeros(b - a, np.int32), np.arange(a, b, dtype=np.int32),
                         np.array([b - a - 1], np.int32), n_write=0)
            last = eng.logits([0]).copy()
            eng.step(nxt, np.zeros(1, np.int32), np.array([600], np.int32), np.array([0], np.int32))
            outs.append((last, eng.logits([0]).copy()))
    for other in outs[1:]:
        assert np.array_equal(outs[0][0].view(np.uint32), other[0].view(np.uint32))
        assert np.array_equal(outs[0][1].view(np.uint32), other[1].view(np.uint32))


def test_chained_steps(tiny):
    """sn_step's chain (sn.h:31-41, sn_step.inc.h:31-212): a write step that samples each row in order has the next
    step queued behind it on the GPU, fed its tokens there. Chained decode gives the same tokens and logits, bit for
    bit, as unchained decode and takes every queued step; a step that is not the queued one, a cache call, or a change
    of how tokens are chosen drops it, and the cache is then exactly as if it had never run (its cell zeroed)."""
    V = TINY["n_vocab"]
    r = np.random.default_rng(31)
    lens = [17, 64, 40]  # slot 1's next cell starts a new page
    prompts = [r.integers(0, V, n).astype(np.int32) for n in lens]
    rows = np.arange(3, dtype=np.int32)
    seq = np.arange(3, dtype=np.int32)
    with S.Engine(tiny, slots=3, ctx=128, max_rows=64) as a, S.Engine(tiny, slots=3, ctx=128, max_rows=64) as b:
        for eng in (a, b):
            for s_, pr in enumerate(prompts):
                eng.step(pr, np.full(len(pr), s_, np.int32), np.arange(len(pr), dtype=np.int32),
                         np.array([len(pr) - 1], np.int32), n_write=0)
        cur = r.integers(0, V, 3).astype(np.int32)
        pos = np.array(lens, np.int32)

        def both(tok, chain=1):
            ta = a.step(tok, seq, pos, rows, chain=chain)
            tb = b.step(tok, seq, pos, rows)
            assert np.array_equal(ta, tb), (ta, tb)
            la, lb = a.logits(rows), b.logits(rows)
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
            return ta

        for it in range(8):  # chained decode: every step after the first is the queued one
            cur = both(cur).astype(np.int32)
            pos += 1
        assert a.chain_count() == (7, 0)
        assert b.chain_count() == (0, 0)

        def cell_zero(eng, slot, p):
            kv = eng.kv_save(slot, p + 1).reshape(-1, 2, p + 1, 256)  # [layers][K, V][cells][KV heads x 128]
            return not kv[:, :, p, :].any()

        # a step that is not the queued one (other tokens): the queued step is dropped, its cells zeroed
        cur = both((cur + 1) % V).astype(np.int32)
        assert a.chain_count() == (7, 1)
        pos += 1
        # a cache call drops the queued step (at pos), then the caches agree cell for cell
        a.clear(2, int(pos[2]) - 1, int(pos[2]))
        b.clear(2, int(pos[2]) - 1, int(pos[2]))
        assert a.chain_count() == (7, 2)
        for s_ in range(3):
            assert cell_zero(a, s_, int(pos[s_]))
            n = int(pos[s_]) - (1 if s_ == 2 else 0)
            assert np.array_equal(a.kv_save(s_, n), b.kv_save(s_, n)), s_
        pos[2] -= 1
        cur[2] = 5
        cur = both(cur).astype(np.int32)  # (not the queued one: nothing queued)
        pos += 1
        cur = both(cur).astype(np.int32)  # the queued one
        pos += 1
        assert a.chain_count() == (8, 2)
        a.want_probs(True)  # a change of how tokens are chosen: the queued step is not the one asked for
        b.want_probs(True)
        cur = both(cur).astype(np.int32)
        assert a.chain_count() == (8, 3)
        assert np.array_equal(a.probs(3), b.probs(3))
        pos += 1
        cur = both(cur, chain=0).astype(np.int32)  # taken, nothing queued after it
        assert a.chain_count() == (9, 3)
        pos += 1
        both(cur, chain=0)
        assert a.chain_count() == (9, 3)
    # a row at the context's last cell queues nothing
    with S.Engine(tiny, slots=1, ctx=64, max_rows=64) as a:
        a.step(prompts[0][:10], np.zeros(10, np.int32), np.arange(10, dtype=np.int32), np.array([9], np.int32), n_write=0)
        a.step(np.array([3], np.int32), np.zeros(1, np.int32), np.array([63], np.int32), np.zeros(1, np.int32), chain=1)
        assert a.chain_count() == (0, 0)
