"""The guess head (MTP) and the fused draft-verify step on the GPU.

Against the oracle (a Qwen3 model with one nextn block, written by snx_write_model): the head's guesses (sn_guess,
sn_cache.inc.h:300-388) and the fused step's drafts, verify targets and accepted lengths (next_engine/draft.rs:135-178,
take.rs:339-357), token for token wherever the oracle's top-2 gap exceeds the model's logit bound (the end-to-end
bound of test_gpu_engine.py; a sequence is followed only while every decision so far was clear of it).
Against the engine itself: guessing never changes the model's own logits (sn.h:115-122), and the fused step equals the
unfused path (sn_guess, one sn_step over the verify rows, host acceptance, sn_clear of the refused cells) bit for bit,
tokens and cache contents.
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000, nextn=1)
MODEL_ATOL = 3e-2
K = 3


def setup_module(module):
    U.torch().cuda.init()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "mtp.gguf")
    S.write_model(path, S.model_cfg(**TINY), seed=21)
    return path


def clear(lg, tok):
    i1, v1, i2, v2, _ = O.top2(lg)
    return i1 == tok and v1 - v2 > 2 * MODEL_ATOL


class Ref:
    """The oracle's model with the guess head's per-step cache fill and kept states (mtp_fill / mtp_keep)."""

    def __init__(self, path, n_seq, ctx):
        self.m = O.Qwen3(GGUF(path), n_seq=n_seq, ctx=ctx)
        self.pend = np.zeros((n_seq, self.m.E), np.float32)

    def step(self, tok, seq, pos, out_rows):
        R = len(tok)
        hn = np.zeros((R, self.m.E), np.float32)
        out, lg, _ = self.m.step(tok, seq, pos, out_rows, hn_all=hn)
        hprev = np.zeros_like(hn)
        for r in range(R):
            if r > 0 and seq[r] == seq[r - 1] and pos[r] == pos[r - 1] + 1:
                hprev[r] = hn[r - 1]
            elif pos[r] > 0:
                hprev[r] = self.pend[seq[r]]
        self.m.mtp_fill(tok, seq, pos, hprev)
        for r in range(R):
            if r + 1 == R or not (seq[r + 1] == seq[r] and pos[r + 1] == pos[r] + 1):
                self.pend[seq[r]] = hn[r]
        return out, lg, hn

    def cut(self, s, a, b):
        """cells [a, b) of slot s zeroed in every layer (the model's and the head's)"""
        self.m.k[s, :, a:b] = 0
        self.m.v[s, :, a:b] = 0


def prefill(eng, ref, prompts):
    tok = np.concatenate(prompts).astype(np.int32)
    seq = np.concatenate([np.full(len(p), s, np.int32) for s, p in enumerate(prompts)])
    pos = np.concatenate([np.arange(len(p), dtype=np.int32) for p in prompts])
    outs = np.cumsum([len(p) for p in prompts]).astype(np.int32) - 1
    got = eng.step(tok, seq, pos, outs, n_write=0)
    if ref is None:
        return got, None
    want, lg, _ = ref.step(tok, seq, pos, outs)
    return got, (want, lg)


def prompts(n, seed, lo=5, hi=12):
    r = np.random.default_rng(seed)
    return [r.integers(0, TINY["n_vocab"], int(r.integers(lo, hi))).astype(np.int32) for _ in range(n)]


def test_guessing_leaves_the_model_alone(model):
    ps = prompts(3, 1)
    out = []
    for on in (False, True):
        with S.Engine(model, slots=4, ctx=64, max_rows=64) as eng:
            assert eng.guess_head()
            assert eng.guess_on(on) == on
            t, _ = prefill(eng, None, ps)
            lg = eng.logits(np.arange(3))
            t2 = eng.step(t, np.arange(3, dtype=np.int32), np.array([len(p) for p in ps], np.int32),
                          np.arange(3, dtype=np.int32))
            out.append((t, t2, lg, eng.logits(np.arange(3))))
    for a, b in zip(out[0], out[1]):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.fixture(scope="module")
def model_q6k_tied(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "mtp_q6k.gguf")
    S.write_model(path, S.model_cfg(**TINY, embd_type=14, tied=1), seed=22)
    return path


@pytest.fixture(scope="module")
def model_q8(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "mtp_q8.gguf")
    S.write_model(path, S.model_cfg(**TINY, wtype=8), seed=23)
    return path


def test_guesses_match_oracle(model):
    guesses_match_oracle(model)


def test_guesses_match_oracle_q8_0(model_q8):
    """the guess head with Q8_0 matrices (its block, eh_proj and the LM head)"""
    guesses_match_oracle(model_q8)


def test_guesses_match_oracle_q6k_tied_head(model_q6k_tied):
    """the guess head through a Q6_K token table tied to the LM head (its Q8_K operand from the head norm's rows)"""
    guesses_match_oracle(model_q6k_tied)


def guesses_match_oracle(model):
    n_seq = 6
    ps = prompts(n_seq, 2)
    ref = Ref(model, n_seq, 64)
    checked = 0
    with S.Engine(model, slots=n_seq, ctx=64, max_rows=96) as eng:
        assert eng.guess_on(True)
        got, (want, lg) = prefill(eng, ref, ps)
        for s in range(n_seq):
            # both sides guess from the oracle's token (the prompt's own decision may sit inside the bound)
            pos = len(ps[s])
            g = eng.guess(s, want[s], pos, K)
            w, wl = ref.m.mtp_guess(s, want[s], pos, K, ref.pend[s])
            for j in range(K):
                if not clear(wl[j], w[j]):
                    break
                assert g[j] == w[j], (s, j, g, w)
                checked += 1
    print(f"guesses checked: {checked}")
    assert checked >= 2


def spec_unfused(eng, seqs, last, pos, k):
    """the reference's flow: sn_guess per sequence, one sn_step over all verify rows, host acceptance, sn_clear"""
    n = len(seqs)
    drafts = [eng.guess(s, last[i], pos[i], k) for i, s in enumerate(seqs)]
    tok = np.concatenate([[last[i]] + list(drafts[i]) for i in range(n)]).astype(np.int32)
    seq = np.repeat(np.asarray(seqs, np.int32), k + 1)
    ps = np.concatenate([np.arange(pos[i], pos[i] + k + 1) for i in range(n)]).astype(np.int32)
    rows = np.arange(n * (k + 1), dtype=np.int32)
    tgt = eng.step(tok, seq, ps, rows, n_write=0).reshape(n, k + 1)
    out_n = np.zeros(n, np.int32)
    out_tok = np.full((n, k + 1), -1, np.int32)
    for i, s in enumerate(seqs):
        a = int(O.accept(drafts[i], tgt[i, :k]))
        out_tok[i, :a] = drafts[i][:a]
        out_tok[i, a] = tgt[i, a]
        out_n[i] = a + 1
        eng.clear(s, pos[i] + a + 1, pos[i] + k + 1)
    return out_n, out_tok


def test_fused_step_equals_unfused(model):
    ps = prompts(3, 3)
    res = []
    for fused in (True, False):
        with S.Engine(model, slots=4, ctx=64, max_rows=64) as eng:
            eng.guess_on(True)
            last, _ = prefill(eng, None, ps)
            pos = np.array([len(p) for p in ps], np.int32)
            seqs = np.arange(3, dtype=np.int32)
            trace = []
            for _ in range(4):
                if fused:
                    n, t = eng.spec_step(seqs, last, pos, K)
                else:
                    n, t = spec_unfused(eng, seqs, last, pos, K)
                trace.append((n.copy(), t.copy()))
                last = t[np.arange(3), n - 1].astype(np.int32)
                pos = pos + n
            kv = [eng.kv_save(s, int(pos[s])) for s in range(3)]
            res.append((trace, kv))
    (ta, kva), (tb, kvb) = res
    for (na, xa), (nb, xb) in zip(ta, tb):
        assert np.array_equal(na, nb) and np.array_equal(xa, xb), (na, nb, xa, xb)
    for a, b in zip(kva, kvb):
        assert np.array_equal(a, b)


def test_fused_step_graph_replay_equals_eager(model):
    """The fused step's device work is captured as a HIP graph per shape (sequences, drafts, attention work-list
    sizes, staging offsets) and replayed while the shape repeats: replays, and recaptures when a sequence's rows cross
    a 256-cell chunk, give the tokens, accepted lengths and cache cells of eager launches, bit for bit."""
    ps = prompts(4, 7)
    res = []
    for graphs in (True, False):
        with S.Engine(model, slots=4, ctx=640, max_rows=64) as eng:
            eng.graphs(graphs)
            eng.guess_on(True)
            last, _ = prefill(eng, None, ps)
            pos = np.array([len(p) for p in ps], np.int32)
            seqs = np.arange(4, dtype=np.int32)
            for s in range(4):  # contexts just short of the 256-cell chunk boundary
                eng.fill_kv(s, 250 + 2 * s, seed=3)
            pos = np.array([250 + 2 * s for s in range(4)], np.int32)
            rf = np.random.default_rng(4)
            trace = []
            for _ in range(8):
                force = (rf.random((4, K)) < 0.6).astype(np.uint8)
                n, t = eng.spec_step(seqs, last, pos, K, force=force)
                trace.append((n.copy(), t.copy()))
                last = t[np.arange(4), n - 1].astype(np.int32)
                pos = pos + n
            kv = [eng.kv_save(s, int(pos[s])) for s in range(4)]
            res.append((trace, kv, eng.graph_count()))
    (ta, kva, ga), (tb, kvb, gb) = res
    for (na, xa), (nb, xb) in zip(ta, tb):
        assert np.array_equal(na, nb) and np.array_equal(xa, xb), (na, nb, xa, xb)
    for a, b in zip(kva, kvb):
        assert np.array_equal(a, b)
    assert ga[1] >= 2 and ga[0] >= 2, ga  # replays, and recaptures at the chunk crossings
    assert gb == (0, 0)


@pytest.mark.parametrize("which", ["model", "model_q6k_tied"])
def test_fused_step_matches_oracle(request, which):
    model = request.getfixturevalue(which)
    n_seq, steps = 4, 5
    ps = prompts(n_seq, 4)
    ref = Ref(model, n_seq, 64)
    rng = np.random.default_rng(5)
    stats = {"decisions": 0, "accepted": 0}
    with S.Engine(model, slots=n_seq, ctx=64, max_rows=64) as eng:
        eng.guess_on(True)
        got, (want, lg) = prefill(eng, ref, ps)
        alive = [True] * n_seq  # both sides go on from the oracle's token
        last = want.astype(np.int32)
        pos = np.array([len(p) for p in ps], np.int32)
        seqs = np.arange(n_seq, dtype=np.int32)
        for _ in range(steps):
            force = (rng.random((n_seq, K)) < 0.6).astype(np.uint8)
            n, t = eng.spec_step(seqs, last, pos, K, force=force)
            for s in range(n_seq):
                # the oracle's drafts, verify rows (forced drafts win their row's argmax), acceptance and cut
                d, dl = ref.m.mtp_guess(s, last[s], pos[s], K, ref.pend[s])
                tok = np.array([last[s]] + list(d), np.int32)
                sq = np.full(K + 1, s, np.int32)
                pp = np.arange(pos[s], pos[s] + K + 1, dtype=np.int32)
                _, vl, hn = ref.step(tok, sq, pp, np.arange(K + 1, dtype=np.int32))
                for i in range(K):
                    if force[s, i]:
                        vl[i, d[i]] = 3.0e38
                tg = np.array([O.argmax(vl[i]) for i in range(K + 1)], np.int32)
                a = int(O.accept(d, tg[:K]))
                ref.cut(s, pos[s] + a + 1, pos[s] + K + 1)
                ref.pend[s] = hn[a]
                # equal results, or a decision inside the bound (then the sequence is no longer followed)
                if alive[s]:
                    same = n[s] == a + 1 and list(t[s, :a + 1]) == list(d[:a]) + [tg[a]]
                    sure = all(clear(dl[j], d[j]) for j in range(min(a + 1, K)))
                    sure = sure and all((i < K and force[s, i]) or clear(vl[i], tg[i]) for i in range(a + 1))
                    assert same or not sure, (s, n[s], t[s], a, d, tg)
                    if same:
                        stats["decisions"] += 1
                        stats["accepted"] += a
                    alive[s] = same
                last[s] = tg[a]
                pos[s] += a + 1
    print(f"spec steps compared: {stats}")
    assert stats["decisions"] >= 8
