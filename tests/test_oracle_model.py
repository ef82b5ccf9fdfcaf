"""The oracle's composed functions pinned on the CPU: or_qwen3_step (dense and MoE layers, the output stage),
or_mtp_fill and or_mtp_guess against tests/ref64.py, a numpy restatement of the step written from the reference's
lines (qwen_layers sn_attn.inc.h:216-231, moe_ffn sn_layers.inc.h:129-144, outputs sn_encode.inc.h:304-317, guess_row
sn_cache.inc.h:357-369, mtp_fill sn_state.inc.h:283-313), not from oracle.c. It keeps ggml's arithmetic operation by
operation (Q8_0 matmul inputs and ggml's block-sum order, fp16 cells, the norms' fp32 steps, RoPE angles and the C
library's expf / cosf / sinf), so every logit, token, normed row and cache cell must equal the oracle's bit for bit:
a difference is a difference in what is computed (a layer order, a norm weight, a rotation pair, a routing weight, the
guess head's input halves), never rounding noise.

Invariants that a plausible mistake (a dropped renormalisation, a swapped half of the guess head's input) fails:
  * a MoE layer whose experts are all one expert is the dense FFN of that expert (the routing weights sum to 1);
  * a guess head whose eh_proj ignores the hidden-state half (those blocks' scales zero) guesses the same whatever the
    hidden state it is given, while the real head does not.
"""
import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF, TYPES
from tests import ref64

TINY = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, n_ff=512, n_vocab=600)
TINY_MOE = dict(TINY, n_expert=8, n_expert_used=3, n_ff_exp=128)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_rows(name, lg_o, tok_o, lg_r):
    assert np.array_equal(bits(lg_o), bits(lg_r)), (name, float(np.abs(lg_o - lg_r).max()))
    assert np.array_equal(tok_o, lg_r.argmax(-1)), name


def same_cells(oracle, kv, seq, pos, layers):
    """the oracle's fp16 cells against the restatement's, bit for bit"""
    for s, p in zip(seq, pos):
        for l in layers:
            k_r, v_r = kv[(int(s), l)][int(p)]
            for got, want in ((oracle.k[s, l, p], k_r), (oracle.v[s, l, p], v_r)):
                assert np.array_equal(got.view(np.float16).astype(np.float64).reshape(want.shape), want), (s, p, l)


def rows(prompts):
    tok = np.concatenate(prompts).astype(np.int32)
    seq = np.concatenate([np.full(len(p), s, np.int32) for s, p in enumerate(prompts)])
    pos = np.concatenate([np.arange(len(p), dtype=np.int32) for p in prompts])
    outs = np.cumsum([len(p) for p in prompts]).astype(np.int32) - 1
    return tok, seq, pos, outs


@pytest.mark.parametrize("cfg,wtype", [(TINY, 2), (TINY, 8), (TINY_MOE, 2), (TINY_MOE, 8)],
                         ids=["dense-q4", "dense-q8", "moe-q4", "moe-q8"])
def test_step_matches_restatement(tmp_path, cfg, wtype):
    path = str(tmp_path / "m.gguf")
    S.write_model(path, S.model_cfg(**cfg, wtype=wtype), seed=31)
    g = GGUF(path)
    orc, ref = O.Qwen3(g, n_seq=2, ctx=32), ref64.Model(g)
    kv = {}
    r = np.random.default_rng(3)
    tok, seq, pos, outs = rows([r.integers(0, cfg["n_vocab"], 9), r.integers(0, cfg["n_vocab"], 6)])
    allr = np.arange(len(tok), dtype=np.int32)  # every prompt row an output row: every row's logits compared
    hn_o = np.zeros((len(tok), ref.E), np.float32)
    to, lo, _ = orc.step(tok, seq, pos, allr, hn_all=hn_o)
    _, lr, hn_r = ref.step(kv, tok, seq, pos, allr)
    same_rows("prompt rows", lo, to, lr)
    assert np.array_equal(bits(hn_o), bits(hn_r))
    same_cells(orc, kv, seq, pos, range(ref.L))
    cur, p = to[outs].astype(np.int32), np.array([9, 6], np.int32)
    for _ in range(3):  # decode steps of both sequences
        s2 = np.array([0, 1], np.int32)
        to, lo, _ = orc.step(cur, s2, p, s2)
        _, lr, _ = ref.step(kv, cur, s2, p, s2)
        same_rows("decode rows", lo, to, lr)
        same_cells(orc, kv, s2, p, range(ref.L))
        cur, p = to.astype(np.int32), p + 1


def test_guess_head_matches_restatement(tmp_path):
    path = str(tmp_path / "mtp.gguf")
    S.write_model(path, S.model_cfg(**TINY, nextn=1), seed=32)
    g = GGUF(path)
    orc, ref = O.Qwen3(g, n_seq=1, ctx=32), ref64.Model(g)
    kv = {}
    r = np.random.default_rng(4)
    tok, seq, pos, outs = rows([r.integers(0, TINY["n_vocab"], 10)])
    hn = np.zeros((len(tok), ref.E), np.float32)
    t_o, _, _ = orc.step(tok, seq, pos, outs, hn_all=hn)
    ref.step(kv, tok, seq, pos, outs)
    # the head's cells of the prompt rows: row r paired with the row before's normed state (zeros at position 0)
    hprev = np.concatenate([np.zeros((1, ref.E), np.float32), hn[:-1]])
    orc.mtp_fill(tok, seq, pos, hprev)
    ref.mtp_fill(kv, tok, seq, pos, hprev)
    same_cells(orc, kv, seq, pos, [ref.L])
    t0 = int(t_o[0])
    for start in (10, 13):  # two rounds of 3 guesses, the second attending over the first's cells
        guess_o, lg_o = orc.mtp_guess(0, t0, start, 3, hn[-1])
        guess_r, lg_r = ref.mtp_guess(kv, 0, t0, start, 3, hn[-1])
        same_rows("guesses", lg_o, guess_o, lg_r)
        same_cells(orc, kv, [0, 0, 0], [start, start + 1, start + 2], [ref.L])
        t0 = int(guess_o[-1])


# ---- invariants on models built from a written one, tensors replaced ----
class Patched:
    """a GGUF reader over another one with some tensors replaced (name: (type name, ne, rows)) and keys changed"""

    def __init__(self, base, tensors=None, kv=None, drop=()):
        self.base = base
        self.kv = {k: v for k, v in base.kv.items() if k not in drop}
        self.kv.update(kv or {})
        self.over = dict(tensors or {})
        codes = {v[0]: k for k, v in TYPES.items()}
        self.tinfo = dict(base.tinfo)
        for n, (tn, ne, _) in self.over.items():
            self.tinfo[n] = (ne, codes[tn], 0)

    def tensor(self, name):
        return self.over[name][2] if name in self.over else self.base.tensor(name)

    def type_name(self, name):
        return self.over[name][0] if name in self.over else self.base.type_name(name)


def test_identical_experts_equal_the_dense_ffn(tmp_path):
    path = str(tmp_path / "moe.gguf")
    S.write_model(path, S.model_cfg(**TINY_MOE), seed=33)
    g = GGUF(path)
    E, NE, FE = TINY_MOE["n_embd"], TINY_MOE["n_expert"], TINY_MOE["n_ff_exp"]
    same, dense = {}, {}
    for i in range(TINY_MOE["n_layer"]):
        for part, ne in (("gate", [E, FE]), ("up", [E, FE]), ("down", [FE, E])):
            x0 = np.ascontiguousarray(g.tensor(f"blk.{i}.ffn_{part}_exps.weight")[0])
            same[f"blk.{i}.ffn_{part}_exps.weight"] = ("Q4_0", ne + [NE], np.ascontiguousarray(
                np.broadcast_to(x0, (NE,) + x0.shape)))
            dense[f"blk.{i}.ffn_{part}.weight"] = ("Q4_0", ne, x0)
    moe_same = O.Qwen3(Patched(g, same), n_seq=1, ctx=32)
    a = "qwen3moe"
    ffn = O.Qwen3(Patched(g, dense, kv={f"{a}.feed_forward_length": FE},
                          drop=(f"{a}.expert_count", f"{a}.expert_used_count")), n_seq=1, ctx=32)
    assert moe_same.NE == NE and ffn.NE == 0
    r = np.random.default_rng(5)
    tok, seq, pos, outs = rows([r.integers(0, TINY_MOE["n_vocab"], 12)])
    t1, l1, _ = moe_same.step(tok, seq, pos, np.arange(12, dtype=np.int32))
    t2, l2, _ = ffn.step(tok, seq, pos, np.arange(12, dtype=np.int32))
    # the weights of one expert's k copies sum to 1 within an fp32 rounding, so the rows may part by a flipped
    # Q8_0 rounding at most; here they are bit for bit the same
    assert np.array_equal(bits(l1), bits(l2)), float(np.abs(l1 - l2).max())
    # and the real experts are not that FFN
    real = O.Qwen3(g, n_seq=1, ctx=32)
    _, l3, _ = real.step(tok, seq, pos, np.arange(12, dtype=np.int32))
    assert np.abs(l3 - l2).max() > 0.1 * np.abs(l2).max()


def test_guess_ignores_the_hidden_state_when_eh_proj_does(tmp_path):
    path = str(tmp_path / "mtp.gguf")
    S.write_model(path, S.model_cfg(**TINY, nextn=1), seed=34)
    g = GGUF(path)
    E = TINY["n_embd"]
    name = f"blk.{TINY['n_layer']}.nextn.eh_proj.weight"
    eh = np.array(g.tensor(name))  # [E][2E / 32 * 18] Q4_0 rows
    blocks = eh.reshape(E, 2 * E // 32, 18)
    blocks[:, E // 32:, :2] = 0  # the hidden-state half's scales: those blocks are zero whatever their nibbles
    r = np.random.default_rng(6)
    ha, hb = r.normal(0, 1, E).astype(np.float32), r.normal(0, 1, E).astype(np.float32)
    outs = []
    for gg in (Patched(g, {name: ("Q4_0", [2 * E, E], blocks.reshape(E, -1))}), g):
        m = O.Qwen3(gg, n_seq=1, ctx=32)
        res = [m.mtp_guess(0, 7, 4, 3, h) for h in (ha, hb)]
        outs.append(res)
    (ga, la), (gb, lb) = outs[0]
    assert np.array_equal(ga, gb) and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    (_, ra), (_, rb) = outs[1]
    assert np.abs(ra - rb).max() > 1e-3  # the real head does read the hidden state
