"""Qwen3-MoE layers on the GPU (moe_ffn, sn_layers.inc.h:129-144; moe_topk1 / moe_lists / qmm_grouped / moe_out,
kernels.metal:3419-3538) against the oracle's MoE step (softmax -> top-k with ties to the lower id -> renormalised
weights, Q4_0 expert matmuls with ggml's Q8_0 activations, the weighted sum in slot order): greedy tokens wherever the
oracle's top-2 gap exceeds the model's logit bound. A row's expert grouping depends on the other rows of the step (which
rows share an expert, where its tile falls); its logits must not: row invariance is checked bit for bit.
"""
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
