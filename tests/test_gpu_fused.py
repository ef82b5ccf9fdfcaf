"""The matmul epilogues fused into decode-sized steps (q|k|v + QK-norm + RoPE + cache write; gate|up + SwiGLU + Q8_0;
the guess head's k|v + its cache write) against the split path (the matmul's k-slice sums, then the row kernel) on
the same engine inputs: logits, tokens and every cache cell bit for bit, with the workgroups of every fused launch on
the XCD the open-time probe predicted (snx_xcd_faults)."""
import numpy as np
import pytest

import sllm_next as S
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000)


def setup_module(module):
    U.torch().cuda.init()


def run(path, fuse, nextn):
    r = np.random.default_rng(21)
    slots, ctx = 8, 512
    out = []
    with S.Engine(path, slots=slots, ctx=ctx, max_rows=64) as eng:
        assert eng.fuse(fuse) == fuse
        if nextn:
            eng.guess_on(True)
        V = eng.V
        # prompt rows of 3 sequences in one step (below 256 rows: the decode-sized launches), outputs at their ends
        lens = [40, 9, 3]
        tok = r.integers(0, V, sum(lens)).astype(np.int32)
        seq = np.concatenate([np.full(n, s, np.int32) for s, n in enumerate(lens)])
        pos = np.concatenate([np.arange(n, dtype=np.int32) for n in lens])
        ends = np.cumsum(lens).astype(np.int32) - 1
        out.append(eng.step(tok, seq, pos, ends, n_write=0))
        out.append(eng.logits(np.arange(3, dtype=np.int32)))
        # decode steps of the 3 sequences, fed their own tokens
        cur, p = out[0].copy(), np.array(lens, np.int32)
        for _ in range(4):
            cur = eng.step(cur, np.arange(3, dtype=np.int32), p, np.arange(3, dtype=np.int32))
            out.append(cur.copy())
            out.append(eng.logits(np.arange(3, dtype=np.int32)))
            p += 1
        # a 4-row verify group of sequence 0
        vt = r.integers(0, V, 4).astype(np.int32)
        out.append(eng.step(vt, np.zeros(4, np.int32), np.arange(p[0], p[0] + 4, dtype=np.int32),
                            np.arange(4, dtype=np.int32)))
        out.append(eng.logits(np.arange(4, dtype=np.int32)))
        for s in range(3):
            out.append(eng.kv_save(s, int(p[s]) + (4 if s == 0 else 0)))
        assert eng.xcd_faults() == 0
    return out


@pytest.mark.parametrize("name,cfg", [
    ("tiny", TINY),
    ("qwen3-4b-width", dict(S.QWEN3_4B, n_layer=2)),
    ("qwen3-4b-width, guess head", dict(S.QWEN3_4B, n_layer=2, nextn=1)),
    ("q8_0 layers", dict(TINY, wtype=8)),
    ("qwen3-30b-a3b-width", dict(S.QWEN3_30B_A3B, n_layer=2)),
])
def test_fused_epilogues_equal_split_path(tmp_path, name, cfg):
    path = S.cached_model(cfg, 42) if cfg.get("n_embd", 0) > 1000 else str(tmp_path / "m.gguf")
    if cfg.get("n_embd", 0) <= 1000:
        S.write_model(path, S.model_cfg(**cfg), seed=31)
    fused = run(path, True, cfg.get("nextn", 0))
    split = run(path, False, cfg.get("nextn", 0))
    for i, (a, b) in enumerate(zip(fused, split)):
        assert a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8)), (name, i)
