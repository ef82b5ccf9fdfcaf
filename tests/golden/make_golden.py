#!/usr/bin/env python3
"""Writes the small fixtures under tests/golden/ (run from the repository root: python tests/golden/make_golden.py).

Vectors from the oracle (oracle/oracle.c, a CPU restatement of ggml's semantics for this path) on seeded inputs:
  q4_0_64x256.npz     fp32 W [64][256] ~N(0, 0.02) (seed 1), its Q4_0 blocks, their dequantized values
  mm_q4_0_8x256.npz   X [8][256] ~N(0, 1), Q8_0(X) blocks, Y = X W^T (ggml integer block dots) and Y in fp64
  paged_attn_2seq.npz a 2-sequence GQA decode case over 32-cell pages: pool, page table, q, outputs fp32 and fp64
  tiny_qwen3_trace.json  a 2-layer Qwen3 (snx_write_model, seed 7): a 6-token prompt and 4 greedy steps per sequence
                      for 2 sequences: tokens, top-2 logits and their gap per step
  accept_table.json   greedy acceptance (draft vs target argmax) on every case of k = 0..3 over a 3-token alphabet
and one extracted from the reference's own test data when /root/reference is present:
  gguf_qwen3_layout.json  engine/sllm-core/tests/fixtures/gguf_py_qwen3-0.6b-Q4_0.json reduced to its model keys and
                      the tensors of the output, the embedding and block 0 (names, ne order, ggml types)
The fixtures are regression vectors: the oracle's correctness is pinned separately (tests/test_oracle.py), these freeze
its outputs and give the GPU tests fixed inputs.
"""
import itertools
import json
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (ROOT, os.path.join(ROOT, "sonic-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import oracle as O  # noqa: E402
from oracle.gguf import GGUF  # noqa: E402

HERE = os.path.join(ROOT, "tests", "golden")
REF_LAYOUT = "/root/reference/engine/sllm-core/tests/fixtures/gguf_py_qwen3-0.6b-Q4_0.json"
TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000)
TINY_SEED = 7


def q4():
    w = np.random.default_rng(1).normal(0, 0.02, (64, 256)).astype(np.float32)
    blocks = O.quantize_q4_0(w)
    deq = O.dequantize_q4_0(blocks, 256)
    np.savez_compressed(os.path.join(HERE, "q4_0_64x256.npz"), w=w, blocks=blocks, deq=deq)
    x = np.random.default_rng(2).normal(0, 1, (8, 256)).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "mm_q4_0_8x256.npz"), x=x, xq=O.quantize_q8_0(x),
                        y=O.mul_mat_q4_0(blocks, 256, x), y64=O.mul_mat_q4_0_f64(blocks, 256, x))


def attn():
    r = np.random.default_rng(3)
    H, KVH, D, pc = 8, 2, 128, 32
    ctx = np.array([70, 129], np.int32)  # ragged: a partial last page each
    n_pages = int(sum((c + pc - 1) // pc for c in ctx)) + 2
    perm = r.permutation(n_pages).astype(np.int32)
    max_pages = int(max((c + pc - 1) // pc for c in ctx))
    pt = np.full((2, max_pages), -1, np.int32)
    k = 0
    for s, c in enumerate(ctx):
        for j in range((c + pc - 1) // pc):
            pt[s, j] = perm[k]
            k += 1
    kpool = O.f32_to_f16_bits(r.normal(0, 1, (n_pages, KVH, pc, D)).astype(np.float32))
    vpool = O.f32_to_f16_bits(r.normal(0, 1, (n_pages, KVH, pc, D)).astype(np.float32))
    # decode rows at the last cell of each sequence plus two verify rows of sequence 1
    qseq = np.array([0, 1, 1, 1], np.int32)
    qpos = np.array([ctx[0] - 1, ctx[1] - 3, ctx[1] - 2, ctx[1] - 1], np.int32)
    q = r.normal(0, 1, (4, H, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    out = O.paged_attn(q, qseq, qpos, KVH, kpool, vpool, pc, pt, scale)
    out64 = O.paged_attn(q, qseq, qpos, KVH, kpool, vpool, pc, pt, scale, f64=True)
    np.savez_compressed(os.path.join(HERE, "paged_attn_2seq.npz"), q=q, qseq=qseq, qpos=qpos, kpool=kpool,
                        vpool=vpool, pt=pt, page_cells=np.int32(pc), kv_heads=np.int32(KVH), scale=np.float32(scale),
                        out=out, out64=out64)


def tiny_trace():
    import sllm_next as S
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        S.write_model(path, S.model_cfg(**TINY), seed=TINY_SEED)
        ref = O.Qwen3(GGUF(path), n_seq=2, ctx=64)
        prompt = np.random.default_rng(4).integers(0, TINY["n_vocab"], (2, 6)).astype(np.int32)
        steps = []
        tok = np.concatenate([prompt[0], prompt[1]])
        seq = np.repeat(np.arange(2, dtype=np.int32), 6)
        pos = np.tile(np.arange(6, dtype=np.int32), 2)
        out_rows = np.array([5, 11], np.int32)
        p = 6
        for _ in range(5):
            t, lg, _ = ref.step(tok, seq, pos, out_rows)
            rec = []
            for j in range(2):
                i1, v1, i2, v2, _ = O.top2(lg[j])
                rec.append({"token": int(t[j]), "top1": [int(i1), float(v1)], "top2": [int(i2), float(v2)],
                            "gap": float(v1 - v2)})
            steps.append(rec)
            tok, seq, pos, out_rows = t.astype(np.int32), np.arange(2, dtype=np.int32), np.full(2, p, np.int32), \
                np.arange(2, dtype=np.int32)
            p += 1
        json.dump({"model": dict(TINY, seed=TINY_SEED), "prompt": prompt.tolist(), "steps": steps},
                  open(os.path.join(HERE, "tiny_qwen3_trace.json"), "w"), indent=1)


def accept_table():
    rows = []
    for k in range(4):
        for draft in itertools.product(range(3), repeat=k):
            for target in itertools.product(range(3), repeat=k + 1):
                rows.append([list(draft), list(target), O.accept(np.array(draft, np.int32),
                                                                 np.array(target[:k], np.int32))])
    json.dump({"rule": "accepted = length of the common prefix of draft[0..k) and target[0..k); the bonus token is "
                       "target[accepted]", "cases": rows}, open(os.path.join(HERE, "accept_table.json"), "w"))


def layout():
    if not os.path.exists(REF_LAYOUT):
        print("reference tree absent: gguf_qwen3_layout.json left as it is")
        return
    d = json.load(open(REF_LAYOUT))
    keep = [t for t in d["tensors"] if not t["name"].startswith("blk.") or t["name"].startswith("blk.0.")]
    kv = {k: v for k, v in d["kv"].items() if k.startswith("qwen3.") or k == "general.architecture"}
    json.dump({"source": "engine/sllm-core/tests/fixtures/gguf_py_qwen3-0.6b-Q4_0.json (reduced)",
               "alignment": d["alignment"], "n_tensors": d["n_tensors"], "kv": kv,
               "tensors": [{k: t[k] for k in ("name", "ne", "type")} for t in keep]},
              open(os.path.join(HERE, "gguf_qwen3_layout.json"), "w"), indent=1)


if __name__ == "__main__":
    O.build() if not os.path.exists(O.LIB_PATH) else None
    q4()
    attn()
    tiny_trace()
    accept_table()
    layout()
    print("written:", sorted(os.listdir(HERE)))
