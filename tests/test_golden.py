"""The committed fixtures under tests/golden/ (written by tests/golden/make_golden.py) on the CPU: the oracle reproduces
them, the package's own quantizer and model writer agree with them, and independent brute-force checks hold on the
fixture data (fp64 dense attention, a pure-Python acceptance rule)."""
import json
import os

import numpy as np
import pytest

import sllm_next as S
from oracle import oracle as O
from oracle.gguf import GGUF

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def test_q4_0_fixture():
    f = load("q4_0_64x256.npz")
    assert np.array_equal(O.quantize_q4_0(f["w"]), f["blocks"])
    assert np.array_equal(O.dequantize_q4_0(f["blocks"], 256).view(np.uint32), f["deq"].view(np.uint32))
    # the quantizer the model writer uses (sonic-llm_amd/csrc/synth.cpp) gives the same bytes
    assert np.array_equal(S.quantize_q4_0(f["w"]).reshape(f["blocks"].shape), f["blocks"])
    # closed form on the fixture bytes: w = d * (q - 8), q[j] = low nibble of byte j, q[j+16] = high nibble
    b = f["blocks"].reshape(64, 8, 18)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
    qs = b[:, :, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=2).astype(np.float32)
    assert np.array_equal((d * (q - 8)).reshape(64, 256), f["deq"])


def test_q4_0_matmul_fixture():
    f = load("mm_q4_0_8x256.npz")
    g = load("q4_0_64x256.npz")
    assert np.array_equal(O.quantize_q8_0(f["x"]), f["xq"])
    y = O.mul_mat_q4_0(g["blocks"], 256, f["x"])
    assert np.array_equal(y.view(np.uint32), f["y"].view(np.uint32))
    ref = f["x"].astype(np.float64) @ g["deq"].astype(np.float64).T  # unquantized activations
    np.testing.assert_allclose(f["y64"], ref, rtol=1e-12, atol=1e-12)
    # ggml's product is exact up to fp32 summation over the Q8_0-rounded activations
    xq = O.dequantize_q8_0(f["xq"], 256).astype(np.float64)
    np.testing.assert_allclose(f["y"], xq @ g["deq"].astype(np.float64).T, rtol=1e-5, atol=1e-6)
    assert np.abs(f["y"] - f["y64"]).max() < 2e-2  # what the Q8_0 rounding of X moves


def test_paged_attn_fixture():
    f = load("paged_attn_2seq.npz")
    pc, KVH = int(f["page_cells"]), int(f["kv_heads"])
    args = (f["q"], f["qseq"], f["qpos"], KVH, f["kpool"], f["vpool"], pc, f["pt"], float(f["scale"]))
    assert np.array_equal(O.paged_attn(*args).view(np.uint32), f["out"].view(np.uint32))
    # independent fp64 dense restatement over the page-gathered cells
    kp = f["kpool"].view(np.float16).astype(np.float64)
    vp = f["vpool"].view(np.float16).astype(np.float64)
    q = f["q"].astype(np.float64)
    H = q.shape[1]
    out = np.zeros_like(q)
    for i, (s, p) in enumerate(zip(f["qseq"], f["qpos"])):
        cells = np.arange(p + 1)
        pages = f["pt"][s, cells // pc]
        assert (pages >= 0).all()
        for h in range(H):
            kh = h // (H // KVH)
            K = kp[pages, kh, cells % pc]
            V = vp[pages, kh, cells % pc]
            sc = K @ (q[i, h] * float(f["scale"]))
            w = np.exp(sc - sc.max())
            out[i, h] = (w / w.sum()) @ V
    np.testing.assert_allclose(f["out64"], out, rtol=1e-6, atol=1e-7)  # fp64 math, stored as fp32
    np.testing.assert_allclose(f["out"], out, rtol=1e-3, atol=2e-3)


def test_tiny_qwen3_trace(tmp_path):
    t = json.load(open(os.path.join(G, "tiny_qwen3_trace.json")))
    m = dict(t["model"])
    seed = m.pop("seed")
    path = str(tmp_path / "tiny.gguf")
    S.write_model(path, S.model_cfg(**m), seed=seed)
    ref = O.Qwen3(GGUF(path), n_seq=2, ctx=64)
    prompt = np.array(t["prompt"], np.int32)
    tok = prompt.reshape(-1)
    seq = np.repeat(np.arange(2, dtype=np.int32), prompt.shape[1])
    pos = np.tile(np.arange(prompt.shape[1], dtype=np.int32), 2)
    out_rows = np.array([prompt.shape[1] - 1, 2 * prompt.shape[1] - 1], np.int32)
    p = prompt.shape[1]
    for rec in t["steps"]:
        got, lg, _ = ref.step(tok, seq, pos, out_rows)
        for j in range(2):
            i1, v1, i2, v2, _ = O.top2(lg[j])
            assert int(got[j]) == rec[j]["token"] == i1
            assert i2 == rec[j]["top2"][0]
            assert abs(v1 - rec[j]["top1"][1]) < 1e-6 and abs(v2 - rec[j]["top2"][1]) < 1e-6
        tok, seq = got.astype(np.int32), np.arange(2, dtype=np.int32)
        pos, out_rows = np.full(2, p, np.int32), np.arange(2, dtype=np.int32)
        p += 1


def test_accept_table():
    t = json.load(open(os.path.join(G, "accept_table.json")))
    assert len(t["cases"]) == sum(3 ** k * 3 ** (k + 1) for k in range(4))
    for draft, target, n in t["cases"]:
        k = len(draft)
        brute = next((i for i in range(k) if draft[i] != target[i]), k)
        assert n == brute
        assert O.accept(np.array(draft, np.int32), np.array(target[:k], np.int32)) == n


def test_writer_layout_matches_reference_gguf(tmp_path):
    """Tensor names, ne order ([K, M]: the row length first), ggml types and model keys of the model writer against the
    reference's Qwen3-0.6B-Q4_0 GGUF table (one block at that model's dims; vocabulary cut to 512). The writer's
    token_embd is F32 and it writes an untied Q4_0 `output.weight`, where that file has a Q6_K embedding tied to the
    head: the engine serves the untied layout the benchmark configs name."""
    ref = json.load(open(os.path.join(G, "gguf_qwen3_layout.json")))
    kv = ref["kv"]
    E, H, KVH = kv["qwen3.embedding_length"], kv["qwen3.attention.head_count"], kv["qwen3.attention.head_count_kv"]
    F = kv["qwen3.feed_forward_length"]
    path = str(tmp_path / "m.gguf")
    S.write_model(path, S.model_cfg(n_layer=1, n_embd=E, n_head=H, n_head_kv=KVH, n_ff=F, n_vocab=512), seed=1)
    g = GGUF(path)
    for k, v in kv.items():
        if k in ("qwen3.block_count", "qwen3.context_length"):
            continue
        assert k in g.kv, k
        if isinstance(v, float):
            assert abs(float(g.kv[k]) - v) <= 1e-6 * max(1.0, abs(v)), k
        else:
            assert g.kv[k] == v, k
    from oracle.gguf import TYPES
    ours = {n: ([int(x) for x in ne] + [1] * (4 - len(ne)), TYPES[t][0]) for n, (ne, t, _) in g.tinfo.items()}
    for t in ref["tensors"]:
        name = t["name"]
        if name == "token_embd.weight":
            assert ours[name][0][0] == E and ours[name][1] == "F32"
            continue
        ne = [512 if x == 151936 else x for x in t["ne"]]
        assert name in ours, name
        assert ours[name] == (ne, t["type"]), (name, ours[name], ne, t["type"])
    assert ours["output.weight"] == ([E, 512, 1, 1], "Q4_0")
