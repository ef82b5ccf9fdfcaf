#!/usr/bin/env python3
"""Headline benchmark: aggregate decode tokens/s of the batched decode step (sn_step) on one MI355X.

Workload: a Qwen3-4B-architecture dense model, random init (seeded N(0, 0.02) weights
quantized to Q4_0 with ggml's reference quantizer; fp32 embedding and norms; untied Q4_0 LM head), 32 sequences whose
2048-cell contexts are already in the paged fp16 KV cache (seeded N(0, 1) cells: a step costs the same whatever they
hold), one new token per sequence per step, greedy argmax fed back as the next token. A step is one sn_step call of 32
rows: inputs resident on the GPU, one host round trip (the 32 tokens back).

Output: one JSON line. `value` = 32 * steps / wall time of the timed steps. `roofline` is the kernel class that takes
the most GPU time in a separate profiled pass of the same steps (HIP events around every launch on the engine's
stream), its algorithmic bytes / time against 8 TB/s; `roofline_gemm` is the Q4_0 matmul's (the metric's "Q4_0 GEMV %
HBM peak"). `cpu_baseline` times the oracle (oracle/, a C restatement of ggml's CPU semantics) on the host cores for
one step of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "sonic-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def model_file(cfg_kw, seed, path=None):
    import sllm_next as S
    d = os.environ.get("SN_BENCH_DIR") or "/tmp"
    tag = ("_mtp" if cfg_kw.get("nextn") else "") + (f"_moe{cfg_kw['n_expert']}" if cfg_kw.get("n_expert") else "") + \
          ("_q8" if cfg_kw.get("wtype") == 8 else "") + ("_q6kt" if cfg_kw.get("tied") else "")
    path = path or os.path.join(d, f"sonic_qwen3_{cfg_kw['n_layer']}L_{cfg_kw['n_embd']}{tag}_{seed}.gguf")
    done = path + ".done"
    if not (os.path.exists(path) and os.path.exists(done)):
        t = time.time()
        S.write_model(path, S.model_cfg(**cfg_kw), seed, nthreads=int(os.environ.get("OMP_NUM_THREADS", "0") or 0))
        open(done, "w").write("ok")
        log(f"[bench] wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    return path


def cpu_baseline(path, seqs, ctx, seed):
    """The oracle's step for the same rows on the host cores: one step of `seqs` rows at position ctx (its KV cells are
    zeros: the cost of a step does not depend on what they hold)."""
    import numpy as np

    from oracle import oracle as O
    from oracle.gguf import GGUF

    O.build() if not os.path.exists(O.LIB_PATH) else None
    ref = O.Qwen3(GGUF(path), n_seq=seqs, ctx=ctx + 1)
    r = np.random.default_rng(seed)
    tok = r.integers(0, ref.V, seqs).astype(np.int32)
    seq = np.arange(seqs, dtype=np.int32)
    pos = np.full(seqs, ctx, np.int32)
    ref.k[:, :, :ctx] = 0  # touch the cells the step reads before timing
    ref.v[:, :, :ctx] = 0
    t = time.perf_counter()
    ref.step(tok, seq, pos, seq)
    dt = time.perf_counter() - t
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count())
    return {"value": seqs / dt, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"one decode step of the full workload ({seqs} rows at position {ctx}, all layers and the LM "
                      f"head) through oracle/oracle.c (ggml-semantics CPU restatement: Q8_0 activations, integer block "
                      f"dots, fp32 attention over fp16 cells; ggml b11669 itself is not available offline), "
                      f"{dt:.1f} s on {cores} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seqs", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--prof-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--model", default=None, help="GGUF path (generated when missing)")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--config", default="decode", choices=("decode", "mtp", "moe"),
                    help="decode: the headline (configs[2]); mtp: the fused draft-verify step (configs[3]); "
                         "moe: Qwen3-30B-A3B-arch batched decode (configs[4])")
    ap.add_argument("--accept", type=float, default=0.6, help="mtp: the seeded share of drafts forced to match")
    ap.add_argument("--no-graphs", action="store_true", help="launch every step eagerly (no HIP graph replay)")
    ap.add_argument("--no-chain", action="store_true", help="decode without sn_step's queued successor (chain = 0)")
    ap.add_argument("--attn-mode", type=int, default=-1, choices=(-1, 0, 1),
                    help="attention work list: -1 chosen per step, 0 per-chunk + merge, 1 whole groups")
    ap.add_argument("--wtype", type=int, default=2, choices=(2, 8),
                    help="decode / moe: the model's matrices in Q4_0 (2, the configs) or Q8_0 (8)")
    ap.add_argument("--table", default="f32", choices=("f32", "q6k-tied"),
                    help="decode: an F32 token table and an untied head of the matrices' type (the configs), or a "
                         "Q6_K token table tied to the LM head (the layout of Qwen3's published GGUFs)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device once (a plain copy kernel of known size, to scale "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.copy_calib:
        import torch
        n = args.copy_calib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {n} bytes device to device")
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (sequences would shard "
              f"across GPUs with no per-step exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import sllm_next as S

    if args.config == "mtp":
        return bench_mtp(args)
    moe = args.config == "moe"
    cfg = dict(S.QWEN3_30B_A3B if moe else S.QWEN3_4B)
    if args.wtype == 8:
        cfg["wtype"] = 8
    tied = args.table == "q6k-tied"
    if tied:
        cfg.update(embd_type=14, tied=1)
    path = model_file(cfg, args.seed, args.model)
    B, ctx = args.seqs, args.ctx
    total = ctx + args.warmup + args.steps + args.prof_steps + 1
    t = time.time()
    eng = S.Engine(path, slots=B, ctx=total, max_rows=B)
    if args.no_graphs:
        eng.graphs(False)
    eng.attn_mode(args.attn_mode)
    for s in range(B):
        eng.fill_kv(s, ctx, args.seed)
    log(f"[bench] engine open + {B} x {ctx} cells in {time.time() - t:.1f}s")
    seq = np.arange(B, dtype=np.int32)
    rows = np.arange(B, dtype=np.int32)
    tok = np.random.default_rng(args.seed).integers(0, eng.V, B).astype(np.int32)
    pos = np.full(B, ctx, np.int32)

    # chain (sn_step's queued successor, as a decoding caller uses it): each step has the next queued behind it on the
    # GPU, fed its tokens there, so the host's turn-around overlaps the GPU. The last warmup step and the last timed
    # step queue nothing, so the timed region holds exactly `steps` steps of GPU work.
    def step(chain):
        nonlocal tok
        tok = eng.step(tok, seq, pos, rows, chain=chain)
        pos[:] += 1

    use_chain = 0 if args.no_chain else 1
    for i in range(args.warmup):
        step(use_chain if i + 1 < args.warmup else 0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gpu_ms = 0.0
    for i in range(args.steps):
        step(use_chain if i + 1 < args.steps else 0)
        gpu_ms += eng.last_gpu_ms()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    value = B * args.steps / dt
    caps, reps = eng.graph_count()
    taken, dropped = eng.chain_count()
    log(f"[bench] {args.steps} steps: {dt * 1e3 / args.steps:.3f} ms/step wall, {gpu_ms / args.steps:.3f} ms/step GPU "
        f"(graph captures {caps}, replays {reps}; queued steps taken {taken}, dropped {dropped})")

    # profiled pass: per-kernel-class time and algorithmic bytes
    eng.prof(True)
    for _ in range(args.prof_steps):
        step(0)
    prof = eng.prof_read()
    eng.prof(False)
    kernels = {}
    for name, p in prof.items():
        if p["launches"]:
            gbs = p["bytes"] / (p["ms"] * 1e-3) / 1e9
            kernels[name] = {"ms_per_step": p["ms"] / args.prof_steps, "launches_per_step": p["launches"] / args.prof_steps,
                             "bytes_per_launch": p["bytes"] / p["launches"], "us_per_launch": 1e3 * p["ms"] / p["launches"],
                             "GBps": gbs, "frac": gbs * 1e9 / HBM_PEAK}
    log("[bench] kernels " + json.dumps(kernels))
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"]) if kernels else None

    # HBM bytes per launch of each class from the committed rocprofv3 counter runs of this workload (FETCH_SIZE and
    # WRITE_SIZE, scaled by a copy of known size): profiles/decode_qwen3_4b_b32_ctx2048_traffic.md
    traffic = {}
    tpath = os.path.join(ROOT, "profiles", "decode_qwen3_4b_b32_ctx2048_traffic.json")
    if not moe and args.wtype == 2 and not tied and (B, ctx) == (32, 2048) and os.path.exists(tpath):
        traffic = json.load(open(tpath))

    def roof(k):
        c = kernels[k]
        return {"kernel": k, "bound": "hbm", "achieved": round(c["GBps"], 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(c["frac"], 4), "traffic": round(traffic[k]) if k in traffic else None,
                "bytes_per_launch": round(c["bytes_per_launch"]), "us_per_launch": round(c["us_per_launch"], 2),
                **({"traffic_source": "profiles/decode_qwen3_4b_b32_ctx2048_traffic.md"} if k in traffic else {})}

    eng.close()
    cpu = None
    if not args.no_cpu and not moe:
        t = time.time()
        cpu = cpu_baseline(path, B, ctx, args.seed)
        log(f"[bench] cpu baseline in {time.time() - t:.1f}s: {cpu['value']:.2f} tok/s")
    q = "Q8_0" if args.wtype == 8 else "Q4_0"
    metric = (f"agg decode tok/s, Qwen3-30B-A3B-arch {q} MoE x32 seqs" if moe else
              f"agg decode tok/s, Qwen3-4B-arch {q} x32 seqs; {q} GEMV % HBM peak")
    workload = (f"Qwen3-30B-A3B-arch {q} MoE batched decode step (BASELINE.json configs[4])" if moe else
                f"Qwen3-4B-arch {q} batched decode step (BASELINE.json configs[2]" +
                (")" if args.wtype == 2 else ", its matrices in Q8_0)")) + \
               ("; Q6_K token table tied to the LM head" if tied else "")
    line = {
        "metric": metric,
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": f"{q.lower()} x q8_0 -> f32 (fp16 MFMA); f16 KV, f32 softmax",
        "data": "synthetic: random-init weights (seeded), random token ids, seeded N(0,1) fp16 context cells",
        "config": {"workload": workload, "seqs": B,
                   "ctx": ctx, "layers": cfg["n_layer"], "hidden": cfg["n_embd"], "heads": cfg["n_head"],
                   "kv_heads": cfg["n_head_kv"], "ffn": cfg["n_ff"], "vocab": cfg["n_vocab"], "page_cells": 64,
                   **({"experts": cfg["n_expert"], "experts_used": cfg["n_expert_used"], "expert_ffn": cfg["n_ff_exp"]}
                      if moe else {}),
                   "gpu_ms_per_step": round(gpu_ms / args.steps, 4), "chain": bool(use_chain),
                   "token_table": "Q6_K, tied LM head" if tied else f"F32, untied {q} LM head"},
        "roofline": roof(dom) if dom else None,
        "roofline_gemm": roof("gemm") if "gemm" in kernels else None,
        "kernels": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in kernels.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_mtp(args):
    """the fused draft-verify step (snx_spec_step) of the Qwen3-4B-arch model with one Q4_0 guess-head
    block: 8 sequences at 4096 cells, k = 3 drafts each, verify rows [last, d1, d2, d3]; a seeded mask forces each draft
    to equal its row's argmax with probability --accept (the rows still run in full). value = tokens kept per second."""
    import numpy as np
    import torch

    import sllm_next as S

    cfg = dict(S.QWEN3_4B, nextn=1)
    path = model_file(cfg, args.seed, args.model)
    B, ctx, k = 8, 4096, 3
    total = ctx + (args.warmup + args.steps + args.prof_steps) * (k + 1) + 8
    t = time.time()
    eng = S.Engine(path, slots=B, ctx=total, max_rows=B * (k + 1))
    eng.attn_mode(args.attn_mode)
    assert eng.guess_head() and eng.guess_on(True)
    for s in range(B):
        eng.fill_kv(s, ctx, args.seed)
    log(f"[bench] engine open + {B} x {ctx} cells in {time.time() - t:.1f}s")
    rng = np.random.default_rng(args.seed)
    seqs = np.arange(B, dtype=np.int32)
    last = rng.integers(0, eng.V, B).astype(np.int32)
    pos = np.full(B, ctx, np.int32)
    kept = 0

    def step():
        nonlocal last, kept
        force = (rng.random((B, k)) < args.accept).astype(np.uint8)
        n, tok = eng.spec_step(seqs, last, pos, k, force=force)
        last = tok[np.arange(B), n - 1].astype(np.int32)
        pos[:] += n
        kept += int(n.sum())

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    kept = 0
    t0 = time.perf_counter()
    gpu_ms = 0.0
    for _ in range(args.steps):
        step()
        gpu_ms += eng.last_gpu_ms()
    dt = time.perf_counter() - t0
    toks = kept
    log(f"[bench] {args.steps} spec steps: {dt * 1e3 / args.steps:.3f} ms/step, {toks / args.steps:.2f} tokens/step")
    eng.prof(True)
    for _ in range(args.prof_steps):
        step(0)
    prof = eng.prof_read()
    eng.prof(False)
    eng.close()
    kernels = {}
    for name, p in prof.items():
        if p["launches"]:
            gbs = p["bytes"] / (p["ms"] * 1e-3) / 1e9
            kernels[name] = {"ms_per_step": round(p["ms"] / args.prof_steps, 4),
                             "launches_per_step": p["launches"] / args.prof_steps,
                             "GBps": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4)}
    line = {
        "metric": "MTP draft+verify tok/s, Qwen3-4B-arch Q4_0 + 1 Q4_0 guess-head block, 8 seqs x 4096, k=3",
        "value": round(toks / dt, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_0 x q8_0 -> f32 (fp16 MFMA); f16 KV, f32 softmax",
        "data": f"synthetic: random-init weights (seeded), seeded N(0,1) fp16 context cells, seeded draft mask "
                f"(p={args.accept})",
        "config": {"workload": "fused MTP draft+verify step (BASELINE.json configs[3])", "seqs": B, "ctx": ctx,
                   "drafts": k, "verify_rows": B * (k + 1), "tokens_per_step": round(toks / args.steps, 3),
                   "gpu_ms_per_step": round(gpu_ms / args.steps, 4)},
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
