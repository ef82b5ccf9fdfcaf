#!/usr/bin/env python3
"""Headline benchmark: aggregate decode tokens/s of the batched decode step (sn_step) on one MI355X.

Workload: a Qwen3-4B-architecture dense model, random init (seeded N(0, 0.02) weights
quantized to Q4_0 with ggml's reference quantizer; fp32 embedding and norms; untied Q4_0 LM head), 32 sequences whose
2048-cell contexts are already in the paged fp16 KV cache (seeded N(0, 1) cells: a step costs the same whatever they
hold), one new token per sequence per step, greedy argmax fed back as the next token. A step is one sn_step call of 32
rows: inputs resident on the GPU, one host round trip (the 32 tokens back).

Output: one JSON line. `value` = 32 * steps / wall time of the timed steps. `roofline` is the Q4_0 matmul class (the
metric's "Q4_0 GEMV % HBM peak"): its algorithmic bytes / time against 8 TB/s in a separate profiled pass of the same
steps (HIP events around every launch on the engine's stream); `roofline_dominant` is the class with the most GPU time
a step (paged attention). `cpu_baseline` times the oracle (oracle/, a C restatement of ggml's CPU semantics) on the
host cores for one step of the same workload. The default run ends the line with a short summary of configs[0], [1],
[3], [4] and the prompt rows (`configs`); every configuration's full line goes to stderr.
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
# the matrices of the Qwen3-4B-arch decode step at its 32 rows: (M, N, K); q|k|v and gate|up fused
DECODE_SHAPES = {"qkv": (32, 6144, 2560), "o": (32, 2560, 4096), "gateup": (32, 19456, 2560), "down": (32, 2560, 9728),
                 "head": (32, 151936, 2560)}
MFMA_F16_PEAK = 2.5e15  # MI355X dense fp16 MFMA, flop/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def model_file(cfg_kw, seed, path=None):
    import sllm_next as S
    return S.cached_model(cfg_kw, seed, path, log=lambda m: log("[bench] " + m))


def cpu_spec_baseline(path, n, ctx, k, seed, layers, accept):
    """The oracle's fused draft-verify step (oracle/oracle.c) for n sequences at position ctx on the host cores: each
    sequence's k guesses (or_mtp_guess), one model step over the n (k + 1) verify rows, the guess head's cells of those
    rows (or_mtp_fill), greedy acceptance with the benchmark's forced share of drafts. Median of at least 10 warm runs
    of a one-layer and a two-layer cut (each with the guess head and the output stage), scaled to `layers`."""
    import numpy as np

    from oracle import oracle as O
    from oracle.gguf import GGUF

    O.build() if not os.path.exists(O.LIB_PATH) else None
    g = GGUF(path)
    rng = np.random.default_rng(seed)
    ts = {}
    for nl in (1, 2):
        ref = O.Qwen3(LayerCut(g, nl), n_seq=n, ctx=ctx + k + 2)
        ref.k[:, :, :ctx] = 0
        ref.v[:, :, :ctx] = 0
        last = rng.integers(0, ref.V, n).astype(np.int32)
        hprev = np.zeros((n, ref.E), np.float32)
        nt = cpu_threads()

        def spec():
            drafts = [ref.mtp_guess(s, int(last[s]), ctx, k, hprev[s], nthreads=nt)[0] for s in range(n)]
            tok = np.concatenate([[last[s]] + list(drafts[s]) for s in range(n)]).astype(np.int32)
            seq = np.repeat(np.arange(n, dtype=np.int32), k + 1)
            pos = np.tile(np.arange(ctx, ctx + k + 1, dtype=np.int32), n)
            hn = np.zeros((n * (k + 1), ref.E), np.float32)
            _, lg, _ = ref.step(tok, seq, pos, np.arange(n * (k + 1), dtype=np.int32), hn_all=hn, nthreads=nt)
            ref.mtp_fill(tok, seq, pos, np.concatenate([hprev[:1], hn[:-1]]), nthreads=nt)
            force = rng.random((n, k)) < accept
            for s in range(n):
                tg = [O.argmax(lg[s * (k + 1) + i]) if not (i < k and force[s, i]) else drafts[s][i] for i in range(k + 1)]
                O.accept(drafts[s], np.array(tg[:k], np.int32))

        ts[nl] = median_time(spec)
        del ref
    t = ts[1][0] + (layers - 1) * max(ts[2][0] - ts[1][0], 0.0)
    sample = (f"{n} sequences' draft-verify step at position {ctx} (k = {k} guesses each, one step over the "
              f"{n * (k + 1)} verify rows, the guess head's cells, acceptance) through oracle/oracle.c "
              f"(ggml-semantics CPU restatement; generic scalar loops): median of {ts[1][1]} / {ts[2][1]} warm runs of "
              f"a 1- and a 2-layer cut of the model with its guess head and output stage ({ts[1][0]:.3f} / "
              f"{ts[2][0]:.3f} s), scaled to {layers} layers: {t:.2f} s a step")
    return t, sample


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
    ap.add_argument("--config", default="all",
                    choices=("all", "decode", "mtp", "moe", "matmul", "attn", "prefill", "fewrows"),
                    help="all (default): the headline (configs[2]) with configs[0], [1], [3], [4] and the prompt "
                         "rows inside its line; "
                         "decode: the headline alone; mtp: the fused draft-verify step (configs[3]); "
                         "moe: Qwen3-30B-A3B-arch batched decode (configs[4]); matmul: one 8 x 4096 x 4096 Q4_0 "
                         "matmul (configs[0]); attn: one layer of paged decode attention (configs[1]); prefill: "
                         "2048-token prompts in 512-row steps; fewrows: the MFMA matmul against the per-column "
                         "integer-dot GEMV at 1-8 rows on the decode step's matrices and configs[0]")
    ap.add_argument("--accept", type=float, default=0.6, help="mtp: the seeded share of drafts forced to match")
    ap.add_argument("--mm-shape", default="c1", choices=("c1",) + tuple(DECODE_SHAPES),
                    help="matmul: configs[0] (c1, the default) or one of the 32-row decode step's matrices")
    ap.add_argument("--no-graphs", action="store_true", help="launch every step eagerly (no HIP graph replay)")
    ap.add_argument("--no-chain", action="store_true", help="decode without sn_step's queued successor (chain = 0)")
    ap.add_argument("--attn-mode", type=int, default=-1, choices=(-1, 0, 1, 2),
                    help="attention work list: -1 chosen per step, 0 per-chunk + merge, 1 whole groups, 2 run items "
                         "for prompt rows wherever possible")
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

    subs = {"mtp": bench_mtp, "matmul": bench_matmul, "attn": bench_attn, "prefill": bench_prefill,
            "fewrows": bench_fewrows}
    if args.config in subs:
        print(json.dumps(subs[args.config](args)), flush=True)
        return
    if args.config in ("decode", "moe"):
        print(json.dumps(bench_decode(args, moe=args.config == "moe")), flush=True)
        return
    # all: the headline with a short summary of the other configurations at the end of its line (each
    # configuration's full line, and the headline's own, go to stderr)
    line = bench_decode(args, moe=False)
    log("[bench] headline full line " + json.dumps(line))
    line["kernels"] = {k: {"ms_per_step": v["ms_per_step"], "frac": v["frac"]} for k, v in line["kernels"].items()}
    t = time.time()
    try:
        shapes = {name: matmul_shape(*mnk, seed=3) for name, mnk in DECODE_SHAPES.items()}
        log("[bench] gemm_shapes " + json.dumps(shapes))
        line["gemm_shapes"] = {n: {"us": v["us_per_launch"], "read_floor_us": v["read_floor_us"], "frac": v["frac"]}
                               for n, v in shapes.items()}
    except Exception as e:
        import traceback
        traceback.print_exc()
        line["gemm_shapes"] = {"error": repr(e)}
    log(f"[bench] gemm shapes in {time.time() - t:.1f}s")
    line["configs"] = {}
    for name, fn in (("c1_matmul", bench_matmul), ("c2_attn", bench_attn), ("c4_mtp", bench_mtp),
                     ("c5_moe", lambda a: bench_decode(a, moe=True)), ("f1_prefill", bench_prefill)):
        t = time.time()
        try:
            full = fn(args)
            log(f"[bench] {name} full line " + json.dumps(full))
            line["configs"][name] = summary(full)
        except Exception as e:  # (the headline stands; the failure is reported in its place)
            import traceback
            traceback.print_exc()
            line["configs"][name] = {"error": repr(e)}
        log(f"[bench] {name} in {time.time() - t:.1f}s")
    print(json.dumps(line), flush=True)


def summary(full):
    """A configuration's line cut to its figures: value, time, the roofline fraction and the CPU baseline"""
    r = full.get("roofline") or {}
    cpu = full.get("cpu_baseline") or {}
    out = {"metric": full.get("metric"), "value": full.get("value"), "unit": full.get("unit"),
           "ms_per_step": full.get("ms_per_step"), "roofline": {k: r.get(k) for k in ("kernel", "bound", "frac", "unit",
                                                                                    "achieved", "traffic")}}
    if "us_per_launch" in full:
        out["us_per_launch"] = full["us_per_launch"]
    if cpu:
        out["cpu_baseline"] = {"value": cpu.get("value"), "unit": cpu.get("unit"), "cores": cpu.get("cores"),
                               "kind": cpu.get("kind")}
    return out


def bench_decode(args, moe):
    """configs[2] (the headline) or configs[4] (moe): batched decode steps of 32 sequences at 2048 cells."""
    import numpy as np
    import torch

    import sllm_next as S

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
    tname = "moe_qwen3_30b_a3b_b32_ctx2048_traffic" if moe else "decode_qwen3_4b_b32_ctx2048_traffic"
    tpath = os.path.join(ROOT, "profiles", tname + ".json")
    if args.wtype == 2 and not tied and (B, ctx) == (32, 2048) and os.path.exists(tpath):
        traffic = json.load(open(tpath))

    def roof(k):
        c = kernels[k]
        return {"kernel": k, "bound": "hbm", "achieved": round(c["GBps"], 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(c["frac"], 4), "traffic": round(traffic[k]) if k in traffic else None,
                "bytes_per_launch": round(c["bytes_per_launch"]), "us_per_launch": round(c["us_per_launch"], 2),
                **({"traffic_source": f"profiles/{tname}.md"} if k in traffic else {})}

    eng.close()
    cpu = None
    if not args.no_cpu:
        t = time.time()
        sec, sample = cpu_step_baseline(path, B, ctx, args.seed, cfg["n_layer"])
        cpu = {"value": round(B / sec, 3), "unit": "tok/s", **cpu_info(), "kind": "port", "sample": sample}
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
        # the metric names the Q4_0 GEMV's fraction of HBM peak: that class is the line's roofline; the class with the
        # most time a step (paged attention) is roofline_dominant
        "roofline": roof("gemm") if "gemm" in kernels else None,
        "roofline_dominant": roof(dom) if dom else None,
        "kernels": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in kernels.items()},
        "cpu_baseline": cpu,
    }
    return line


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
    if args.no_graphs:
        eng.graphs(False)
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
    caps, reps = eng.graph_count()
    log(f"[bench] {args.steps} spec steps: {dt * 1e3 / args.steps:.3f} ms/step, {toks / args.steps:.2f} tokens/step "
        f"(graph captures {caps}, replays {reps})")
    eng.prof(True)
    for _ in range(args.prof_steps):
        step()
    prof = eng.prof_read()
    eng.prof(False)
    eng.close()
    cpu = None
    if not args.no_cpu:
        t = time.time()
        sec, sample = cpu_spec_baseline(path, B, ctx, k, args.seed, cfg["n_layer"], args.accept)
        per_step = toks / args.steps
        cpu = {"value": round(per_step / sec, 3), "unit": "tok/s", **cpu_info(), "kind": "port",
               "sample": sample + f"; tokens kept a step as on the GPU ({per_step:.2f})"}
        log(f"[bench] cpu baseline in {time.time() - t:.1f}s: {cpu['value']:.2f} tok/s")
    kernels = {}
    for name, p in prof.items():
        if p["launches"]:
            gbs = p["bytes"] / (p["ms"] * 1e-3) / 1e9
            kernels[name] = {"ms_per_step": round(p["ms"] / max(args.prof_steps, 1), 4),
                             "launches_per_step": p["launches"] / max(args.prof_steps, 1),
                             "bytes_per_launch": round(p["bytes"] / p["launches"]),
                             "us_per_launch": round(1e3 * p["ms"] / p["launches"], 2),
                             "GBps": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4)}
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"]) if kernels else None
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
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": kernels[dom]["GBps"], "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": kernels[dom]["frac"],
                     "traffic": profile_traffic("mtp_qwen3_4b_b8_ctx4096_k3_traffic.json", dom),
                     "bytes_per_launch": kernels[dom]["bytes_per_launch"],
                     "us_per_launch": kernels[dom]["us_per_launch"]} if dom else None,
        "verify_gemm_mfma": profile_value("mtp_qwen3_4b_b8_ctx4096_k3_traffic.json",
                                          ("verify_gemm_mfma_busy", "verify_gemm_tflops")),
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    return line


def bench_prefill(args):
    """Prompt rows (the next row after the decode step): 8 sequences of 2048 prompt tokens on the Qwen3-4B-arch model,
    fed 512 rows a step (4 steps a sequence; every row writes its cell, the last row's token is sampled), as a serving
    loop prefills. value = prompt tokens per second over the timed sequences (after one warmup sequence)."""
    import numpy as np
    import torch

    import sllm_next as S

    cfg = dict(S.QWEN3_4B)
    path = model_file(cfg, args.seed, args.model)
    n_seq, ctx, rows = 8, 2048, 512
    eng = S.Engine(path, slots=n_seq + 1, ctx=ctx + 1, max_rows=rows)
    rng = np.random.default_rng(args.seed)

    def prefill(s):
        toks = rng.integers(0, eng.V, ctx).astype(np.int32)
        for c0 in range(0, ctx, rows):
            eng.step(toks[c0:c0 + rows], np.full(rows, s, np.int32), np.arange(c0, c0 + rows, dtype=np.int32),
                     np.array([rows - 1], np.int32), n_write=0)

    prefill(n_seq)  # warmup on the spare slot
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(n_seq):
        prefill(s)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    toks = n_seq * ctx
    # profiled pass: one more sequence's steps on the spare slot (cleared first)
    eng.clear(n_seq, 0, ctx)
    eng.prof(True)
    prefill(n_seq)
    prof = eng.prof_read()
    eng.prof(False)
    eng.close()
    steps = ctx // rows
    kernels = {}
    for name, p in prof.items():
        if p["launches"]:
            gbs = p["bytes"] / (p["ms"] * 1e-3) / 1e9
            kernels[name] = {"ms_per_step": round(p["ms"] / steps, 4), "launches_per_step": p["launches"] / steps,
                             "bytes_per_launch": round(p["bytes"] / p["launches"]),
                             "us_per_launch": round(1e3 * p["ms"] / p["launches"], 2),
                             "GBps": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4)}
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"]) if kernels else None
    # at 512 rows the matmuls are MFMA work: 2 M N K flop per matrix (q|k|v, o, gate|up, down per layer; the LM head
    # for the step's one output row), against MI355X's dense fp16 peak (the operands are fp16)
    E, F, H, KVH = cfg["n_embd"], cfg["n_ff"], cfg["n_head"], cfg["n_head_kv"]
    layer = (H + 2 * KVH) * 128 * E + E * H * 128 + 2 * F * E + E * F
    flop = 2.0 * rows * layer * cfg["n_layer"] + 2.0 * E * cfg["n_vocab"]
    g = kernels.get("gemm")
    roof_mfma = {"kernel": "k_q4_gemm / k_q4_gemm_fk2 (the full-K walk)", "bound": "mfma", "achieved": round(flop / (g["ms_per_step"] * 1e-3) / 1e12, 1),
                 "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                 "frac": round(flop / (g["ms_per_step"] * 1e-3) / MFMA_F16_PEAK, 4),
                 "traffic": profile_traffic("prefill_qwen3_4b_2048_rows512_traffic.json", "k_q4_gemm"),
                 "flop_per_launch": round(flop / g["launches_per_step"]),
                 "us_per_launch": g["us_per_launch"],
                 "mfma_busy": profile_value("prefill_qwen3_4b_2048_rows512_traffic.json",
                                            ("gemm_mfma_busy", "gemm_valu_per_mfma"))} if g else None
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        from oracle.gguf import GGUF
        O.build() if not os.path.exists(O.LIB_PATH) else None
        ref = O.Qwen3(GGUF(path), n_seq=1, ctx=ctx)
        n = 64
        tok = rng.integers(0, ref.V, n).astype(np.int32)
        t = time.perf_counter()
        ref.step(tok, np.zeros(n, np.int32), np.arange(n, dtype=np.int32), np.array([n - 1], np.int32))
        cdt = time.perf_counter() - t
        nt = cpu_threads()
        cpu = {"value": round(n / cdt, 2), "unit": "tok/s", "cores": nt, "kind": "port",
               "sample": f"one 64-row prompt step (positions 0..63, all layers, the last row's LM head) through "
                         f"oracle/oracle.c, {cdt:.1f} s on {nt} threads"}
    log(f"[bench] prefill: {n_seq} x {ctx} prompt tokens in {dt:.3f} s ({dt * 1e3 / (n_seq * steps):.2f} ms per "
        f"{rows}-row step)")
    line = {
        "metric": "prefill tok/s, Qwen3-4B-arch Q4_0, 512-row prompt steps",
        "value": round(toks / dt, 1), "unit": "tok/s", "n_gpus": 1, "steps": n_seq * steps, "warmup": steps,
        "ms_per_step": round(dt * 1e3 / (n_seq * steps), 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_0 x q8_0 -> f32 (fp16 MFMA); f16 KV, f32 softmax",
        "data": "synthetic: random-init weights (seeded), random prompt token ids",
        "config": {"workload": "prompt rows of the batched step (sn_step prompt rows, 512 a step)", "seqs": n_seq,
                   "prompt": ctx, "rows_per_step": rows, "layers": cfg["n_layer"], "hidden": cfg["n_embd"]},
        "roofline": roof_mfma if dom == "gemm" else None,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    return line


def graph_us(fn, n, reps=10):
    """Device time (microseconds) of one of n calls fn(i, stream) captured into a HIP graph (torch.cuda.graph: the
    launches replay back to back with no host launch cost), timed with HIP events over `reps` replays."""
    import ctypes as C

    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(n):
            fn(i, st)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps / n


def profile_traffic(name, key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter runs (profiles/), or None"""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    v = json.load(open(path)).get(key)
    return round(v) if v is not None else None


def profile_value(name, keys):
    """values measured by the committed rocprofv3 counter runs (profiles/), with their source, or None"""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    d = json.load(open(path))
    return {**{k: d.get(k) for k in keys}, "source": "profiles/" + name.replace(".json", ".md")}


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count())


def cpu_info():
    """the host the CPU baseline ran on: threads used, logical CPUs, CPU model"""
    model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cores": cpu_threads(), "nproc": os.cpu_count(), "cpu_model": model}


def median_time(fn, min_runs=10, min_s=0.0):
    """median wall time of fn() over at least min_runs runs (and at least min_s seconds) after one warm-up run"""
    import statistics
    fn()
    ts = []
    t_all = time.perf_counter()
    while len(ts) < min_runs or time.perf_counter() - t_all < min_s:
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts), len(ts)


class LayerCut:
    """A GGUF model read as its first n layers (and its guess-head block, renumbered after them): the oracle's CPU
    baseline times a cut of one and of two layers and scales by the layer count (every layer of these models costs
    the same)."""

    def __init__(self, g, n):
        a = g.kv["general.architecture"]
        self.g, self.n = g, n
        self.n_mtp = int(g.kv.get(f"{a}.nextn_predict_layers", 0))
        self.L = int(g.kv[f"{a}.block_count"]) - self.n_mtp
        self.kv = dict(g.kv)
        self.kv[f"{a}.block_count"] = n + self.n_mtp
        self.tinfo = {self._rename(k): v for k, v in g.tinfo.items() if self._keep(k)}

    def _keep(self, name):
        if not name.startswith("blk."):
            return True
        i = int(name.split(".")[1])
        return i < self.n or i == self.L

    def _rename(self, name):  # the guess head's block L -> n
        if name.startswith(f"blk.{self.L}."):
            return f"blk.{self.n}." + name[len(f"blk.{self.L}."):]
        return name

    def _orig(self, name):
        if self.n_mtp and name.startswith(f"blk.{self.n}."):
            return f"blk.{self.L}." + name[len(f"blk.{self.n}."):]
        return name

    def tensor(self, name):
        return self.g.tensor(self._orig(name))

    def type_name(self, name):
        return self.g.type_name(self._orig(name))


def cpu_step_baseline(path, n_rows, ctx, seed, layers):
    """The oracle's step (oracle/oracle.c, ggml-semantics CPU restatement) of n_rows decode rows at position ctx on the
    host cores: the median of at least 10 warm runs of a one-layer and of a two-layer cut of the model (each with the
    output stage), scaled to `layers`: per step = t1 + (layers - 1) (t2 - t1). Returns (seconds per step, sample)."""
    import numpy as np

    from oracle import oracle as O
    from oracle.gguf import GGUF

    O.build() if not os.path.exists(O.LIB_PATH) else None
    g = GGUF(path)
    r = np.random.default_rng(seed)
    ts = {}
    for n in (1, 2):
        ref = O.Qwen3(LayerCut(g, n), n_seq=n_rows, ctx=ctx + 1)
        ref.k[:, :, :ctx] = 0  # (touch the cells the step reads)
        ref.v[:, :, :ctx] = 0
        tok = r.integers(0, ref.V, n_rows).astype(np.int32)
        seq = np.arange(n_rows, dtype=np.int32)
        pos = np.full(n_rows, ctx, np.int32)
        ts[n] = median_time(lambda: ref.step(tok, seq, pos, seq, nthreads=cpu_threads()))
        del ref
    per_layer = max(ts[2][0] - ts[1][0], 0.0)
    t = ts[1][0] + (layers - 1) * per_layer
    sample = (f"{n_rows} decode rows at position {ctx} through oracle/oracle.c (ggml-semantics CPU restatement: Q8_0 "
              f"activations, integer block dots, fp32 attention over fp16 cells; ggml b11669 is not available offline, "
              f"and these generic scalar loops are slower than ggml's AVX2 / AVX-512 kernels): median of "
              f"{ts[1][1]} / {ts[2][1]} warm runs of a 1- and a 2-layer cut of the model with its output stage "
              f"({ts[1][0]:.3f} / {ts[2][0]:.3f} s), scaled to {layers} layers: {t:.2f} s a step")
    return t, sample


class Dev:
    """Device buffers through torch (allocation and streams only): the kernel ABI takes plain pointers."""

    @staticmethod
    def copy(a):
        import numpy as np
        import torch
        return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).to("cuda")

    @staticmethod
    def empty(nbytes):
        import torch
        return torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device="cuda")

    @staticmethod
    def host(t, dtype):
        import torch
        torch.cuda.synchronize()
        return t.cpu().numpy().view(dtype)

    @staticmethod
    def ptr(t):
        import ctypes as C
        return C.c_void_p(t.data_ptr())

    @staticmethod
    def stream():
        import ctypes as C

        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def matmul_shape(M, N, K, seed, copies=None, Wq=None):
    """One Q4_0 matmul shape: the matmul kernel's average launch time (its k-slice sums, launches back to back on one
    stream, weight copies in turn beyond the 256 MB Infinity Cache) beside a plain streaming read of the same weight
    bytes from the same copies (snk_read_time): the floor a launch of that size meets on this box."""
    import ctypes as C

    import numpy as np
    import torch

    import sllm_next as S

    U = Dev
    L = S.lib()
    r = np.random.default_rng(seed)
    if Wq is None:  # (a seeded block of up to 8192 rows, repeated: a launch costs the same whatever W holds)
        nb = min(N, 8192)
        Wq = S.quantize_q4_0((r.standard_normal((nb, K)) * 0.02).astype(np.float32))
        Wq = np.ascontiguousarray(np.tile(Wq, ((N + nb - 1) // nb, 1))[:N])
    sb = L.snk_q4_stripes_bytes(N, K)
    copies = copies or max(2, int(np.ceil(600e6 / sb)))
    st0 = U.stream()
    dW = U.copy(Wq)
    tiles = [U.empty(sb) for _ in range(copies)]
    for t in tiles:
        assert L.snk_q4_repack(U.ptr(dW), N, K, U.ptr(t), st0) == 0
    X = r.standard_normal((M, K)).astype(np.float32)
    dX = U.copy(X)
    xa = U.empty(L.snk_xa_bytes(M, K))
    assert L.snk_quant_act(U.ptr(dX), M, K, K, None, C.c_float(0.0), U.ptr(xa), st0) == 0
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    ws = U.empty(wsb)
    y = U.empty(M * N * 4)
    sink = U.empty(1024)
    torch.cuda.synchronize()
    ptrs = (C.c_void_p * copies)(*[t.data_ptr() for t in tiles])
    us = L.snk_q4_gemm_time(C.cast(ptrs, C.c_void_p), copies, U.ptr(xa), M, N, K, U.ptr(y), N, U.ptr(ws),
                            C.c_size_t(wsb), 200, st0)
    us_read = L.snk_read_time(C.cast(ptrs, C.c_void_p), copies, C.c_size_t(sb // 16 * 16), C.c_void_p(sink.data_ptr()),
                              200, st0)
    alg = N * K // 32 * 18 + M * K * 4 + M * N * 4
    out = {"M": M, "N": N, "K": K, "weight_copies": copies, "algorithmic_bytes": alg, "us_per_launch": round(us, 3),
           "GBps": round(alg / (us * 1e-6) / 1e9, 1), "frac": round(alg / (us * 1e-6) / HBM_PEAK, 4),
           "read_floor_us": round(us_read, 3), "read_floor_GBps": round(sb / (us_read * 1e-6) / 1e9, 1),
           "floor_frac": round(us_read / us, 4)}
    log(f"[bench] matmul {M}x{N}x{K}: {us:.2f} us ({out['GBps']} GB/s); a plain read of its {sb / 1e6:.1f} MB of "
        f"weights {us_read:.2f} us ({out['read_floor_GBps']} GB/s)")
    del tiles
    torch.cuda.empty_cache()
    return out


def bench_fewrows(args):
    """The matmul at few rows (1, 2, 4, 8): the default MFMA launch against the per-column integer-dot GEMV (the
    north star's mat-vec design; snk_q4_gemm_plan_time with mt 0, at most 4 rows), both with the default plan's
    slices and the same bits, average launch time with weight copies in turn beyond the Infinity Cache. The line's
    value is the geometric mean of GEMV / MFMA time over the shapes and row counts the GEMV takes (below 1: the GEMV
    is faster)."""
    import ctypes as C

    import numpy as np
    import torch

    import sllm_next as S

    U = Dev
    L = S.lib()
    st = U.stream()
    r = np.random.default_rng(1)
    shapes = dict(c1=(4096, 4096), **{k: v[1:] for k, v in DECODE_SHAPES.items()})
    res, ratios = {}, []
    for name, (N, K) in shapes.items():
        nb = min(N, 8192)
        Wq = S.quantize_q4_0((r.standard_normal((nb, K)) * 0.02).astype(np.float32))
        Wq = np.ascontiguousarray(np.tile(Wq, ((N + nb - 1) // nb, 1))[:N])
        sb = L.snk_q4_stripes_bytes(N, K)
        copies = max(2, int(np.ceil(600e6 / sb)))
        dW = U.copy(Wq)
        tiles = [U.empty(sb) for _ in range(copies)]
        for t in tiles:
            assert L.snk_q4_repack(U.ptr(dW), N, K, U.ptr(t), st) == 0
        ptrs = C.cast((C.c_void_p * copies)(*[t.data_ptr() for t in tiles]), C.c_void_p)
        res[name] = {"N": N, "K": K}
        for M in (1, 2, 4, 8):
            X = r.standard_normal((M, K)).astype(np.float32)
            xa = U.empty(L.snk_xa_bytes(M, K))
            assert L.snk_quant_act(U.ptr(U.copy(X)), M, K, K, None, C.c_float(0.0), U.ptr(xa), st) == 0
            wsb = L.snk_q4_workspace_bytes(M, N, K)
            ws = U.empty(wsb)
            torch.cuda.synchronize()
            t_m = L.snk_q4_gemm_plan_time(ptrs, copies, U.ptr(xa), M, N, K, U.ptr(ws), C.c_size_t(wsb), 1, 1, 0, 100, st)
            row = {"mfma_us": round(t_m, 2)}
            if M <= 4:
                t_v = L.snk_q4_gemm_plan_time(ptrs, copies, U.ptr(xa), M, N, K, U.ptr(ws), C.c_size_t(wsb), 0, 0, 0,
                                              100, st)
                row["gemv_us"] = round(t_v, 2)
                ratios.append(t_v / t_m)
            res[name][f"M{M}"] = row
            log(f"[bench] fewrows {name} M={M}: {row}")
        del tiles
        torch.cuda.empty_cache()
    gm = float(np.exp(np.mean(np.log(ratios))))
    return {"metric": "few-row Q4_0 matmul: per-column integer-dot GEMV time / MFMA time (geometric mean)",
            "value": round(gm, 4), "unit": "ratio", "n_gpus": 1, "higher_is_better": False, "vs_baseline": None,
            "dtype": "q4_0 x q8_0 -> f32 (both kernels: the same bits)", "data": "synthetic: seeded weights, rows",
            "config": {"workload": "decode step matrices and configs[0] at 1-8 rows", "shapes": res}}


def bench_matmul(args):
    """configs[0] (C1): one Q4_0 matmul Y[8][4096] = X[8][4096] . W[4096][4096]^T. W ~ N(0, 0.02) (seed 1) quantized
    by ggml's reference Q4_0 rule, X ~ N(0, 1). One call is the op as a drop-in runs it: X quantized to the Q8_0 operand,
    the matmul's k-slices, their reduction into Y. 40 copies of W (377 MB, beyond the 256 MB Infinity Cache) are used
    in turn; the calls replay from a HIP graph. value = algorithmic bytes (W + X + Y) per call / time per call."""
    import ctypes as C

    import numpy as np
    import torch

    import sllm_next as S

    if args.mm_shape != "c1":  # one of the decode step's matrices: the kernel beside its read floor, no CPU line
        M, N, K = DECODE_SHAPES[args.mm_shape]
        sh = matmul_shape(M, N, K, seed=3)
        return {"metric": f"Q4_0 matmul GB/s (algorithmic W + X + Y bytes), {M} x {N} x {K}", "value": sh["GBps"],
                "unit": "GB/s", "n_gpus": 1, "steps": 200, "warmup": sh["weight_copies"],
                "ms_per_step": round(sh["us_per_launch"] * 1e-3, 5), "higher_is_better": True, "scaling": "weak",
                "vs_baseline": None, "dtype": "q4_0 x q8_0 -> f32 (fp16 MFMA)",
                "data": "synthetic: W ~ N(0, 0.02) seed 3 quantized to Q4_0, X ~ N(0, 1)",
                "config": {"workload": f"the {args.mm_shape} matrix of the 32-row decode step (BASELINE.json "
                                       f"configs[2])", **sh}}
    U = Dev
    L = S.lib()
    N = K = 4096
    M = 8
    r = np.random.default_rng(1)
    Wq = S.quantize_q4_0((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    X = r.standard_normal((M, K)).astype(np.float32)
    copies = 40
    st0 = U.stream()
    dW = U.copy(Wq)
    tiles = [U.empty(L.snk_q4_stripes_bytes(N, K)) for _ in range(copies)]
    for t in tiles:
        assert L.snk_q4_repack(U.ptr(dW), N, K, U.ptr(t), st0) == 0
    dX = U.copy(X)
    xa = U.empty(L.snk_xa_bytes(M, K))
    wsb = L.snk_q4_workspace_bytes(M, N, K)
    ws = U.empty(wsb)
    y = U.empty(M * N * 4)
    torch.cuda.synchronize()

    def op(i, st):
        L.snk_quant_act(U.ptr(dX), M, K, K, None, C.c_float(0.0), U.ptr(xa), st)
        L.snk_q4_gemm(U.ptr(tiles[i % copies]), U.ptr(xa), M, N, K, U.ptr(y), N, 0, U.ptr(ws), C.c_size_t(wsb), st)

    for _ in range(args.warmup):
        op(0, st0)
    torch.cuda.synchronize()
    n = max(copies, args.steps)
    us = graph_us(op, n)
    # the matmul kernel alone (its k-slice sums, launches timed with HIP events on the stream they run on)
    ptrs = (C.c_void_p * copies)(*[t.data_ptr() for t in tiles])
    us_gemm = L.snk_q4_gemm_time(C.cast(ptrs, C.c_void_p), copies, U.ptr(xa), M, N, K, U.ptr(y), N, U.ptr(ws), C.c_size_t(wsb), 200, st0)
    alg = N * K // 32 * 18 + M * K * 4 + M * N * 4
    got = U.host(y, np.float32)[:M * N].reshape(M, N)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        O.build() if not os.path.exists(O.LIB_PATH) else None
        nt = cpu_threads()
        want = O.mul_mat_q4_0(Wq, K, X, nthreads=nt)
        dt, reps = median_time(lambda: O.mul_mat_q4_0(Wq, K, X, nthreads=nt), min_s=2.0)
        err = float(np.abs(got - want).max())
        log(f"[bench] max |GPU - oracle| {err:.3g} (max |y| {float(np.abs(want).max()):.3g})")
        cpu = {"value": round(alg / dt / 1e9, 3), "unit": "GB/s", **cpu_info(), "kind": "port",
               "sample": f"the same 8 x 4096 x 4096 matmul through oracle/oracle.c (ggml-semantics CPU restatement: "
                         f"Q8_0 activations, integer block dots; generic scalar loops, slower than ggml's AVX2 / "
                         f"AVX-512 kernels): median of {reps} warm calls, {dt * 1e3:.2f} ms each"}
    gbs, gbs_k = alg / (us * 1e-6) / 1e9, alg / (us_gemm * 1e-6) / 1e9
    sink = U.empty(1024)
    us_read = L.snk_read_time(C.cast(ptrs, C.c_void_p), copies, C.c_size_t(L.snk_q4_stripes_bytes(N, K)),
                              C.c_void_p(sink.data_ptr()), 200, st0)
    log(f"[bench] C1 matmul: {us:.2f} us per call (quantize + matmul + reduce), matmul kernel {us_gemm:.2f} us; a "
        f"plain read of the weights {us_read:.2f} us")
    line = {
        "metric": "Q4_0 matmul GB/s (algorithmic W + X + Y bytes), 8 x 4096 x 4096",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": n, "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_0 x q8_0 -> f32 (fp16 MFMA)",
        "data": "synthetic: W ~ N(0, 0.02) seed 1 quantized to Q4_0 (ggml reference rule), X ~ N(0, 1)",
        "config": {"workload": "single Q4_0 matmul (BASELINE.json configs[0])", "M": M, "N": N, "K": K,
                   "weight_copies": copies, "algorithmic_bytes": alg, "us_per_call": round(us, 3),
                   "us_matmul_kernel": round(us_gemm, 3), "read_floor_us": round(us_read, 3),
                   "floor_frac": round(us_read / us_gemm, 4)},
        "roofline": {"kernel": "k_q4_gemm_s", "bound": "hbm", "achieved": round(gbs_k, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(gbs_k * 1e9 / HBM_PEAK, 4),
                     "traffic": profile_traffic("matmul_q4_0_b8_4096x4096_traffic.json", "k_q4_gemm"),
                     "traffic_source": "profiles/matmul_q4_0_b8_4096x4096_traffic.md",
                     "bytes_per_launch": alg, "us_per_launch": round(us_gemm, 3)},
        "cpu_baseline": cpu,
    }
    return line


def config2_case(seed=2, n_seq=32, page=32, lo=256, hi=4096, n_share=8, share_cells=1024):
    """configs[1] (C2): contexts ~ U[lo, hi] (the n_share sharers' from [share_cells, hi], so each holds the whole
    shared prefix), the page table a seeded permutation of one pool, sequences 0 .. n_share - 1 sharing the pages of
    their first share_cells cells. Returns (ctx, page table [n_seq][max_pages] (-1: none), pool pages)."""
    import numpy as np
    r = np.random.default_rng(seed)
    ctx = r.integers(lo, hi + 1, n_seq)
    ctx[:n_share] = r.integers(share_cells, hi + 1, n_share)
    maxp = (hi + page - 1) // page
    sp = share_cells // page
    npages = [(c + page - 1) // page for c in ctx]
    need = sum(npages) - (n_share - 1) * sp if n_share else sum(npages)
    perm = r.permutation(need).astype(np.int32)
    pt = np.full((n_seq, maxp), -1, np.int32)
    nxt = 0
    shared = perm[:sp] if n_share else None
    if n_share:
        nxt = sp
    for s in range(n_seq):
        for c in range(npages[s]):
            if s < n_share and c < sp:
                pt[s, c] = shared[c]
            else:
                pt[s, c] = perm[nxt]
                nxt += 1
    return ctx, pt, need


def bench_attn(args):
    """configs[1] (C2): paged GQA decode attention, one layer: 32 sequences, 32 query heads, 8 KV heads, head_dim 128,
    contexts ~ U[256, 4096] (seed 2), fp16 K/V ~ N(0, 1) in 32-cell pages of one pool (a seeded permutation), 8
    sequences sharing the pages of their first 1024 cells; q ~ N(0, 1), scale 1/sqrt(128). One row per sequence at
    its last position. 3 pool copies (beyond the Infinity Cache) are used in turn; launches replay from a HIP graph.
    value = unique algorithmic bytes (every cell once, shared pages once; q, output, page-table entries) / time."""
    import ctypes as C

    import numpy as np
    import torch

    import sllm_next as S

    U = Dev
    L = S.lib()
    H, KVH, D, page = 32, 8, 128, 32
    n_seq, n_share, share = 32, 8, 1024
    ctx, pt, need = config2_case(page=page, n_seq=n_seq, n_share=n_share, share_cells=share)
    seq = np.arange(n_seq, dtype=np.int32)
    pos = (ctx - 1).astype(np.int32)
    r = np.random.default_rng(3)
    q = r.standard_normal((n_seq, H, D), dtype=np.float32)
    copies = 3
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2)
    pools = [(torch.randn(need * KVH * page * D, generator=gen, device="cuda").half(),
              torch.randn(need * KVH * page * D, generator=gen, device="cuda").half()) for _ in range(copies)]
    dpt, dq = U.copy(pt), U.copy(q)
    out = U.empty(n_seq * H * D * 4)
    err = C.create_string_buffer(256)
    # the planner sees the page table: the sharers' common 1024-cell prefix is read once per (chunk, KV head)
    ptc = np.ascontiguousarray(pt, np.int32)
    plan = L.snk_attn_new_pt(n_seq, seq.ctypes.data, pos.ctypes.data, H, KVH, pt.shape[1], page, args.attn_mode,
                             ptc.ctypes.data, err, 256)
    assert plan, err.value
    whole = bool(L.snk_attn_whole(plan))
    fold = bool(L.snk_attn_fold(plan, 0))  # (the two launches: the fold measured slower, and this list shares chunks)
    scale = C.c_float(1.0 / np.sqrt(D))

    def run(i, st):
        kp, vp = pools[i % copies]
        L.snk_attn_run(plan, U.ptr(dq), H * D, U.ptr(kp), U.ptr(vp), U.ptr(dpt), scale, U.ptr(out), H * D, st)

    st0 = U.stream()
    for _ in range(args.warmup):
        run(0, st0)
    torch.cuda.synchronize()
    n = max(36, args.steps)
    us = graph_us(run, n)
    cells = int(ctx.sum()) - int(np.minimum(ctx[1:n_share], share).sum())
    pages = int(sum((c + page - 1) // page for c in ctx))
    alg = cells * KVH * D * 2 * 2 + 2 * n_seq * H * D * 4 + 4 * pages
    alg_per_seq = int(ctx.sum()) * KVH * D * 2 * 2 + 2 * n_seq * H * D * 4 + 4 * pages
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        O.build() if not os.path.exists(O.LIB_PATH) else None
        kp, vp = pools[0]
        # (K regions are stored chunk-major, [16][cells][8]: back to cell-major for the oracle)
        kh = np.ascontiguousarray(kp.cpu().numpy().view(np.uint16).reshape(need, KVH, D // 8, page, 8)
                                  .transpose(0, 1, 3, 2, 4)).reshape(need, KVH, page, D)
        vh = vp.cpu().numpy().view(np.uint16).reshape(need, KVH, page, D)
        run(0, st0)
        got = U.host(out, np.float32)[:n_seq * H * D].reshape(n_seq, H, D)
        nt = cpu_threads()

        def attn_cpu():
            return O.paged_attn(q, seq, pos, KVH, kh, vh, page, pt, 1.0 / np.sqrt(D), nthreads=nt)

        want = attn_cpu()
        dt, reps = median_time(attn_cpu)
        log(f"[bench] max |GPU - oracle| {float(np.abs(got - want).max()):.3g}")
        cpu = {"value": round(alg / dt / 1e9, 3), "unit": "GB/s", **cpu_info(), "kind": "port",
               "sample": f"the same 32-row attention through oracle/oracle.c (fp32 softmax over fp16 cells): median "
                         f"of {reps} warm calls, {dt * 1e3:.1f} ms each"}
    gbs = alg / (us * 1e-6) / 1e9
    kern = "k_attn_whole" if whole else "k_attn_fold" if fold else "k_attn_part + k_attn_merge"
    log(f"[bench] C2 attention: {us:.2f} us per launch ({kern}), {alg / 1e6:.1f} MB unique, "
        f"{alg_per_seq / 1e6:.1f} MB counting shared pages per sequence")
    line = {
        "metric": "paged GQA decode attention GB/s (unique algorithmic bytes), 32 seqs, ctx U[256,4096], 32-cell pages",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": n, "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 K/V, f32 q / softmax / output (fp16 MFMA with split operands)",
        "data": "synthetic: contexts U[256, 4096] seed 2 (sharers' from [1024, 4096]), K/V ~ N(0, 1) fp16, q ~ N(0, 1)",
        "config": {"workload": "paged GQA decode attention, one layer (BASELINE.json configs[1])", "seqs": n_seq,
                   "heads": H, "kv_heads": KVH, "page_cells": page, "shared_prefix_seqs": n_share,
                   "shared_prefix_cells": share, "mean_ctx": round(float(ctx.mean()), 1), "form": kern,
                   "unique_bytes": alg, "bytes_counting_shared_per_seq": alg_per_seq,
                   "GBps_counting_shared_per_seq": round(alg_per_seq / (us * 1e-6) / 1e9, 1)},
        "roofline": {"kernel": kern, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(gbs * 1e9 / HBM_PEAK, 4),
                     "traffic": profile_traffic("attn_config2_b32_ctx256_4096_page32_traffic.json", kern),
                     "traffic_source": "profiles/attn_config2_b32_ctx256_4096_page32_traffic.md",
                     "bytes_per_launch": alg, "us_per_launch": round(us, 3)},
        "cpu_baseline": cpu,
    }
    L.snk_attn_free(plan)
    return line


if __name__ == "__main__":
    main()
