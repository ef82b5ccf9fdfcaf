"""Python binding of libsn_hip.so: the sn.h engine ABI, the kernel-level sn_kernels.h ABI and the sn_synth.h tool.

This mirrors the reference's Rust binding of the same C ABI (engine/sllm-server/src/next_engine/ffi.rs:16-63: one
`extern "C"` declaration per sn.h function, and `call`, which turns a non-zero return plus the 512-byte error buffer
into an error, ffi.rs:65-73). The library must be built (sonic-llm_amd/Makefile); there is no fallback: loading fails
loudly when it is missing.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsn_hip.so")

_lib = None


class SnError(RuntimeError):
    def __init__(self, rc: int, message: str):
        super().__init__(f"{message} (rc {rc})")
        self.rc = rc


def lib():
    """The loaded library (raises when it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C sonic-llm_amd` (or __graft_entry__.build())")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
I = C.c_int
I32P = C.POINTER(C.c_int32)
CH = C.c_char_p

# (name, restype, argtypes) of every exported function, in the order of include/sn.h, sn_kernels.h, sn_synth.h
SN_API = [
    ("sn_open", P, [CH, CH, I, I, I, I, CH, I]),
    ("sn_check", I, [CH, C.POINTER(I), CH, I]),
    ("sn_quiet_rows", I, [CH]),
    ("sn_n_vocab", I, [P]),
    ("sn_n_ctx_train", I, [P]),
    ("sn_arch", CH, [P]),
    ("sn_step", I, [P, I, P, P, P, I, I, I, P, P, I, CH, I]),
    ("sn_last_gpu_ms", C.c_double, [P]),
    ("sn_logits", I, [P, I, P, CH, I]),
    ("sn_logits_rows", I, [P, I, P, P, CH, I]),
    ("sn_want_probs", None, [P, I]),
    ("sn_probs", I, [P, I, P, CH, I]),
    ("sn_latent", I, [P, I, P, P, P, CH, I]),
    ("sn_n_embd", I, [P]),
    ("sn_soft_config", I, [P, C.c_float, I, P, I, CH, I]),
    ("sn_soft_rows", I, [P, I, P, I, P, CH, I]),
    ("sn_embed_rows", I, [P, I, P, P, CH, I]),
    ("sn_embd_norm", C.c_float, [P]),
    ("sn_set_eog", I, [P, P, I]),
    ("sn_no_end", None, [P, I, I]),
    ("sn_copy", I, [P, I, I, I, CH, I]),
    ("sn_clear", I, [P, I, I, I, CH, I]),
    ("sn_cut_ok", I, [P, I, I]),
    ("sn_recurrent", I, [P]),
    ("sn_guess_head", I, [P]),
    ("sn_guess_on", I, [P, I]),
    ("sn_guess", I, [P, I, C.c_int32, I, I, P, CH, I]),
    ("sn_draft_rows", I, [P, I, I]),
    ("sn_small_rows", I, [P]),
    ("sn_chat_exact", I, [P]),
    ("sn_mark", I, [P, I]),
    ("sn_state_take", I, [P, I]),
    ("sn_cut_best", I, [P, I, I]),
    ("sn_pages_total", I, [P]),
    ("sn_pages_free", I, [P]),
    ("sn_page_bytes", C.c_size_t, [P]),
    ("sn_seq_pages", I, [P, I, C.POINTER(I)]),
    ("sn_win_need", I, [P, I]),
    ("sn_win_room", I, [P]),
    ("sn_win_pages", I, [P, I]),
    ("sn_kv_bytes", C.c_size_t, [P, I]),
    ("sn_kv_save", I, [P, I, I, P, CH, I]),
    ("sn_kv_load", I, [P, I, I, P, CH, I]),
    ("sn_trim", C.c_size_t, [P, I]),
    ("sn_trim_pending", I, [P]),
    ("sn_mem_used", C.c_size_t, [P]),
    ("sn_state_bytes", C.c_size_t, [P]),
    ("sn_state_entries", I, [P, I]),
    ("sn_close", None, [P]),
]
SNK_API = [
    ("snk_q4_stripes_bytes", C.c_size_t, [I, I]),
    ("snk_q4_repack", I, [P, I, I, P, P]),
    ("snk_q4_dequant", I, [P, I, I, P, P]),
    ("snk_xa_bytes", C.c_size_t, [I, I]),
    ("snk_q6k_tiles_bytes", C.c_size_t, [I, I]),
    ("snk_q6k_repack", I, [P, I, I, P, P]),
    ("snk_q6k_dequant", I, [P, I, I, P, P]),
    ("snk_xk_bytes", C.c_size_t, [I, I]),
    ("snk_quant_q8k", I, [P, I, I, I, P, C.c_float, P, P]),
    ("snk_q6k_gemm", I, [P, P, I, I, I, P, I, P]),
    ("snk_q8_tiles_bytes", C.c_size_t, [I, I]),
    ("snk_q8_repack", I, [P, I, I, P, P]),
    ("snk_q8_dequant", I, [P, I, I, P, P]),
    ("snk_q8_workspace_bytes", C.c_size_t, [I, I, I]),
    ("snk_q8_gemm", I, [P, P, I, I, I, P, I, I, P, C.c_size_t, P]),
    ("snk_quant_act", I, [P, I, I, I, P, C.c_float, P, P]),
    ("snk_q4_workspace_bytes", C.c_size_t, [I, I, I]),
    ("snk_q4_plan", I, [I, I, I, C.POINTER(I), C.POINTER(I)]),
    ("snk_q4_gemm", I, [P, P, I, I, I, P, I, I, P, C.c_size_t, P]),
    ("snk_q4_gemm_swiglu", I, [P, P, I, I, I, P, P, P]),
    ("snk_q4_gemm_noalloc", I, [P, P, I, I, I, P, I, I, P, CH, I]),
    ("snk_q4_gemm_time", C.c_double, [P, I, P, I, I, I, P, I, P, C.c_size_t, I, P]),
    ("snk_q4_gemm_plan_time", C.c_double, [P, I, P, I, I, I, P, C.c_size_t, I, I, I, I, P]),
    ("snk_read_time", C.c_double, [P, I, C.c_size_t, P, I, P]),
    ("snk_q4_gemm_plan_sums", I, [P, P, I, I, I, P, P, C.c_size_t, I, I, I, P]),
    ("snk_attn_new", P, [I, P, P, I, I, I, I, CH, I]),
    ("snk_attn_new_mode", P, [I, P, P, I, I, I, I, I, CH, I]),
    ("snk_attn_new_pt", P, [I, P, P, I, I, I, I, I, P, CH, I]),
    ("snk_attn_run", I, [P, P, I, P, P, P, C.c_float, P, I, P]),
    ("snk_attn_time", C.c_double, [P, P, I, P, P, P, C.c_float, P, I, I, P]),
    ("snk_attn_whole", I, [P]),
    ("snk_attn_runs", I, [P]),
    ("snk_attn_fold", I, [P, I]),
    ("snk_attn_xcd_faults", I, [P]),
    ("snk_attn_free", None, [P]),
    ("snk_qk_rope", I, [P, I, I, I, I, P, P, C.c_float, C.c_float, P, P, P, I, I, P, P, P]),
    ("snk_moe_router", I, [P, I, I, P, I, P, P]),
    ("snk_moe_tile_rows", I, [I, I, I]),
    ("snk_moe_select", I, [P, I, I, I, P, P, P, P, P, P, P]),
    ("snk_moe_route", I, [P, I, I, P, I, I, P, P, P, P, P, P, P, P, P]),
    ("snk_gemm_grouped", I, [I, P, C.c_size_t, P, P, I, P, I, I, I, P, C.c_size_t, P, P]),
    ("snk_argmax_workspace_bytes", C.c_size_t, [I, I]),
    ("snk_argmax", I, [P, I, I, P, I, P, P, P, P, C.c_size_t, P]),
    ("snk_mfma_probe", I, [P, P, P, P]),
]
EXT_API = [
    ("snx_graphs", None, [P, I]),
    ("snx_attn_mode", None, [P, I]),
    ("snx_fuse", I, [P, I]),
    ("snx_xcd_faults", I, [P]),
    ("snx_step_key", I, [I, I, I, I, I, P, P, P, I, P]),
    ("snx_chain_count", C.c_long, [P, I]),
    ("snx_graph_count", C.c_long, [P, I]),
    ("snx_prof", None, [P, I]),
    ("snx_prof_read", I, [P, I, C.POINTER(C.c_double), C.POINTER(I), C.POINTER(C.c_double)]),
    ("snx_fill_kv", I, [P, I, I, C.c_uint64, CH, I]),
    ("snx_debug_read", I, [P, I, P, C.c_size_t]),
    ("snx_spec_step", I, [P, I, P, P, P, I, P, P, P, CH, I]),
]
SYNTH_API = [
    ("snx_write_model", I, [CH, P, C.c_uint64, I, CH, I]),
    ("snx_quantize_q4_0", None, [P, P, C.c_int64]),
    ("snx_quantize_q8_0", None, [P, P, C.c_int64]),
]


def _declare(L):
    for name, res, args in SN_API + SNK_API + EXT_API + SYNTH_API:
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data_as(C.c_void_p)
    return C.c_void_p(a)


def call(f, *args):
    """A library call whose last two arguments are the error buffer: its return code, or SnError with the reason."""
    buf = C.create_string_buffer(512)
    rc = f(*args, buf, 512)
    if rc != 0:
        raise SnError(rc, buf.value.decode(errors="replace"))
    return rc


# ---- sn_synth.h ----
class ModelCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                                       "n_expert", "n_expert_used", "n_ff_exp", "nextn")] + \
               [(n, C.c_float) for n in ("rope_base", "eps", "w_std", "emb_std")] + \
               [(n, C.c_int) for n in ("wtype", "embd_type", "tied")]


def model_cfg(n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, head_dim=128, n_expert=0, n_expert_used=0,
              n_ff_exp=0, nextn=0, rope_base=1e6, eps=1e-6, w_std=0.02, emb_std=0.02, wtype=2, embd_type=0,
              tied=0) -> ModelCfg:
    """wtype: the matrices' block type, 2 Q4_0 or 8 Q8_0; embd_type: token_embd's, 0 F32, 2 Q4_0, 8 Q8_0, 14 Q6_K;
    tied: no output.weight (the LM head is token_embd)."""
    return ModelCfg(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_expert, n_expert_used, n_ff_exp,
                    nextn, rope_base, eps, w_std, emb_std, wtype, embd_type, tied)


# The configs' models
QWEN3_4B = dict(n_layer=36, n_embd=2560, n_head=32, n_head_kv=8, n_ff=9728, n_vocab=151936)
QWEN3_30B_A3B = dict(n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, n_ff=6144, n_vocab=151936, n_expert=128,
                     n_expert_used=8, n_ff_exp=768)


def q4_plan(N: int, K: int, wt: int = 2) -> tuple:
    """snk_q4_plan (host only): (stripes per wavefront, k-slices) of an N x K matrix's matmul launches."""
    spw, ks = C.c_int(), C.c_int()
    if lib().snk_q4_plan(N, K, wt, C.byref(spw), C.byref(ks)) != 0:
        raise SnError(-1, "snk_q4_plan: bad shape or type")
    return spw.value, ks.value


def cached_model(cfg_kw: dict, seed: int, path: str | None = None, log=None) -> str:
    """A random-init model file of configuration cfg_kw (model_cfg's keywords) and seed, written once into
    $SN_BENCH_DIR (default /tmp) under a name made of the two and reused while its ".done" marker exists (the
    benchmark and the config-shaped tests share the files)."""
    d = os.environ.get("SN_BENCH_DIR") or "/tmp"
    tag = ("_mtp" if cfg_kw.get("nextn") else "") + (f"_moe{cfg_kw['n_expert']}" if cfg_kw.get("n_expert") else "") + \
          ("_q8" if cfg_kw.get("wtype") == 8 else "") + ("_q6kt" if cfg_kw.get("tied") else "")
    path = path or os.path.join(d, f"sonic_qwen3_{cfg_kw['n_layer']}L_{cfg_kw['n_embd']}{tag}_{seed}.gguf")
    done = path + ".done"
    if not (os.path.exists(path) and os.path.exists(done)):
        import time
        t = time.time()
        write_model(path, model_cfg(**cfg_kw), seed, nthreads=int(os.environ.get("OMP_NUM_THREADS", "0") or 0))
        open(done, "w").write("ok")
        if log:
            log(f"wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    return path


def write_model(path: str, cfg: ModelCfg, seed: int, nthreads: int = 0) -> None:
    call(lib().snx_write_model, path.encode(), C.byref(cfg), seed, nthreads)


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 18, np.uint8)
    lib().snx_quantize_q4_0(_p(x), _p(out), x.size)
    return out.reshape(x.shape[:-1] + (x.shape[-1] // 32 * 18,))


def step_key(H: int, KVH: int, page_cells: int, mode: int, seq, pos):
    """snx_step_key (host only): the graph key sn_step forms for a step of rows (seq, pos), every row sampled, and
    whether its attention runs as whole groups. Two steps replay one captured graph exactly when their keys are equal."""
    seq = np.ascontiguousarray(seq, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    key = np.zeros(64, np.int64)
    whole = C.c_int(-1)
    n = lib().snx_step_key(H, KVH, page_cells, mode, seq.size, _p(seq), _p(pos), _p(key), key.size, C.byref(whole))
    if n < 0:
        raise SnError(n, "snx_step_key: bad arguments")
    return tuple(int(v) for v in key[:n]), bool(whole.value)


# ---- sn.h ----
class Engine:
    """sn_open .. sn_close with numpy arrays in and out."""

    def __init__(self, path: str, slots: int, ctx: int, max_rows: int, pages: int = 0):
        L = lib()
        buf = C.create_string_buffer(512)
        self.e = L.sn_open(path.encode(), b"", slots, ctx, max_rows, pages, buf, 512)
        if not self.e:
            raise SnError(-1, buf.value.decode(errors="replace"))
        self.L = L
        self.V = L.sn_n_vocab(self.e)
        self.E = L.sn_n_embd(self.e)

    def close(self):
        if self.e:
            self.L.sn_close(self.e)
            self.e = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def step(self, tok, seq, pos, out_rows, n_write=None, n_fast=0, chain=0):
        tok = np.ascontiguousarray(tok, np.int32)
        seq = np.ascontiguousarray(seq, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        out_rows = np.ascontiguousarray(out_rows, np.int32)
        R = tok.size
        n_write = R if n_write is None else n_write
        out = np.zeros(max(out_rows.size, 1), np.int32)
        call(self.L.sn_step, self.e, R, _p(tok), _p(seq), _p(pos), n_write, n_fast, out_rows.size, _p(out_rows),
             _p(out), chain)
        return out[:out_rows.size]

    def logits(self, ks) -> np.ndarray:
        ks = np.ascontiguousarray(ks, np.int32)
        dst = np.empty((ks.size, self.V), np.float32)
        call(self.L.sn_logits_rows, self.e, ks.size, _p(ks), _p(dst))
        return dst

    def probs(self, n_out) -> np.ndarray:
        dst = np.empty((n_out, 8), np.float32)
        call(self.L.sn_probs, self.e, n_out, _p(dst))
        return dst

    def want_probs(self, on: bool):
        self.L.sn_want_probs(self.e, int(on))

    def set_eog(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        if self.L.sn_set_eog(self.e, _p(ids), ids.size) != 0:
            raise SnError(-1, "sn_set_eog")

    def no_end(self, slot, on):
        self.L.sn_no_end(self.e, slot, int(on))

    def copy(self, src, dst, n):
        call(self.L.sn_copy, self.e, src, dst, n)

    def clear(self, slot, a, b):
        call(self.L.sn_clear, self.e, slot, a, b)

    def kv_save(self, slot, n) -> np.ndarray:
        nb = self.L.sn_kv_bytes(self.e, n)
        dst = np.empty(nb // 2, np.uint16)
        call(self.L.sn_kv_save, self.e, slot, n, _p(dst))
        return dst

    def kv_load(self, slot, n, src: np.ndarray):
        call(self.L.sn_kv_load, self.e, slot, n, _p(np.ascontiguousarray(src)))

    def pages_free(self):
        return self.L.sn_pages_free(self.e)

    def pages_total(self):
        return self.L.sn_pages_total(self.e)

    def seq_pages(self, seq):
        own = C.c_int()
        n = self.L.sn_seq_pages(self.e, seq, C.byref(own))
        return n, own.value

    def last_gpu_ms(self):
        return self.L.sn_last_gpu_ms(self.e)

    def fill_kv(self, slot, n, seed):
        call(self.L.snx_fill_kv, self.e, slot, n, seed)

    # ---- the guess head (sn_guess_head / sn_guess_on / sn_guess) and the fused draft-verify step
    def guess_head(self) -> bool:
        return bool(self.L.sn_guess_head(self.e))

    def guess_on(self, on: bool) -> bool:
        return bool(self.L.sn_guess_on(self.e, int(on)))

    def guess(self, seq, tok, pos, k) -> np.ndarray:
        out = np.empty(k, np.int32)
        call(self.L.sn_guess, self.e, int(seq), int(tok), int(pos), int(k), _p(out))
        return out

    def spec_step(self, seq, last, pos, k, force=None):
        """snx_spec_step: per sequence (accepted + 1, tokens [k + 1] with -1 after the bonus)."""
        seq = np.ascontiguousarray(seq, np.int32)
        last = np.ascontiguousarray(last, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        n = seq.size
        fr = None if force is None else np.ascontiguousarray(force, np.uint8).reshape(n, k)
        out_n = np.empty(n, np.int32)
        out_tok = np.empty((n, k + 1), np.int32)
        call(self.L.snx_spec_step, self.e, n, _p(seq), _p(last), _p(pos), int(k), _p(fr) if fr is not None else None,
             _p(out_n), _p(out_tok))
        return out_n, out_tok

    def graphs(self, on: bool):
        """snx_graphs: replay each step shape's device work as a HIP graph (the default) or launch it eagerly."""
        self.L.snx_graphs(self.e, int(on))

    def attn_mode(self, mode: int):
        """snx_attn_mode: the attention work list's form, -1 per step (default), 0 per-chunk + merge, 1 whole groups,
        2 run items for prompt rows wherever possible."""
        self.L.snx_attn_mode(self.e, int(mode))

    def fuse(self, on: bool) -> bool:
        """snx_fuse: the matmul epilogues fused into decode-sized steps (q|k|v + RoPE, gate|up + SwiGLU), on (where
        sn_open's XCD probe allows) or off (the split path, the same bits); returns whether they are on."""
        return bool(self.L.snx_fuse(self.e, int(on)))

    def xcd_faults(self) -> int:
        """snx_xcd_faults: 1 when a fused launch ran a workgroup on another XCD than predicted, else 0."""
        return self.L.snx_xcd_faults(self.e)

    def chain_count(self) -> tuple:
        """(queued steps taken, queued steps dropped) since the engine opened (sn_step's chain)."""
        return self.L.snx_chain_count(self.e, 0), self.L.snx_chain_count(self.e, 1)

    def graph_count(self) -> tuple:
        """(steps captured as a new graph, steps replayed from the cached graph) since the engine opened."""
        return self.L.snx_graph_count(self.e, 0), self.L.snx_graph_count(self.e, 1)

    def prof(self, on: bool):
        self.L.snx_prof(self.e, int(on))

    KINDS = ("gemm", "attn", "quant", "rope", "other", "merge")

    def prof_read(self) -> dict:
        out = {}
        for k, name in enumerate(self.KINDS):
            ms, n, b = C.c_double(), C.c_int(), C.c_double()
            self.L.snx_prof_read(self.e, k, C.byref(ms), C.byref(n), C.byref(b))
            out[name] = {"ms": ms.value, "launches": n.value, "bytes": b.value}
        return out
