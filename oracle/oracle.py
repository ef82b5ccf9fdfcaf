"""ctypes face of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product package. Every function restates the reference's (or ggml's) arithmetic; oracle.h names the file:line each
follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
I64 = C.c_int64


def _declare(L):
    L.or_f32_to_f16.argtypes = [C.c_float]
    L.or_f32_to_f16.restype = C.c_uint16
    L.or_f16_to_f32.argtypes = [C.c_uint16]
    L.or_f16_to_f32.restype = C.c_float
    for f in ("or_quantize_row_q4_0", "or_dequantize_row_q4_0", "or_quantize_row_q8_0", "or_dequantize_row_q8_0"):
        getattr(L, f).argtypes = [P, P, I64]
        getattr(L, f).restype = None
    L.or_vec_dot_q4_0_q8_0.argtypes = [I64, P, P]
    L.or_vec_dot_q4_0_q8_0.restype = C.c_float
    L.or_quantize_row_q8_0_ref.argtypes = [P, P, I64]
    L.or_quantize_row_q8_0_ref.restype = None
    L.or_vec_dot_q8_0_q8_0.argtypes = [I64, P, P]
    L.or_vec_dot_q8_0_q8_0.restype = C.c_float
    L.or_mul_mat_q8_0.argtypes = [P, I64, I64, P, I64, P, C.c_int]
    for f in ("or_dequantize_row_q6_K", "or_quantize_row_q8_K"):
        getattr(L, f).argtypes = [P, P, I64]
        getattr(L, f).restype = None
    L.or_vec_dot_q6_K_q8_K.argtypes = [I64, P, P]
    L.or_vec_dot_q6_K_q8_K.restype = C.c_float
    L.or_mul_mat_q6_K.argtypes = [P, I64, I64, P, I64, P, C.c_int]
    L.or_mul_mat_q4_0.argtypes = [P, I64, I64, P, I64, P, C.c_int]
    L.or_set_sum_order.argtypes = [C.c_int]
    L.or_set_sum_order.restype = None
    L.or_moe_trace.argtypes = [P, C.c_int]
    L.or_moe_trace.restype = None
    L.or_moe_trace_count.restype = C.c_int
    L.or_mul_mat_q4_0_f64.argtypes = [P, I64, I64, P, I64, P, C.c_int]
    L.or_rmsnorm.argtypes = [P, P, I64, C.c_float, P]
    L.or_silu.argtypes = [C.c_float]
    L.or_silu.restype = C.c_float
    L.or_argmax.argtypes = [P, I64, P, C.c_int]
    L.or_argmax.restype = C.c_int32
    L.or_top2.argtypes = [P, I64, P, P, P, P, P]
    L.or_rope_cache.argtypes = [C.c_int32, C.c_float, C.c_int, P]
    L.or_qk_norm_rope.argtypes = [P, P, C.c_int, C.c_float, P, C.c_int]
    L.or_paged_attn.argtypes = [P, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P, P, C.c_int, P, C.c_int, C.c_float,
                                P, C.c_int, C.c_int]
    L.or_paged_attn_chunked.argtypes = [P, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P, P, C.c_int, P, C.c_int,
                                        C.c_float, C.c_int, P]
    L.or_moe_route.argtypes = [P, C.c_int, C.c_int, P, P]
    L.or_accept.argtypes = [P, P, C.c_int]
    L.or_accept.restype = C.c_int
    L.or_qwen3_step.argtypes = [P, P, C.c_int, P, P, P, C.c_int, P, P, P, P, P, C.c_int]
    L.or_mtp_fill.argtypes = [P, P, C.c_int, P, P, P, P, C.c_int]
    L.or_mtp_guess.argtypes = [P, P, C.c_int, C.c_int32, C.c_int, C.c_int, P, P, P, C.c_int]


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- fp16 ----
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """RNE fp16 bits (uint16) of fp32 values, via the oracle's F16C conversion."""
    x = np.ascontiguousarray(x, np.float32)
    return np.array([lib().or_f32_to_f16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def set_sum_order(reverse: bool) -> None:
    """Test hook: the Q4_0 / Q8_0 dots add their blocks' fp32 terms last block first (True) or in ggml's order."""
    lib().or_set_sum_order(int(reverse))


class MoeTrace:
    """Test hook: while open, every MoE routing of a model step records its margin (the smallest router logit chosen
    minus the largest not chosen), layer by layer, row by row; .margins() after the steps."""

    def __init__(self, cap=1 << 20):
        self.buf = np.zeros(cap, np.float32)

    def __enter__(self):
        lib().or_moe_trace(_p(self.buf), self.buf.size)
        return self

    def __exit__(self, *a):
        self.n = lib().or_moe_trace_count()
        lib().or_moe_trace(None, 0)

    def margins(self):
        return self.buf[:self.n].copy()


# ---- Q4_0 / Q8_0 ----
def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """[N][K] fp32 -> [N][K/32*18] uint8 (ggml quantize_row_q4_0_ref per row)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty((N, K // 32 * 18), np.uint8)
    lib().or_quantize_row_q4_0(_p(w), _p(out), N * K)
    return out


def dequantize_q4_0(q: np.ndarray, K: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    N = q.size // (K // 32 * 18)
    out = np.empty((N, K), np.float32)
    lib().or_dequantize_row_q4_0(_p(q), _p(out), N * K)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    out = np.empty((M, K // 32 * 34), np.uint8)
    lib().or_quantize_row_q8_0(_p(x), _p(out), M * K)
    return out


def dequantize_q8_0(q: np.ndarray, K: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    M = q.size // (K // 32 * 34)
    out = np.empty((M, K), np.float32)
    lib().or_dequantize_row_q8_0(_p(q), _p(out), M * K)
    return out


def dequantize_q6_K(q: np.ndarray, K: int) -> np.ndarray:
    """[N][K/256*210] uint8 block_q6_K rows -> [N][K] fp32 (ggml dequantize_row_q6_K)."""
    q = np.ascontiguousarray(q, np.uint8)
    N = q.size // (K // 256 * 210)
    out = np.empty((N, K), np.float32)
    lib().or_dequantize_row_q6_K(_p(q), _p(out), N * K)
    return out


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    """[M][K] fp32 -> [M][K/256*292] uint8 block_q8_K rows (ggml quantize_row_q8_K_ref)."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    out = np.empty((M, K // 256 * 292), np.uint8)
    lib().or_quantize_row_q8_K(_p(x), _p(out), M * K)
    return out


def vec_dot_q6_K_q8_K(w_row: np.ndarray, xq_row: np.ndarray, K: int) -> float:
    return float(lib().or_vec_dot_q6_K_q8_K(K, _p(np.ascontiguousarray(w_row, np.uint8)),
                                            _p(np.ascontiguousarray(xq_row, np.uint8))))


def mul_mat_q6_K(Wq: np.ndarray, K: int, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """Y[M][N] = X[M][K] . W[N][K]^T for Q6_K weights, ggml CPU semantics (Q8_K activations, vec_dot_q6_K_q8_K)."""
    Wq = np.ascontiguousarray(Wq, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    N = Wq.size // (K // 256 * 210)
    M = X.shape[0]
    Y = np.empty((M, N), np.float32)
    lib().or_mul_mat_q6_K(_p(Wq), N, K, _p(X), M, _p(Y), nthreads)
    return Y


def quantize_q8_0_ref(w: np.ndarray) -> np.ndarray:
    """[N][K] fp32 -> [N][K/32*34] uint8 (ggml quantize_row_q8_0_ref per row: the quantizer of Q8_0 model weights)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty((N, K // 32 * 34), np.uint8)
    lib().or_quantize_row_q8_0_ref(_p(w), _p(out), N * K)
    return out


def mul_mat_q8_0(Wq: np.ndarray, K: int, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """Y[M][N] = X[M][K] . W[N][K]^T for Q8_0 weights, ggml CPU semantics (Q8_0 activations, vec_dot_q8_0_q8_0)."""
    Wq = np.ascontiguousarray(Wq, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    N = Wq.size // (K // 32 * 34)
    M = X.shape[0]
    Y = np.empty((M, N), np.float32)
    lib().or_mul_mat_q8_0(_p(Wq), N, K, _p(X), M, _p(Y), nthreads)
    return Y


def mul_mat_q4_0(Wq: np.ndarray, K: int, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """Y[M][N] = X[M][K] . W[N][K]^T, ggml CPU semantics (Q8_0 activations, integer block dots)."""
    Wq = np.ascontiguousarray(Wq, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    N = Wq.size // (K // 32 * 18)
    M = X.shape[0]
    Y = np.empty((M, N), np.float32)
    lib().or_mul_mat_q4_0(_p(Wq), N, K, _p(X), M, _p(Y), nthreads)
    return Y


def mul_mat_q4_0_f64(Wq: np.ndarray, K: int, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    Wq = np.ascontiguousarray(Wq, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    N = Wq.size // (K // 32 * 18)
    M = X.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().or_mul_mat_q4_0_f64(_p(Wq), N, K, _p(X), M, _p(Y), nthreads)
    return Y


def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    wp = None if w is None else _p(np.ascontiguousarray(w, np.float32))
    n = x.shape[-1]
    for i in range(x.size // n):
        lib().or_rmsnorm(C.c_void_p(x.ctypes.data + 4 * n * i), wp, n, eps, C.c_void_p(y.ctypes.data + 4 * n * i))
    return y


def argmax(x: np.ndarray, ban=()) -> int:
    x = np.ascontiguousarray(x, np.float32)
    b = np.ascontiguousarray(np.array(ban, np.int32))
    return int(lib().or_argmax(_p(x), x.size, _p(b) if len(ban) else None, len(ban)))


def top2(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    i1, i2 = C.c_int32(), C.c_int32()
    v1, v2, lse = C.c_float(), C.c_float(), C.c_float()
    lib().or_top2(_p(x), x.size, C.byref(i1), C.byref(v1), C.byref(i2), C.byref(v2), C.byref(lse))
    return i1.value, v1.value, i2.value, v2.value, lse.value


def rope_cache(pos: int, theta_scale: float, D: int) -> np.ndarray:
    cs = np.empty(D, np.float32)
    lib().or_rope_cache(pos, theta_scale, D, _p(cs))
    return cs


def qk_norm_rope(x: np.ndarray, w: np.ndarray, eps: float, cs: np.ndarray, do_norm: bool = True) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().or_qk_norm_rope(_p(y), _p(np.ascontiguousarray(w, np.float32)), y.size, eps, _p(cs), int(do_norm))
    return y


def paged_attn(q, qseq, qpos, KVH, kpool, vpool, page_cells, pt, scale, f64=False, nthreads=0):
    """q: [nq][H][D] fp32; kpool/vpool: uint16 fp16 bits [pages][KVH][page_cells][D]; pt: [S][max_pages] int32."""
    q = np.ascontiguousarray(q, np.float32)
    nq, H, D = q.shape
    out = np.empty_like(q)
    qs = np.ascontiguousarray(qseq, np.int32)
    qp = np.ascontiguousarray(qpos, np.int32)
    pt = np.ascontiguousarray(pt, np.int32)
    lib().or_paged_attn(_p(q), nq, _p(qs), _p(qp), H, KVH, D, _p(np.ascontiguousarray(kpool)),
                        _p(np.ascontiguousarray(vpool)), page_cells, _p(pt), pt.shape[1], scale, _p(out), int(f64),
                        nthreads)
    return out


def paged_attn_chunked(q, qseq, qpos, KVH, kpool, vpool, page_cells, pt, scale, chunk):
    q = np.ascontiguousarray(q, np.float32)
    nq, H, D = q.shape
    out = np.empty_like(q)
    qs = np.ascontiguousarray(qseq, np.int32)
    qp = np.ascontiguousarray(qpos, np.int32)
    pt = np.ascontiguousarray(pt, np.int32)
    lib().or_paged_attn_chunked(_p(q), nq, _p(qs), _p(qp), H, KVH, D, _p(np.ascontiguousarray(kpool)),
                                _p(np.ascontiguousarray(vpool)), page_cells, _p(pt), pt.shape[1], scale, chunk,
                                _p(out))
    return out


def moe_route(logits: np.ndarray, k: int):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().or_moe_route(_p(lg), lg.size, k, _p(ids), _p(w))
    return ids, w


def accept(draft, target) -> int:
    d = np.ascontiguousarray(draft, np.int32)
    t = np.ascontiguousarray(target, np.int32)
    return int(lib().or_accept(_p(d), _p(t), d.size))


# ---- the Qwen3 model step ----
class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "wq", "wk", "wv", "wo", "wg",
                                          "wu", "wd", "router", "eg", "eu", "ed")]


class _Model(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int), ("n_head_kv", C.c_int),
                ("head_dim", C.c_int), ("n_ff", C.c_int), ("n_vocab", C.c_int), ("n_expert", C.c_int),
                ("n_expert_used", C.c_int), ("n_ff_exp", C.c_int), ("eps", C.c_float), ("rope_base", C.c_float),
                ("tok_embd", C.c_void_p), ("output_norm", C.c_void_p), ("output", C.c_void_p),
                ("layers", C.POINTER(_Layer)), ("mtp", C.POINTER(_Layer)), ("mtp_eh", C.c_void_p),
                ("mtp_enorm", C.c_void_p), ("mtp_hnorm", C.c_void_p), ("mtp_head_norm", C.c_void_p),
                ("wtype", C.c_int), ("head_type", C.c_int)]


class _KV(C.Structure):
    _fields_ = [("n_seq", C.c_int), ("ctx", C.c_int), ("n_layer", C.c_int), ("n_kv", C.c_int),
                ("head_dim", C.c_int), ("k", C.c_void_p), ("v", C.c_void_p)]


class Qwen3:
    """The oracle's Qwen3 model over a parsed GGUF (oracle.gguf.GGUF) and its own contiguous fp16 KV cache."""

    def __init__(self, gguf, n_seq: int, ctx: int):
        g = gguf
        a = g.kv["general.architecture"]
        self.arch = a
        self.E = int(g.kv[f"{a}.embedding_length"])
        self.n_mtp = int(g.kv.get(f"{a}.nextn_predict_layers", 0))  # block_count counts the guess head's block too
        self.L = int(g.kv[f"{a}.block_count"]) - self.n_mtp
        self.H = int(g.kv[f"{a}.attention.head_count"])
        self.KVH = int(g.kv[f"{a}.attention.head_count_kv"])
        self.D = int(g.kv.get(f"{a}.attention.key_length", self.E // self.H))
        self.F = int(g.kv.get(f"{a}.feed_forward_length", 0))
        self.NE = int(g.kv.get(f"{a}.expert_count", 0))
        self.NEU = int(g.kv.get(f"{a}.expert_used_count", 0))
        self.FE = int(g.kv.get(f"{a}.expert_feed_forward_length", 0))
        self.eps = float(g.kv[f"{a}.attention.layer_norm_rms_epsilon"])
        self.base = float(g.kv[f"{a}.rope.freq_base"])
        emb = g.tensor("token_embd.weight")
        self.V = emb.shape[0]
        self._keep = []
        # a quantized token table (Q4_0, Q8_0, Q6_K: ggml's dequantize_row_*) is used as its fp32 rows
        et = g.type_name("token_embd.weight")
        self._emb = emb if et == "F32" else {"Q4_0": dequantize_q4_0, "Q8_0": dequantize_q8_0,
                                             "Q6_K": dequantize_q6_K}[et](emb, self.E)

        def ptr(name):
            t = g.tensor(name)
            t = np.ascontiguousarray(t)
            self._keep.append(t)
            return t.ctypes.data

        layers = (_Layer * (self.L + self.n_mtp))()
        for i in range(self.L + self.n_mtp):
            p = f"blk.{i}."
            ly = layers[i]
            for f, n in (("attn_norm", "attn_norm"), ("q_norm", "attn_q_norm"), ("k_norm", "attn_k_norm"),
                         ("ffn_norm", "ffn_norm"), ("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"),
                         ("wo", "attn_output")):
                setattr(ly, f, ptr(p + n + ".weight"))
            if self.NE:
                ly.router = ptr(p + "ffn_gate_inp.weight")
                ly.eg = ptr(p + "ffn_gate_exps.weight")
                ly.eu = ptr(p + "ffn_up_exps.weight")
                ly.ed = ptr(p + "ffn_down_exps.weight")
            else:
                ly.wg = ptr(p + "ffn_gate.weight")
                ly.wu = ptr(p + "ffn_up.weight")
                ly.wd = ptr(p + "ffn_down.weight")
        self._layers = layers
        types = {"Q4_0": 2, "Q8_0": 8, "Q6_K": 14}
        wt = types[g.type_name("blk.0.attn_q.weight")]
        head = "output.weight" if "output.weight" in g.tinfo else "token_embd.weight"  # no output: tied
        self.wtype = wt
        self.head_type = types[g.type_name(head)]
        emb32 = np.ascontiguousarray(self._emb, np.float32)
        self._keep.append(emb32)
        self.m = _Model(self.L, self.E, self.H, self.KVH, self.D, self.F, self.V, self.NE, self.NEU, self.FE,
                        self.eps, self.base, emb32.ctypes.data, ptr("output_norm.weight"), ptr(head), layers)
        self.m.wtype = wt
        self.m.head_type = self.head_type
        if self.n_mtp:
            p = f"blk.{self.L}.nextn."
            self.m.mtp = C.cast(C.byref(layers, self.L * C.sizeof(_Layer)), C.POINTER(_Layer))
            self.m.mtp_eh = ptr(p + "eh_proj.weight")
            self.m.mtp_enorm = ptr(p + "enorm.weight")
            self.m.mtp_hnorm = ptr(p + "hnorm.weight")
            hn = p + "shared_head_norm.weight"
            self.m.mtp_head_norm = ptr(hn if hn in g.tinfo else "output_norm.weight")
        self.n_seq, self.ctx = n_seq, ctx
        shape = (n_seq, self.L + self.n_mtp, ctx, self.KVH, self.D)
        self.k = np.zeros(shape, np.uint16)
        self.v = np.zeros(shape, np.uint16)
        self.kv = _KV(n_seq, ctx, self.L + self.n_mtp, self.KVH, self.D, self.k.ctypes.data, self.v.ctypes.data)

    def step(self, tok, seq, pos, out_rows, want_hidden=False, nthreads=0, hn_all=None):
        """hn_all (optional float32 [R][E]): receives every row's hidden state after the output norm."""
        tok = np.ascontiguousarray(tok, np.int32)
        seq = np.ascontiguousarray(seq, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        out_rows = np.ascontiguousarray(out_rows, np.int32)
        n_out = out_rows.size
        logits = np.empty((max(n_out, 1), self.V), np.float32)
        hidden = np.empty((max(n_out, 1), self.E), np.float32) if want_hidden else None
        out_tok = np.empty(max(n_out, 1), np.int32)
        lib().or_qwen3_step(C.byref(self.m), C.byref(self.kv), tok.size, _p(tok), _p(seq), _p(pos), n_out,
                            _p(out_rows), _p(logits), _p(hidden) if want_hidden else None, _p(out_tok),
                            _p(hn_all) if hn_all is not None else None, nthreads)
        return out_tok[:n_out], logits[:n_out], (hidden[:n_out] if want_hidden else None)

    def mtp_fill(self, tok, seq, pos, hprev, nthreads=0):
        """The guess head's cache cells of rows (tok, seq, pos); hprev [R][E]: the model's normed hidden state at pos - 1."""
        tok = np.ascontiguousarray(tok, np.int32)
        seq = np.ascontiguousarray(seq, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        hp = np.ascontiguousarray(hprev, np.float32)
        lib().or_mtp_fill(C.byref(self.m), C.byref(self.kv), tok.size, _p(tok), _p(seq), _p(pos), _p(hp), nthreads)

    def mtp_guess(self, seq, tok, pos, k, hprev, nthreads=0):
        """k guesses of one sequence; returns (tokens [k], logits [k][V])."""
        out = np.empty(k, np.int32)
        lg = np.empty((k, self.V), np.float32)
        hp = np.ascontiguousarray(hprev, np.float32)
        lib().or_mtp_guess(C.byref(self.m), C.byref(self.kv), int(seq), int(tok), int(pos), int(k), _p(hp), _p(out),
                           _p(lg), nthreads)
        return out, lg
