"""An fp64 numpy restatement of the Qwen3 step, the MoE FFN and the guess head, written from the reference's own lines
(not from oracle/oracle.c), to pin the oracle's composed functions: or_qwen3_step (dense and MoE layers, the output
stage), or_mtp_fill and or_mtp_guess. Test infrastructure only.

What it follows:
  * the layer program, qwen_layers (engine/sllm-next/proto/sn_attn.inc.h:216-231): x_norm(attn_norm), q|k|v,
    qwen_rope (per-head RMSNorm of q and k, NEOX rotation of pairs (i, i + 64), K and V into the cache), attention
    over cells 0 .. pos, x += o(attention), qwen_ffn (:205-210): x_norm(ffn_norm), silu(gate) * up, x += down;
  * rmsnorm (kernels.metal:121-140): y = (x / sqrt(mean(x^2) + eps)) * w; qk_rope (kernels.metal:149-197);
  * the MoE FFN, moe_ffn (sn_layers.inc.h:129-144) with moe_topk1 (kernels.metal:3419-3467: softmax over the router
    logits, the k largest, ties to the lower id, weights p / max(sum p, 6.103515625e-5)) and moe_out
    (kernels.metal:3520-3538: the experts' rows weighted and summed in slot order, added to x);
  * the output stage, outputs (sn_encode.inc.h:304-317): gather, rmsnorm(output_norm), the LM head, argmax;
  * the guess head: guess_row (sn_cache.inc.h:357-369): [rmsnorm(embed(tok)) * enorm ; rmsnorm(h) * hnorm] through
    eh_proj, the head's block, rmsnorm(shared_head_norm), the LM head, argmax; and mtp_fill (sn_state.inc.h:283-313):
    the head's K / V cells of a step's rows from eh_proj([enorm(embed(tok)); hnorm(h_before)]), the block's attn_norm,
    k (QK-norm, RoPE) and v.

ggml's CPU arithmetic, operation by operation: the fp32 input rows of a Q4_0 / Q8_0 matmul are quantized to Q8_0 (x86
quantize_row_q8_0: d = amax / 127 stored as fp16, q = round-half-even(x * 127 / amax), in fp32), a row's dot is the
generic vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0 (exact integer block sums, then fp32 terms sumi * d_w * d_x added block by
block), norms are rms_norm then mul (the fp32 squares summed in double, fp32 scale and products), RoPE angles are
ggml_rope_cache_init's (theta_i = pos * s^i by i fp32 multiplies) with the C library's cosf / sinf, SwiGLU is
ggml_silu_f32 (x / (1 + expf(-x))), attention is an fp32 two-pass softmax (the oracle's documented fp32 form:
scores summed over the dims in order, expf, the sum in double, p times fp32 1 / l, the outputs summed over the cells in
order), the MoE router is an fp32 dot in element order with moe_topk1's fp32 weights, and K / V cells are stored as
fp16. Every op's result is an fp32 tensor. So the restatement and the oracle must agree bit for bit: any difference is
a difference in what is computed, not in how it is rounded.
"""
import ctypes

import numpy as np

D = 128

# the C library's single-precision exp, cos and sin (the functions ggml's CPU path calls: ggml_silu_f32, soft_max,
# ggml_rope_cache_init), element by element
_libm = ctypes.CDLL("libm.so.6")
for _f in ("expf", "cosf", "sinf"):
    getattr(_libm, _f).restype = ctypes.c_float
    getattr(_libm, _f).argtypes = [ctypes.c_float]


def _f32_map(f, x):
    x = np.asarray(x, np.float32)
    return np.array([f(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def expf(x):
    return _f32_map(_libm.expf, x)


def f32(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float64)


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


class QMat:
    """a matrix of GGUF Q4_0 / Q8_0 rows as integers q [..., N, K] (Q4_0: the low nibbles of bytes 0..15, then the
    high ones, minus 8; Q8_0: the int8 values) and fp16 scales d [..., N, K / 32] (block_q4_0 / block_q8_0,
    kernels.metal:7-9, :21-28)"""

    def __init__(self, raw: np.ndarray, tname: str, K: int):
        lead = raw.shape[:-1]
        self.q8 = tname == "Q8_0"
        if tname == "Q4_0":
            b = np.ascontiguousarray(raw).reshape(-1, 18)
            qs = b[:, 2:]
            q = np.concatenate([(qs & 15).astype(np.int32), (qs >> 4).astype(np.int32)], 1) - 8
        elif tname == "Q8_0":
            b = np.ascontiguousarray(raw).reshape(-1, 34)
            q = b[:, 2:].copy().view(np.int8).astype(np.int32)
        else:
            raise ValueError(tname)
        self.d = b[:, :2].copy().view(np.float16).astype(np.float32).reshape(lead + (K // 32,))
        self.q = q.reshape(lead + (K,))

    def __getitem__(self, e):  # expert e of a stacked [NE][N][K] matrix
        m = QMat.__new__(QMat)
        m.q8, m.q, m.d = self.q8, self.q[e], self.d[e]
        return m

    def values(self):
        return self.q.astype(np.float64) * np.repeat(self.d.astype(np.float64), 32, axis=-1)


def q8_quantize(x: np.ndarray):
    """rows of fp32 values -> ggml x86 quantize_row_q8_0: integers q [..., K] and fp16 scales d [..., K / 32]"""
    x = np.asarray(x, np.float32)
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(1, keepdims=True)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(amax != 0, np.float32(127.0) / np.where(amax != 0, amax, 1), np.float32(0)).astype(np.float32)
    v = (b * inv).astype(np.float32)
    q = np.rint(v).astype(np.int32)
    return q.reshape(x.shape), d.astype(np.float16).astype(np.float32).reshape(x.shape[:-1] + (x.shape[-1] // 32,))


def matmul(W: QMat, x: np.ndarray) -> np.ndarray:
    """ggml's CPU mul_mat of Q4_0 / Q8_0 weights: x [M][K] fp32 rows quantized to Q8_0, per output the integer block
    sums sumi and, block by block, sumf += sumi * d_w * d_x in fp32 (Q4_0: (sumi * d_w) * d_x; Q8_0: sumi * (d_w *
    d_x)), ggml's generic vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0"""
    qx, dx = q8_quantize(x)
    M, K = qx.shape
    N, nb = W.q.shape[0], K // 32
    isum = np.einsum("mbj,nbj->mnb", qx.reshape(M, nb, 32).astype(np.int64),
                     W.q.reshape(N, nb, 32).astype(np.int64)).astype(np.float32)
    acc = np.zeros((M, N), np.float32)
    for b in range(nb):
        if W.q8:
            t = isum[:, :, b] * (W.d[None, :, b] * dx[:, None, b])
        else:
            t = (isum[:, :, b] * W.d[None, :, b]).astype(np.float32) * dx[:, None, b]
        acc = (acc + t.astype(np.float32)).astype(np.float32)
    return acc.astype(np.float64)


def rmsnorm(x, w, eps):
    """ggml rms_norm then mul (rmsnorm, kernels.metal:121-140): the fp32 squares summed in double, mean = sum / n and
    scale = 1 / sqrt(mean + eps) in fp32, y = x * scale, then y * w, each product rounded to fp32"""
    x = np.asarray(x, np.float32)
    mean = ((x * x).astype(np.float64).sum(-1, keepdims=True) / x.shape[-1]).astype(np.float32)
    scale = (np.float32(1.0) / np.sqrt((mean + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = (x * scale).astype(np.float32)
    return (y * np.asarray(w, np.float32)).astype(np.float64) if w is not None else y.astype(np.float64)


def attend(q, ks, vs):
    """softmax(q . K^T / sqrt(128)) . V of one query over its cells (attn_part / attn_merge, kernels.metal:1122-1192),
    in the fp32 steps of a two-pass softmax (the oracle's fp32 form, or_paged_attn): each score an fp32 sum over the
    dims in order, times the scale; p = exp(s - max) rounded to fp32; l their sum in double; p times fp32 1 / l; each
    output an fp32 sum over the cells in order"""
    q32, k32, v32 = (np.asarray(a, np.float32) for a in (q, ks, vs))
    s = np.zeros(k32.shape[0], np.float32)
    for d in range(D):
        s = (s + (q32[d] * k32[:, d]).astype(np.float32)).astype(np.float32)
    s = (s * np.float32(1.0 / np.sqrt(np.float32(D)))).astype(np.float32)
    p = expf((s - s.max()).astype(np.float32))
    p = (p * np.float32(1.0 / p.astype(np.float64).sum())).astype(np.float32)
    o = np.zeros(D, np.float32)
    for c in range(k32.shape[0]):
        o = (o + (p[c] * v32[c]).astype(np.float32)).astype(np.float32)
    return o.astype(np.float64)


def silu(g):
    """ggml_silu_f32: x / (1 + expf(-x)) in fp32"""
    g = np.asarray(g, np.float32)
    return (g / (np.float32(1.0) + expf(-g)).astype(np.float32)).astype(np.float32).astype(np.float64)


class Model:
    """the GGUF's tensors as fp64 (weights dequantized), a Qwen3 or Qwen3-MoE model with an optional guess head"""

    def __init__(self, g):
        a = g.kv["general.architecture"]
        kv = lambda k, dflt=None: g.kv.get(f"{a}.{k}", dflt)
        self.n_mtp = int(kv("nextn_predict_layers", 0))
        self.L = int(kv("block_count")) - self.n_mtp
        self.E, self.H, self.KVH = int(kv("embedding_length")), int(kv("attention.head_count")), int(
            kv("attention.head_count_kv"))
        self.NE, self.NEU = int(kv("expert_count", 0)), int(kv("expert_used_count", 0))
        self.eps, self.base = float(kv("attention.layer_norm_rms_epsilon")), float(kv("rope.freq_base"))
        E = self.E

        def w(name):
            t = g.tensor(name)
            tn = g.type_name(name)
            K = g.tinfo[name][0][0]
            return np.asarray(t, np.float64) if tn == "F32" else QMat(t, tn, K)

        self.emb = w("token_embd.weight")
        assert isinstance(self.emb, np.ndarray), "an F32 token table"
        self.V = self.emb.shape[0]
        self.out_norm = w("output_norm.weight")
        self.head = w("output.weight") if "output.weight" in g.tinfo else self.emb
        assert g.type_name("output.weight" if "output.weight" in g.tinfo else "token_embd.weight") in ("Q4_0", "Q8_0")
        self.layers = []
        for i in range(self.L + self.n_mtp):
            p = f"blk.{i}."
            ly = {n: w(p + n + ".weight") for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm", "attn_q",
                                                     "attn_k", "attn_v", "attn_output")}
            if self.NE and i < self.L:
                for n in ("ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
                    ly[n] = w(p + n + ".weight")
            else:
                for n in ("ffn_gate", "ffn_up", "ffn_down"):
                    ly[n] = w(p + n + ".weight")
            self.layers.append(ly)
        if self.n_mtp:
            p = f"blk.{self.L}.nextn."
            self.eh = w(p + "eh_proj.weight")
            self.enorm, self.hnorm = w(p + "enorm.weight"), w(p + "hnorm.weight")
            hn = p + "shared_head_norm.weight"
            self.head_norm = w(hn) if hn in g.tinfo else self.out_norm
        self.theta_scale = np.float32(np.float32(self.base) ** np.float32(-2.0 / D))

    # ---- pieces
    def mm(self, W, x):
        return matmul(W, np.asarray(x, np.float64).reshape(-1, np.asarray(x).shape[-1]))

    def rope(self, x, pos):
        """NEOX rotation of pairs (i, i + 64), theta_i = pos * s^i by i successive fp32 multiplies"""
        th = np.empty(D // 2, np.float32)
        t = np.float32(pos)
        for i in range(D // 2):
            th[i] = t
            t = np.float32(t * self.theta_scale)
        c, s = _f32_map(_libm.cosf, th).astype(np.float64), _f32_map(_libm.sinf, th).astype(np.float64)
        a, b = np.asarray(x[..., :D // 2], np.float32), np.asarray(x[..., D // 2:], np.float32)
        c32, s32 = c.astype(np.float32), s.astype(np.float32)
        y0 = ((a * c32).astype(np.float32) - (b * s32).astype(np.float32)).astype(np.float32)
        y1 = ((a * s32).astype(np.float32) + (b * c32).astype(np.float32)).astype(np.float32)
        return np.concatenate([y0, y1], -1).astype(np.float64)

    def block(self, ly, x, kv, layer, seq, pos):
        """one layer over rows x [R][E] (in place semantics: returns the new x); every row's K / V written to
        kv[(seq, layer)][pos] before any row attends"""
        R, H, KVH, E = x.shape[0], self.H, self.KVH, self.E
        h = rmsnorm(x, ly["attn_norm"], self.eps)
        q = self.mm(ly["attn_q"], h).reshape(R, H, D)
        k = self.mm(ly["attn_k"], h).reshape(R, KVH, D)
        v = self.mm(ly["attn_v"], h).reshape(R, KVH, D)
        for r in range(R):
            q[r] = f32(self.rope(rmsnorm(q[r], ly["attn_q_norm"], self.eps), pos[r]))
            kr = f32(self.rope(rmsnorm(k[r], ly["attn_k_norm"], self.eps), pos[r]))
            cell = kv.setdefault((int(seq[r]), layer), {})
            cell[int(pos[r])] = (f16(kr), f16(v[r]))
        G = H // KVH
        ao = np.zeros((R, H, D))
        for r in range(R):
            cells = kv[(int(seq[r]), layer)]
            ks = np.stack([cells[c][0] if c in cells else np.zeros((KVH, D)) for c in range(pos[r] + 1)])
            vs = np.stack([cells[c][1] if c in cells else np.zeros((KVH, D)) for c in range(pos[r] + 1)])
            for hh in range(H):
                ao[r, hh] = attend(q[r, hh], ks[:, hh // G], vs[:, hh // G])
        x = f32(x + self.mm(ly["attn_output"], f32(ao.reshape(R, H * D))))
        h = rmsnorm(x, ly["ffn_norm"], self.eps)
        if "ffn_gate_inp" in ly:
            return f32(x + self.moe(ly, h))
        f = f32(silu(self.mm(ly["ffn_gate"], h)) * self.mm(ly["ffn_up"], h))
        return f32(x + self.mm(ly["ffn_down"], f))

    def moe(self, ly, h):
        """moe_ffn: the fp32 router, softmax, the NEU largest (ties to the lower id), renormalised weights, SwiGLU
        experts, their rows weighted and summed in slot order"""
        out = np.zeros_like(h)
        R = h.shape[0]
        # the router: fp32 dots in element order
        lg = np.zeros((R, self.NE), np.float32)
        h32, w32 = np.asarray(h, np.float32), np.asarray(ly["ffn_gate_inp"], np.float32)
        for i in range(self.E):
            lg = (lg + (h32[:, None, i] * w32[None, :, i]).astype(np.float32)).astype(np.float32)
        for r in range(R):
            e = expf((lg[r] - lg[r].max()).astype(np.float32))
            tot = np.float32(0)
            for v in e:
                tot = np.float32(tot + v)
            ids = sorted(range(self.NE), key=lambda x: (-e[x], x))[:self.NEU]
            w = [np.float32(e[x] / tot) for x in ids]
            sel = np.float32(0)
            for v in w:
                sel = np.float32(sel + v)
            sel = max(sel, np.float32(6.103515625e-5))
            acc = np.zeros(self.E, np.float32)
            for x, wx in zip(ids, w):
                g = self.mm(ly["ffn_gate_exps"][x], h[r:r + 1])
                u = self.mm(ly["ffn_up_exps"][x], h[r:r + 1])
                y = self.mm(ly["ffn_down_exps"][x], f32(silu(g) * u))
                acc = (acc + (np.float32(wx / sel) * y[0].astype(np.float32)).astype(np.float32)).astype(np.float32)
            out[r] = acc
        return out

    def step(self, kv, tok, seq, pos, out_rows):
        """or_qwen3_step's contract: (greedy tokens, logits of out_rows, every row after the final norm)"""
        x = f32(self.emb[tok])
        for i in range(self.L):
            x = self.block(self.layers[i], x, kv, i, seq, pos)
        hn = rmsnorm(x, self.out_norm, self.eps)
        lg = self.mm(self.head, hn[out_rows])
        return lg.argmax(-1), lg, hn

    def mtp_in(self, tok, hprev):
        cat = np.concatenate([rmsnorm(self.emb[tok], self.enorm, self.eps), rmsnorm(hprev, self.hnorm, self.eps)], -1)
        return self.mm(self.eh, cat)

    def mtp_fill(self, kv, tok, seq, pos, hprev):
        """the head's K / V cells of rows (tok at seq, pos) paired with hprev [R][E]"""
        ly = self.layers[self.L]
        x = self.mtp_in(tok, hprev)
        h = rmsnorm(x, ly["attn_norm"], self.eps)
        R = len(tok)
        k = self.mm(ly["attn_k"], h).reshape(R, self.KVH, D)
        v = self.mm(ly["attn_v"], h).reshape(R, self.KVH, D)
        for r in range(R):
            kr = f32(self.rope(rmsnorm(k[r], ly["attn_k_norm"], self.eps), pos[r]))
            kv.setdefault((int(seq[r]), self.L), {})[int(pos[r])] = (f16(kr), f16(v[r]))

    def mtp_guess(self, kv, seq, tok, pos, k, hprev):
        """k guesses: row j at pos + j takes tok (then guess j - 1) and hprev (then the head's own output state)"""
        out, lgs = [], []
        h = np.asarray(hprev, np.float64)[None]
        t = tok
        for j in range(k):
            x = self.mtp_in(np.array([t]), h)
            x = self.block(self.layers[self.L], x, kv, self.L, np.array([seq]), np.array([pos + j]))
            h = rmsnorm(x, self.head_norm, self.eps)
            lg = self.mm(self.head, h)[0]
            t = int(lg.argmax())
            out.append(t)
            lgs.append(lg)
        return np.array(out), np.array(lgs)
