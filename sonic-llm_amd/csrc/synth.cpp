// Synthetic random-init models as GGUF files: the Qwen3-architecture dense model of the configs (optionally with one
// multi-token-prediction "nextn" layer) and the Qwen3-MoE architecture, Q4_0 matrices quantized with ggml's reference
// quantizer (quantize_row_q4_0_ref), fp32 embedding and norms. Values come from a seeded splitmix64 stream per tensor
// row through Box-Muller, so a file is the same bytes for any thread count.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <thread>
#include <vector>

#include "../../include/sn_synth.h"
#include "gguf.h"

void sn_set_err(char* err, int err_len, const char* fmt, ...);

static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// n normal values (mean, std) from the stream seeded by (seed, tensor, row)
static void normals(uint64_t seed, uint64_t tensor, uint64_t row, float mean, float std, float* out, int64_t n) {
    uint64_t s = seed ^ (tensor * 0xD1B54A32D192ED03ull) ^ (row * 0x9E3779B97F4A7C15ull);
    splitmix64(&s);
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = ((splitmix64(&s) >> 11) + 1) * 0x1.0p-53;  // (0, 1]
        const double u2 = (splitmix64(&s) >> 11) * 0x1.0p-53;        // [0, 1)
        const double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
        out[i] = (float) (mean + std * r * cos(t));
        if (i + 1 < n) out[i + 1] = (float) (mean + std * r * sin(t));
    }
}

// ggml quantize_row_q4_0_ref: d = (the value of largest magnitude, first on ties) / -8, q = min(15, (int8)(x/d + 8.5))
void sn_quantize_row_q4_0(const float* x, uint8_t* y, int64_t k) {
    for (int64_t i = 0; i < k / 32; i++) {
        const float* xb = x + i * 32;
        uint8_t* yb = y + i * 18;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(xb[j])) {
                amax = fabsf(xb[j]);
                max = xb[j];
            }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        const _Float16 dh = (_Float16) d;
        memcpy(yb, &dh, 2);
        for (int j = 0; j < 16; ++j) {
            const int8_t a = (int8_t) (xb[j] * id + 8.5f), b = (int8_t) (xb[16 + j] * id + 8.5f);
            yb[2 + j] = (uint8_t) (std::min<int>(15, a) | (std::min<int>(15, b) << 4));
        }
    }
}

// ggml quantize_row_q8_0_ref: d = amax / 127 (stored fp16), id = 1/d (0 when d is 0), q = roundf(x * id)
void sn_quantize_row_q8_0(const float* x, uint8_t* y, int64_t k) {
    for (int64_t i = 0; i < k / 32; i++) {
        const float* xb = x + i * 32;
        uint8_t* yb = y + i * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = std::max(amax, fabsf(xb[j]));
        const float d = amax / 127.f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const _Float16 dh = (_Float16) d;
        memcpy(yb, &dh, 2);
        for (int j = 0; j < 32; ++j) yb[2 + j] = (uint8_t) (int8_t) (int) roundf(xb[j] * id);
    }
}

// A Q6_K row of seeded valid blocks (block_q6_K: ql[128], qh[64], int8 scales[16], fp16 d): q uniform in 0..63,
// scales uniform in -15..15, d = std / 165 (the values' std is then about `std`)
static void q6k_row(uint64_t seed, uint64_t tensor, uint64_t row, float std, uint8_t* dst, int64_t K) {
    uint64_t s = seed ^ (tensor * 0xD1B54A32D192ED03ull) ^ (row * 0x9E3779B97F4A7C15ull) ^ 0x6A09E667F3BCC909ull;
    splitmix64(&s);
    for (int64_t b = 0; b < K / 256; ++b) {
        uint8_t* blk = dst + b * 210;
        for (int i = 0; i < 192; i += 8) {  // ql and qh: every bit pattern is a valid quant
            const uint64_t v = splitmix64(&s);
            memcpy(blk + i, &v, 8);
        }
        for (int i = 0; i < 16; ++i) blk[192 + i] = (uint8_t) (int8_t) ((int) (splitmix64(&s) % 31) - 15);
        const _Float16 d = (_Float16) (std / 165.0f);
        memcpy(blk + 208, &d, 2);
    }
}

namespace {
struct Gen {
    std::string name;
    int type;
    std::vector<int64_t> ne;
    float mean, std;
};
}  // namespace

extern "C" int snx_write_model(const char* path, const snx_model_cfg* c, uint64_t seed, int nthreads, char* err,
                               int err_len) {
    const bool moe = c->n_expert > 0;
    const char* arch = moe ? "qwen3moe" : "qwen3";
    const int64_t E = c->n_embd, H = c->n_head, KVH = c->n_head_kv, D = c->head_dim, F = c->n_ff, V = c->n_vocab;
    if (E % 32 || (H * D) % 32 || F % 32 || (moe && c->n_ff_exp % 32)) {
        sn_set_err(err, err_len, "snx_write_model: dims must be multiples of 32");
        return -1;
    }
    GgufWriter w;
    const std::string a = arch;
    w.str("general.architecture", a);
    w.str("general.name", "sonic-mi355x synthetic random-init");
    w.u32(a + ".block_count", (uint32_t) (c->n_layer + (c->nextn ? 1 : 0)));
    w.u32(a + ".embedding_length", (uint32_t) E);
    w.u32(a + ".feed_forward_length", (uint32_t) F);
    w.u32(a + ".attention.head_count", (uint32_t) H);
    w.u32(a + ".attention.head_count_kv", (uint32_t) KVH);
    w.u32(a + ".attention.key_length", (uint32_t) D);
    w.u32(a + ".attention.value_length", (uint32_t) D);
    w.u32(a + ".context_length", 40960);
    w.f32(a + ".rope.freq_base", c->rope_base);
    w.f32(a + ".attention.layer_norm_rms_epsilon", c->eps);
    if (c->nextn) w.u32(a + ".nextn_predict_layers", 1);
    if (moe) {
        w.u32(a + ".expert_count", (uint32_t) c->n_expert);
        w.u32(a + ".expert_used_count", (uint32_t) c->n_expert_used);
        w.u32(a + ".expert_feed_forward_length", (uint32_t) c->n_ff_exp);
    }
    const int ET = c->embd_type;
    if ((ET != GGML_F32 && ET != GGML_Q4_0 && ET != GGML_Q8_0 && ET != GGML_Q6_K) || (ET == GGML_Q6_K && E % 256) ||
        (c->tied && ET == GGML_F32)) {
        sn_set_err(err, err_len, "snx_write_model: embd_type must be 0, 2, 8 or 14 (Q6_K: n_embd %% 256 == 0), and "
                                 "quantized when the head is tied");
        return -1;
    }
    if (c->wtype != 0 && c->wtype != GGML_Q4_0 && c->wtype != GGML_Q8_0) {
        sn_set_err(err, err_len, "snx_write_model: wtype must be 2 (Q4_0) or 8 (Q8_0)");
        return -1;
    }
    const int WQ = c->wtype == GGML_Q8_0 ? GGML_Q8_0 : GGML_Q4_0;  // the matrices' type
    const float ws = c->w_std, nstd = 0.1f;
    std::vector<Gen> g;
    g.push_back({"token_embd.weight", ET, {E, V}, 0.0f, c->emb_std});
    g.push_back({"output_norm.weight", GGML_F32, {E}, 1.0f, nstd});
    if (!c->tied) g.push_back({"output.weight", WQ, {E, V}, 0.0f, ws});
    const int nl = c->n_layer + (c->nextn ? 1 : 0);
    for (int i = 0; i < nl; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        g.push_back({p + "attn_norm.weight", GGML_F32, {E}, 1.0f, nstd});
        g.push_back({p + "attn_q.weight", WQ, {E, H * D}, 0.0f, ws});
        g.push_back({p + "attn_k.weight", WQ, {E, KVH * D}, 0.0f, ws});
        g.push_back({p + "attn_v.weight", WQ, {E, KVH * D}, 0.0f, ws});
        g.push_back({p + "attn_output.weight", WQ, {H * D, E}, 0.0f, ws});
        g.push_back({p + "attn_q_norm.weight", GGML_F32, {D}, 1.0f, nstd});
        g.push_back({p + "attn_k_norm.weight", GGML_F32, {D}, 1.0f, nstd});
        g.push_back({p + "ffn_norm.weight", GGML_F32, {E}, 1.0f, nstd});
        if (moe && i < c->n_layer) {
            const int64_t NE = c->n_expert, FE = c->n_ff_exp;
            g.push_back({p + "ffn_gate_inp.weight", GGML_F32, {E, NE}, 0.0f, 1.0f / sqrtf((float) E)});
            g.push_back({p + "ffn_gate_exps.weight", WQ, {E, FE, NE}, 0.0f, ws});
            g.push_back({p + "ffn_up_exps.weight", WQ, {E, FE, NE}, 0.0f, ws});
            g.push_back({p + "ffn_down_exps.weight", WQ, {FE, E, NE}, 0.0f, ws});
        } else {
            g.push_back({p + "ffn_gate.weight", WQ, {E, F}, 0.0f, ws});
            g.push_back({p + "ffn_up.weight", WQ, {E, F}, 0.0f, ws});
            g.push_back({p + "ffn_down.weight", WQ, {F, E}, 0.0f, ws});
        }
        if (c->nextn && i == c->n_layer) {
            g.push_back({p + "nextn.eh_proj.weight", WQ, {2 * E, E}, 0.0f, ws});
            g.push_back({p + "nextn.enorm.weight", GGML_F32, {E}, 1.0f, nstd});
            g.push_back({p + "nextn.hnorm.weight", GGML_F32, {E}, 1.0f, nstd});
            g.push_back({p + "nextn.shared_head_norm.weight", GGML_F32, {E}, 1.0f, nstd});
        }
    }
    for (const Gen& t : g) w.tensor(t.name, t.type, t.ne);

    FILE* f = fopen(path, "wb");
    if (!f) {
        sn_set_err(err, err_len, "snx_write_model: cannot create %s", path);
        return -1;
    }
    size_t start = 0;
    bool ok = w.begin(f, &start);
    const unsigned nt = nthreads > 0 ? (unsigned) nthreads : std::max(1u, std::thread::hardware_concurrency());
    std::vector<uint8_t> buf;
    for (size_t ti = 0; ti < g.size() && ok; ++ti) {
        const Gen& t = g[ti];
        const int64_t K = t.ne[0];
        int64_t rows = 1;
        for (size_t d = 1; d < t.ne.size(); ++d) rows *= t.ne[d];
        const size_t rb = ggml_row_bytes(t.type, K);
        // pad to the tensor's offset
        const size_t at = start + w.ts[ti].offset;
        const long cur = ftell(f);
        if ((size_t) cur < at) {
            std::vector<uint8_t> z(at - (size_t) cur, 0);
            ok = ok && fwrite(z.data(), 1, z.size(), f) == z.size();
        }
        const int64_t chunk = std::max<int64_t>(1, (int64_t) ((64u << 20) / rb));
        for (int64_t r0 = 0; r0 < rows && ok; r0 += chunk) {
            const int64_t nr = std::min(chunk, rows - r0);
            buf.resize((size_t) nr * rb);
            std::vector<std::thread> th;
            for (unsigned k = 0; k < nt; ++k)
                th.emplace_back([&, k]() {
                    std::vector<float> row((size_t) K + 1);
                    for (int64_t r = r0 + k; r < r0 + nr; r += nt) {
                        normals(seed, ti, (uint64_t) r, t.mean, t.std, row.data(), K);
                        uint8_t* dst = buf.data() + (size_t) (r - r0) * rb;
                        if (t.type == GGML_F32) memcpy(dst, row.data(), rb);
                        else if (t.type == GGML_Q6_K) q6k_row(seed, ti, (uint64_t) r, t.std, dst, K);
                        else if (t.type == GGML_Q8_0) sn_quantize_row_q8_0(row.data(), dst, K);
                        else sn_quantize_row_q4_0(row.data(), dst, K);
                    }
                });
            for (auto& x : th) x.join();
            ok = ok && fwrite(buf.data(), 1, buf.size(), f) == buf.size();
        }
    }
    ok = (fclose(f) == 0) && ok;
    if (!ok) {
        sn_set_err(err, err_len, "snx_write_model: write failed (%s)", path);
        return -1;
    }
    return 0;
}

extern "C" void snx_quantize_q4_0(const float* x, uint8_t* y, int64_t k) { sn_quantize_row_q4_0(x, y, k); }
extern "C" void snx_quantize_q8_0(const float* x, uint8_t* y, int64_t k) { sn_quantize_row_q8_0(x, y, k); }
