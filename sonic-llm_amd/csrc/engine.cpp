// The engine behind sn.h on one MI355X: model upload, the paged KV pool, and the batched decode/verify step.
//
// Replaces the reference's sllm-next library (engine/sllm-next/proto/sn.m and its *.inc.h parts): sn_open
// (sn_open.inc.h:390-412, dense_open sn_load.inc.h:341-359), sn_step (sn_step.inc.h:187-220, encode
// sn_encode.inc.h:321-349, the layer program sn_attn.inc.h:216-231, outputs sn_encode.inc.h:304-317), the page pool
// (sn_cache.inc.h:180-241) and the cache calls (sn_seq.inc.h). Every step is one stream of HIP kernels and one host
// round trip (the tokens back); the step's per-row data go to the GPU in one copy.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/sn.h"
#include "../../include/sn_ext.h"
#include "gguf.h"
#include "sn_kernels_internal.h"

void sn_set_err(char* err, int err_len, const char* fmt, ...) {
    if (!err || err_len <= 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t) err_len, fmt, ap);
    va_end(ap);
}

namespace {

struct DevLayer {
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    uint8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;
};

}  // namespace

struct sn_engine {
    GgufFile gg;
    std::string arch;
    int E = 0, L = 0, H = 0, KVH = 0, D = 128, F = 0, V = 0, QD = 0, KD = 0, NQKV = 0, n_ctx_train = 0;
    float eps = 1e-6f, rope_base = 1e6f, theta_scale = 1.0f;
    int slots = 0, ctx = 0, max_rows = 0, n_pages = 0, page_cells = 64, max_pages = 0, max_out = 0;
    bool has_nextn = false;

    hipStream_t st = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<void*> allocs;

    float *tok_embd = nullptr, *out_norm = nullptr;
    uint8_t* head = nullptr;
    std::vector<DevLayer> ly;
    uint16_t *kbase = nullptr, *vbase = nullptr;
    size_t layer_halves = 0;  // one layer's K (or V) pool, in fp16 values
    int32_t* d_pt = nullptr;

    float *x = nullptr, *qkv = nullptr, *ao = nullptr, *hb = nullptr, *logits = nullptr, *gemm_ws = nullptr;
    size_t gemm_ws_bytes = 0;
    uint8_t* xa = nullptr;
    float* apart = nullptr;
    int max_chunks = 0;
    uint8_t *d_stage = nullptr, *h_stage = nullptr;
    size_t stage_bytes = 0;
    int32_t *d_otok = nullptr, *h_otok = nullptr;
    float *d_rec = nullptr, *h_rec = nullptr;
    int32_t* d_ban = nullptr;

    std::vector<int32_t> pt;  // [slots][max_pages], -1: no page
    std::vector<int> ref;     // holders of each page
    std::vector<int> freel;   // free pages
    bool pt_dirty = true;
    std::vector<int32_t> eog;
    std::vector<uint8_t> no_end;
    bool want_probs = false;
    int last_n_out = 0, last_pn = 0;
    std::vector<float> last_probs;
    double last_ms = 0.0;
    int guess_on = 0;

    // per-kernel-class profiling (sn_ext.h): event pairs around each launch while on
    struct ProfRec {
        int kind, e0, e1;
        double bytes;
    };
    bool prof_on = false;
    std::vector<hipEvent_t> prof_ev;
    std::vector<ProfRec> prof_recs;
    double prof_ms[SNX_K_COUNT] = {0}, prof_bytes[SNX_K_COUNT] = {0};
    int prof_n[SNX_K_COUNT] = {0};

    // run a launch (or a few) of class `kind` moving `bytes` algorithmic bytes, bracketed by events when profiling
    template <class Fn>
    int launch(int kind, double bytes, Fn fn) {
        if (!prof_on || prof_recs.size() * 2 + 2 > prof_ev.size()) return fn();
        const int a = (int) prof_recs.size() * 2;
        hipEventRecord(prof_ev[a], st);
        const int rc = fn();
        hipEventRecord(prof_ev[a + 1], st);
        prof_recs.push_back({kind, a, a + 1, bytes});
        return rc;
    }

    template <class T>
    T* dalloc(size_t bytes, char* err, int err_len) {
        void* p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(bytes, 256)) != hipSuccess) {
            sn_set_err(err, err_len, "hipMalloc of %zu bytes failed", bytes);
            return nullptr;
        }
        allocs.push_back(p);
        return (T*) p;
    }
    int32_t* seq_pages(int s) { return pt.data() + (size_t) s * max_pages; }
};

// ---------------------------------------------------------------------------------------------------------------------
// open

namespace {

const GgufTensor* need(const GgufFile& g, const std::string& name, int type, std::string* why) {
    const GgufTensor* t = g.find(name);
    if (!t) *why = "missing tensor " + name;
    else if (t->type != type) {
        *why = "tensor " + name + " has an unsupported type (Q4_0 matrices and F32 norms / embedding are served)";
        t = nullptr;
    }
    return t;
}

// a GGUF Q4_0 matrix (ne = [K, N]) into stripes at dst (stripe stride / offset for interleaving)
bool upload_q4(sn_engine* e, const GgufTensor* t, uint8_t* tmp, uint8_t* dst, int sstride, int soff, char* err,
               int err_len) {
    SN_HIP_TRY(hipMemcpyAsync(tmp, t->data, t->nbytes, hipMemcpyHostToDevice, e->st), false);
    q4_repack(tmp, (int) t->ne[1], (int) t->ne[0], dst, sstride, soff, e->st);
    SN_HIP_TRY(hipStreamSynchronize(e->st), false);
    return true;
}

float* upload_f32(sn_engine* e, const GgufTensor* t, char* err, int err_len) {
    float* d = e->dalloc<float>(t->nbytes, err, err_len);
    if (!d) return nullptr;
    if (hipMemcpy(d, t->data, t->nbytes, hipMemcpyHostToDevice) != hipSuccess) {
        sn_set_err(err, err_len, "upload of %s failed", t->name.c_str());
        return nullptr;
    }
    return d;
}

bool model_check(const GgufFile& g, std::string* why) {
    const std::string a = g.str("general.architecture");
    if (a != "qwen3") {
        *why = "architecture '" + a + "': this engine serves qwen3 models";
        return false;
    }
    const int H = (int) g.num(a + ".attention.head_count", 0), KVH = (int) g.num(a + ".attention.head_count_kv", 0);
    const int E = (int) g.num(a + ".embedding_length", 0);
    const int D = (int) g.num(a + ".attention.key_length", E / std::max(H, 1));
    if (D != 128) {
        *why = "head_dim " + std::to_string(D) + ": the attention kernels take 128";
        return false;
    }
    if (H <= 0 || KVH <= 0 || H % KVH || 16 % (H / KVH)) {
        *why = "head counts: G = heads / kv heads must divide 16";
        return false;
    }
    if (E % 32) {
        *why = "embedding length must be a multiple of 32";
        return false;
    }
    if (!g.find("output.weight")) {
        *why = "an untied Q4_0 output.weight is required";
        return false;
    }
    return true;
}

}  // namespace

extern "C" sn_engine* sn_open(const char* path, const char* kernels, int slots, int ctx, int max_rows, int pages,
                              char* err, int err_len) {
    (void) kernels;
    if (slots <= 0 || ctx <= 0 || max_rows <= 0 || pages < 0) {
        sn_set_err(err, err_len, "sn_open: bad slots / ctx / max_rows / pages");
        return nullptr;
    }
    sn_engine* e = new sn_engine();
    std::string why;
    auto fail = [&](const std::string& w) -> sn_engine* {
        if (!w.empty()) sn_set_err(err, err_len, "%s", w.c_str());
        sn_close(e);
        return nullptr;
    };
    if (!e->gg.open(path, &why) || !model_check(e->gg, &why)) return fail(why);
    const GgufFile& g = e->gg;
    const std::string a = e->arch = g.str("general.architecture");
    const int nextn = (int) g.num(a + ".nextn_predict_layers", 0);
    e->has_nextn = nextn > 0;
    e->L = (int) g.num(a + ".block_count", 0) - nextn;
    e->E = (int) g.num(a + ".embedding_length", 0);
    e->H = (int) g.num(a + ".attention.head_count", 0);
    e->KVH = (int) g.num(a + ".attention.head_count_kv", 0);
    e->F = (int) g.num(a + ".feed_forward_length", 0);
    e->eps = (float) g.num(a + ".attention.layer_norm_rms_epsilon", 1e-6);
    e->rope_base = (float) g.num(a + ".rope.freq_base", 1e6);
    e->n_ctx_train = (int) g.num(a + ".context_length", 0);
    e->theta_scale = powf(e->rope_base, -2.0f / (float) e->D);
    e->QD = e->H * e->D;
    e->KD = e->KVH * e->D;
    e->NQKV = e->QD + 2 * e->KD;
    const GgufTensor* emb = need(g, "token_embd.weight", GGML_F32, &why);
    if (!emb) return fail(why);
    e->V = (int) emb->ne[1];
    const char* pe = getenv("SN_PAGE");
    e->page_cells = pe && atoi(pe) == 32 ? 32 : 64;
    e->slots = slots;
    e->ctx = (ctx + e->page_cells - 1) / e->page_cells * e->page_cells;
    e->max_pages = e->ctx / e->page_cells;
    e->n_pages = pages > 0 ? pages : slots * e->max_pages;
    e->max_rows = max_rows;
    e->max_out = slots + 4;
    e->max_chunks = (e->ctx + ATT_CHUNK - 1) / ATT_CHUNK;
    if (hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&e->ev0) != hipSuccess ||
        hipEventCreate(&e->ev1) != hipSuccess)
        return fail("HIP stream / event creation failed (no GPU?)");

    // ---- weights
    const int E = e->E, QD = e->QD, KD = e->KD, F = e->F;
    size_t max_t = 0;
    for (const GgufTensor& t : g.tensors) max_t = std::max(max_t, t.nbytes);
    uint8_t* tmp = nullptr;
    if (hipMalloc(&tmp, max_t) != hipSuccess) return fail("hipMalloc of the upload buffer failed");
    bool ok = true;
    auto q4 = [&](const std::string& n, int N, int K) -> const GgufTensor* {
        const GgufTensor* t = need(g, n, GGML_Q4_0, &why);
        if (t && (t->ne[0] != K || t->ne[1] != N)) {
            why = "tensor " + n + " has unexpected dimensions";
            t = nullptr;
        }
        ok = ok && t;
        return t;
    };
    auto f32 = [&](const std::string& n, int64_t ne0) -> float* {
        const GgufTensor* t = need(g, n, GGML_F32, &why);
        if (t && t->ne[0] != ne0) {
            why = "tensor " + n + " has unexpected dimensions";
            t = nullptr;
        }
        float* d = t ? upload_f32(e, t, err, err_len) : nullptr;
        ok = ok && d;
        return d;
    };
    e->tok_embd = upload_f32(e, emb, err, err_len);
    e->out_norm = f32("output_norm.weight", E);
    if (const GgufTensor* t = ok ? q4("output.weight", e->V, E) : nullptr) {
        e->head = e->dalloc<uint8_t>(q4t_bytes(e->V, E), err, err_len);
        ok = e->head && upload_q4(e, t, tmp, e->head, 1, 0, err, err_len);
    }
    e->ly.resize(e->L);
    for (int i = 0; i < e->L && ok; ++i) {
        DevLayer& l = e->ly[i];
        const std::string p = "blk." + std::to_string(i) + ".";
        l.attn_norm = f32(p + "attn_norm.weight", E);
        l.q_norm = f32(p + "attn_q_norm.weight", e->D);
        l.k_norm = f32(p + "attn_k_norm.weight", e->D);
        l.ffn_norm = f32(p + "ffn_norm.weight", E);
        const GgufTensor *tq = q4(p + "attn_q.weight", QD, E), *tk = q4(p + "attn_k.weight", KD, E),
                         *tv = q4(p + "attn_v.weight", KD, E), *to = q4(p + "attn_output.weight", E, QD),
                         *tg = q4(p + "ffn_gate.weight", F, E), *tu = q4(p + "ffn_up.weight", F, E),
                         *td = q4(p + "ffn_down.weight", E, F);
        if (!ok) break;
        l.wqkv = e->dalloc<uint8_t>(q4t_bytes(e->NQKV, E), err, err_len);
        l.wo = e->dalloc<uint8_t>(q4t_bytes(E, QD), err, err_len);
        l.wgu = e->dalloc<uint8_t>(q4t_bytes(2 * F, E), err, err_len);
        l.wd = e->dalloc<uint8_t>(q4t_bytes(E, F), err, err_len);
        ok = l.wqkv && l.wo && l.wgu && l.wd;
        // q, k, v stripes one after another (one matmul for all three); gate and up stripes interleaved in pairs
        ok = ok && upload_q4(e, tq, tmp, l.wqkv, 1, 0, err, err_len) &&
             upload_q4(e, tk, tmp, l.wqkv + q4t_bytes(QD, E), 1, 0, err, err_len) &&
             upload_q4(e, tv, tmp, l.wqkv + q4t_bytes(QD + KD, E), 1, 0, err, err_len) &&
             upload_q4(e, to, tmp, l.wo, 1, 0, err, err_len) && upload_q4(e, tg, tmp, l.wgu, 2, 0, err, err_len) &&
             upload_q4(e, tu, tmp, l.wgu, 2, 1, err, err_len) && upload_q4(e, td, tmp, l.wd, 1, 0, err, err_len);
    }
    hipFree(tmp);
    if (!ok) return fail(why.empty() ? std::string() : why);

    // ---- the KV pool: per layer, K then V, pages of [KVH][page_cells][128] fp16, zeroed
    e->layer_halves = (size_t) e->n_pages * e->KVH * e->page_cells * e->D;
    e->kbase = e->dalloc<uint16_t>(e->layer_halves * 2 * e->L * sizeof(uint16_t), err, err_len);
    if (!e->kbase) return fail("");
    e->vbase = e->kbase + e->layer_halves * e->L;
    if (hipMemset(e->kbase, 0, e->layer_halves * 2 * e->L * 2) != hipSuccess) return fail("KV pool clear failed");
    e->pt.assign((size_t) slots * e->max_pages, -1);
    e->ref.assign(e->n_pages, 0);
    for (int p = e->n_pages - 1; p >= 0; --p) e->freel.push_back(p);
    e->no_end.assign(slots, 0);

    // ---- step buffers
    const int R = max_rows, MO = e->max_out;
    const int KMAX = std::max(std::max(E, QD), F);
    e->d_pt = e->dalloc<int32_t>(e->pt.size() * 4, err, err_len);
    e->x = e->dalloc<float>((size_t) R * E * 4, err, err_len);
    e->qkv = e->dalloc<float>((size_t) R * e->NQKV * 4, err, err_len);
    e->ao = e->dalloc<float>((size_t) R * QD * 4, err, err_len);
    e->hb = e->dalloc<float>((size_t) R * F * 4, err, err_len);
    e->logits = e->dalloc<float>((size_t) MO * e->V * 4, err, err_len);
    e->xa = e->dalloc<uint8_t>(xa_bytes(R, KMAX), err, err_len);
    size_t ws = 0;
    ws = std::max(ws, q4_workspace_bytes(R, e->NQKV, E));
    ws = std::max(ws, q4_workspace_bytes(R, E, QD));
    ws = std::max(ws, q4_workspace_bytes(R, 2 * F, E));
    ws = std::max(ws, q4_workspace_bytes(R, E, F));
    ws = std::max(ws, q4_workspace_bytes(MO, e->V, E));
    e->gemm_ws_bytes = ws;
    e->gemm_ws = e->dalloc<float>(ws, err, err_len);
    e->apart = e->dalloc<float>((size_t) R * e->H * e->max_chunks * (e->D + 2) * 4, err, err_len);
    // staging: tok, seq, pos (R each), out_rows (MO), skip (MO bytes, padded), groups (R), items (R * max_chunks), pt
    e->stage_bytes = (size_t) 3 * R * 4 + (size_t) MO * 4 + ((MO + 15) / 16 * 16) + (size_t) R * sizeof(AttnGroup) +
                     (size_t) R * e->max_chunks * sizeof(AttnItem) + e->pt.size() * 4 + 256;
    e->d_stage = e->dalloc<uint8_t>(e->stage_bytes, err, err_len);
    e->d_otok = e->dalloc<int32_t>((size_t) MO * 4, err, err_len);
    e->d_rec = e->dalloc<float>((size_t) MO * 32, err, err_len);
    e->d_ban = e->dalloc<int32_t>(8 * 4, err, err_len);
    if (!e->d_pt || !e->x || !e->qkv || !e->ao || !e->hb || !e->logits || !e->xa || !e->gemm_ws || !e->apart ||
        !e->d_stage || !e->d_otok || !e->d_rec || !e->d_ban)
        return fail("");
    if (hipHostMalloc((void**) &e->h_stage, e->stage_bytes, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->h_otok, (size_t) MO * 4, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->h_rec, (size_t) MO * 32, 0) != hipSuccess)
        return fail("pinned host buffers failed");
    return e;
}

extern "C" void sn_close(sn_engine* e) {
    if (!e) return;
    if (e->st) hipStreamSynchronize(e->st);
    for (void* p : e->allocs) hipFree(p);
    if (e->h_stage) hipHostFree(e->h_stage);
    if (e->h_otok) hipHostFree(e->h_otok);
    if (e->h_rec) hipHostFree(e->h_rec);
    if (e->ev0) hipEventDestroy(e->ev0);
    if (e->ev1) hipEventDestroy(e->ev1);
    for (auto& ev : e->prof_ev) hipEventDestroy(ev);
    if (e->st) hipStreamDestroy(e->st);
    delete e;
}

extern "C" int sn_check(const char* path, int* rows, char* err, int err_len) {
    GgufFile g;
    std::string why;
    if (!g.open(path, &why) || !model_check(g, &why)) {
        sn_set_err(err, err_len, "%s", why.c_str());
        return -1;
    }
    if (rows) *rows = 512;
    return 0;
}
extern "C" int sn_quiet_rows(const char* path) {
    (void) path;
    return 0;
}

// ---------------------------------------------------------------------------------------------------------------------
// the page pool (page_new / pages_drop / rows_pages, sn_cache.inc.h:180-241)

namespace {

int page_new(sn_engine* e) {
    if (e->freel.empty()) return -1;
    // the lowest free page
    auto it = std::min_element(e->freel.begin(), e->freel.end());
    const int p = *it;
    *it = e->freel.back();
    e->freel.pop_back();
    e->ref[p] = 1;
    return p;
}

// one holder less for page p; a page nobody holds is zeroed (every layer) and free again
void page_drop(sn_engine* e, int p) {
    if (p < 0) return;
    if (--e->ref[p] == 0) {
        kv_page_op(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, e->page_cells, -1, p, 0, e->page_cells, e->st);
        e->freel.push_back(p);
    }
}

bool slot_ok(const sn_engine* e, int slot, int a, int b) {
    return slot >= 0 && slot < e->slots && a >= 0 && a <= b && b <= e->ctx;
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------------
// the step

namespace {

bool step_shape_bad(const sn_engine* e, int R, int n_write, int n_fast, int n_out) {
    return R <= 0 || R > e->max_rows || n_write < 0 || n_write > R || n_write > e->slots + 4 || n_fast > 4 ||
           -n_fast > 8 || abs(n_fast) > n_write || n_out < 0 || n_out > e->max_out;
}

}  // namespace

extern "C" int sn_step(sn_engine* e, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos, int n_write,
                       int n_fast, int n_out, const int32_t* out_rows, int32_t* out_tok, int chain, char* err,
                       int err_len) {
    (void) chain;  // a chained step is run as an ordinary step: the same tokens (sn.h:36-38)
    if (step_shape_bad(e, R, n_write, n_fast, n_out)) {
        sn_set_err(err, err_len, "bad step shape");
        return -1;
    }
    for (int r = 0; r < R; ++r)
        if (seq[r] < 0 || seq[r] >= e->slots || pos[r] < 0 || pos[r] >= e->ctx || tok[r] < 0 || tok[r] >= e->V) {
            sn_set_err(err, err_len, "a row is out of range (slot, position or token)");
            return -1;
        }
    for (int j = 0; j < n_out; ++j)
        if (out_rows[j] < 0 || out_rows[j] >= R) {
            sn_set_err(err, err_len, "an output row is outside the step");
            return -1;
        }
    // a page for every cell a row reads or writes (pages_for gives the row's own chunk; here also any earlier chunk a
    // sequence never wrote, as a zero page: the attention reads cells 0 .. pos of every row, and unwritten cells are
    // zero). Out of pages: -2 with nothing run.
    std::vector<std::pair<int, int>> fresh;
    for (int r = 0; r < R; ++r)
        for (int c = 0; c <= pos[r] / e->page_cells; ++c) {
        int32_t* t = e->seq_pages(seq[r]) + c;
        if (*t < 0) {
            const int p = page_new(e);
            if (p < 0) {
                for (auto& f : fresh) {  // give back what this step took (never written, so still zero)
                    int32_t* tp = e->seq_pages(f.first) + f.second;
                    e->ref[*tp] = 0;
                    e->freel.push_back(*tp);
                    *tp = -1;
                }
                sn_set_err(err, err_len, "out of cache pages");
                return -2;
            }
            *t = p;
            fresh.push_back({seq[r], c});
            e->pt_dirty = true;
        }
        }

    // ---- the step's rows, attention work list and page table into one staging copy
    const int G = e->H / e->KVH, gmax = 16 / G;
    uint8_t* hs = e->h_stage;
    size_t off = 0;
    auto put = [&](const void* src, size_t n) {
        const size_t at = off;
        memcpy(hs + at, src, n);
        off = (off + n + 15) / 16 * 16;
        return at;
    };
    const size_t o_tok = put(tok, (size_t) R * 4), o_seq = put(seq, (size_t) R * 4), o_pos = put(pos, (size_t) R * 4);
    const size_t o_out = put(out_rows, (size_t) n_out * 4);
    std::vector<uint8_t> skip(n_out + 1, 0);
    for (int j = 0; j < n_out; ++j) skip[j] = e->no_end[seq[out_rows[j]]];
    const size_t o_skip = put(skip.data(), (size_t) n_out + 1);
    std::vector<AttnGroup> groups;
    std::vector<AttnItem> items;
    for (int r = 0; r < R;) {
        int n = 1;
        while (r + n < R && n < gmax && seq[r + n] == seq[r] && pos[r + n] == pos[r] + n) ++n;
        const int gi = (int) groups.size();
        groups.push_back({r, n, seq[r], pos[r]});
        const int last = pos[r] + n - 1;
        for (int c = 0; c <= last / ATT_CHUNK; ++c) items.push_back({gi, c});
        r += n;
    }
    const size_t o_grp = put(groups.data(), groups.size() * sizeof(AttnGroup));
    const size_t o_itm = put(items.data(), items.size() * sizeof(AttnItem));
    const bool send_pt = e->pt_dirty;
    const size_t o_pt = send_pt ? put(e->pt.data(), e->pt.size() * 4) : 0;
    const size_t copy_bytes = off;
    hipStream_t st = e->st;
    SN_HIP_TRY(hipEventRecord(e->ev0, st), -1);
    SN_HIP_TRY(hipMemcpyAsync(e->d_stage, hs, copy_bytes, hipMemcpyHostToDevice, st), -1);
    if (send_pt) {
        SN_HIP_TRY(hipMemcpyAsync(e->d_pt, e->d_stage + o_pt, e->pt.size() * 4, hipMemcpyDeviceToDevice, st), -1);
        e->pt_dirty = false;
    }
    const int32_t* d_tok = (const int32_t*) (e->d_stage + o_tok);
    const int32_t* d_seq = (const int32_t*) (e->d_stage + o_seq);
    const int32_t* d_pos = (const int32_t*) (e->d_stage + o_pos);
    const int32_t* d_out = (const int32_t*) (e->d_stage + o_out);
    const uint8_t* d_skip = e->d_stage + o_skip;

    // ---- the layers (qwen_layers, sn_attn.inc.h:216-231)
    const int E = e->E, QD = e->QD, KD = e->KD, F = e->F;
    e->prof_recs.clear();
    auto gemm_bytes = [](int M, int N, int K) { return (double) N * (K / 32) * 18 + (double) M * K * 4 + (double) M * N * 4; };
    // attention: each (sequence, KV head) reads its cells once; q in, output out, page-table entries
    double attn_bytes = (double) R * QD * 8;
    {
        std::vector<int> seen;
        for (const AttnGroup& g : groups) {
            int last = g.pos0 + g.nrows - 1;
            for (const AttnGroup& h : groups)
                if (h.seq == g.seq) last = std::max(last, h.pos0 + h.nrows - 1);
            if (std::find(seen.begin(), seen.end(), g.seq) != seen.end()) continue;
            seen.push_back(g.seq);
            attn_bytes += (double) (last + 1) * KD * 2 * 2 + 4.0 * (last / e->page_cells + 1);
        }
    }
    int rc = 0;
    rc |= e->launch(SNX_K_OTHER, (double) R * E * 8, [&] { embed_rows(e->tok_embd, E, d_tok, R, e->x, st); return 0; });
    AttnArgs aa{};
    aa.q = e->qkv;
    aa.ldq = e->NQKV;
    aa.pt = e->d_pt;
    aa.max_pages = e->max_pages;
    aa.page_cells = e->page_cells;
    aa.groups = (const AttnGroup*) (e->d_stage + o_grp);
    aa.items = (const AttnItem*) (e->d_stage + o_itm);
    aa.n_items = (int) items.size();
    aa.part = e->apart;
    aa.max_chunks = e->max_chunks;
    aa.out = e->ao;
    aa.ldo = QD;
    aa.H = e->H;
    aa.KVH = e->KVH;
    aa.scale = 1.0f / sqrtf((float) e->D);
    aa.n_rows = R;
    aa.row_pos = d_pos;
    auto quant = [&](const float* x, const int32_t* rows, int M, int K, const float* nw) {
        return e->launch(SNX_K_QUANT, (double) M * K * 8, [&] {
            quant_act(x, rows, M, K, K, nw, e->eps, e->xa, nullptr, 0, st);
            return 0;
        });
    };
    // Matmuls leave their k-slice sums in the workspace; the next row kernel adds them in slice order and applies the
    // epilogue (RoPE for q|k|v, residual add + RMSNorm + Q8_0 for o and down, SwiGLU + Q8_0 for gate/up).
    float* part = e->gemm_ws;
    int ks = 0;  // k-slices of the last matmul
    auto gemm = [&](const uint8_t* w, int M, int N, int K) {
        return e->launch(SNX_K_GEMM, gemm_bytes(M, N, K), [&] {
            ks = q4_gemm_raw(w, e->xa, M, N, K, part, e->gemm_ws_bytes, st);
            return ks < 0 ? -1 : 0;
        });
    };
    auto resid = [&](const float* nw, bool quantize) {
        return e->launch(SNX_K_QUANT, (double) R * E * (8 + 4 * ks) + (quantize ? (double) R * E * 2 : 0.0), [&] {
            return resid_quant(e->x, part, ks, R, E, nw, e->eps, quantize ? e->xa : nullptr, st);
        });
    };
    rc |= quant(e->x, nullptr, R, E, e->ly[0].attn_norm);  // layer 0: x is the embedding
    for (int i = 0; i < e->L && rc == 0; ++i) {
        const DevLayer& l = e->ly[i];
        uint16_t* kp = e->kbase + (size_t) i * e->layer_halves;
        uint16_t* vp = e->vbase + (size_t) i * e->layer_halves;
        if (i > 0) rc |= resid(l.attn_norm, true);  // x += the previous layer's down projection
        rc |= gemm(l.wqkv, R, e->NQKV, E);
        rc |= e->launch(SNX_K_ROPE, (double) R * (e->NQKV * 4.0 * (ks + 1) + QD * 4 + 2 * KD * 2), [&] {
            qk_norm_rope_kv(e->qkv, e->NQKV, part, ks, R, e->H, e->KVH, l.q_norm, l.k_norm, e->eps, e->theta_scale,
                            d_seq, d_pos, e->d_pt, e->max_pages, e->page_cells, kp, vp, st);
            return 0;
        });
        aa.kpool = kp;
        aa.vpool = vp;
        aa.xa = e->xa;  // the merge writes the o-projection's Q8_0 operand itself
        rc |= e->launch(SNX_K_ATTN, attn_bytes, [&] { return paged_attention(aa, st); });
        rc |= gemm(l.wo, R, E, QD);
        rc |= resid(l.ffn_norm, true);
        rc |= gemm(l.wgu, R, 2 * F, E);
        rc |= e->launch(SNX_K_QUANT, (double) R * 2 * F * 4 * ks + (double) R * F * 6, [&] {
            swiglu_quant(part, ks, R, F, e->hb, e->xa, st);
            return 0;
        });
        rc |= gemm(l.wd, R, E, F);
    }
    if (rc == 0) rc |= resid(nullptr, false);  // x += the last layer's down projection
    // ---- outputs (sn_encode.inc.h:304-317): final norm of the output rows, LM head, argmax
    if (n_out > 0 && rc == 0) {
        rc |= quant(e->x, d_out, n_out, E, e->out_norm);
        rc |= e->launch(SNX_K_GEMM, gemm_bytes(n_out, e->V, E), [&] {
            if (q4_plan(e->V, E).ks == 1)  // one slice: the sums are the logits
                return q4_gemm_raw(e->head, e->xa, n_out, e->V, E, e->logits, (size_t) n_out * e->V * 4, st) < 0 ? -1 : 0;
            return q4_gemm(e->head, e->xa, n_out, e->V, E, e->logits, e->V, EPI_STORE, e->gemm_ws, e->gemm_ws_bytes, st);
        });
        const int nban = (int) e->eog.size();
        rc |= e->launch(SNX_K_OTHER, (double) n_out * e->V * 4, [&] {
            argmax_rows(e->logits, e->V, n_out, e->d_ban, nban, d_skip, e->d_otok, e->want_probs ? e->d_rec : nullptr,
                        st);
            return 0;
        });
        SN_HIP_TRY(hipMemcpyAsync(e->h_otok, e->d_otok, (size_t) n_out * 4, hipMemcpyDeviceToHost, st), -1);
        if (e->want_probs)
            SN_HIP_TRY(hipMemcpyAsync(e->h_rec, e->d_rec, (size_t) n_out * 32, hipMemcpyDeviceToHost, st), -1);
    }
    SN_HIP_TRY(hipEventRecord(e->ev1, st), -1);
    SN_HIP_TRY(hipStreamSynchronize(st), -1);
    if (rc != 0) {
        sn_set_err(err, err_len, "a kernel launch was refused (workspace or shape)");
        return -1;
    }
    const hipError_t ke = hipGetLastError();
    if (ke != hipSuccess) {
        sn_set_err(err, err_len, "step failed on the GPU: %s", hipGetErrorString(ke));
        return -1;
    }
    float ms = 0.0f;
    hipEventElapsedTime(&ms, e->ev0, e->ev1);
    e->last_ms = ms;
    for (const auto& pr : e->prof_recs) {
        float t = 0.0f;
        hipEventElapsedTime(&t, e->prof_ev[pr.e0], e->prof_ev[pr.e1]);
        e->prof_ms[pr.kind] += t;
        e->prof_bytes[pr.kind] += pr.bytes;
        e->prof_n[pr.kind] += 1;
    }
    if (n_out > 0) memcpy(out_tok, e->h_otok, (size_t) n_out * 4);
    e->last_n_out = n_out;
    e->last_pn = e->want_probs ? n_out : 0;
    if (e->want_probs) e->last_probs.assign(e->h_rec, e->h_rec + (size_t) n_out * 8);
    return 0;
}

extern "C" double sn_last_gpu_ms(const sn_engine* e) { return e->last_ms; }

extern "C" void snx_prof(sn_engine* e, int on) {
    e->prof_on = on != 0;
    for (int k = 0; k < SNX_K_COUNT; ++k) {
        e->prof_ms[k] = e->prof_bytes[k] = 0.0;
        e->prof_n[k] = 0;
    }
    if (e->prof_on && e->prof_ev.empty()) {
        e->prof_ev.resize(4096);
        for (auto& ev : e->prof_ev) hipEventCreate(&ev);
    }
}

extern "C" int snx_prof_read(const sn_engine* e, int kind, double* ms, int* launches, double* bytes) {
    if (kind < 0 || kind >= SNX_K_COUNT) return -1;
    if (ms) *ms = e->prof_ms[kind];
    if (launches) *launches = e->prof_n[kind];
    if (bytes) *bytes = e->prof_bytes[kind];
    return 0;
}

extern "C" int snx_debug_read(sn_engine* e, int which, float* dst, size_t n) {
    const float* src = which == 0 ? e->x : which == 1 ? e->qkv : which == 2 ? e->ao : which == 3 ? e->hb : nullptr;
    const size_t cap = (size_t) e->max_rows * (which == 0 ? e->E : which == 1 ? e->NQKV : which == 2 ? e->QD : e->F);
    if (!src || n > cap) return -1;
    return hipMemcpy(dst, src, n * 4, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}

extern "C" int sn_logits_rows(sn_engine* e, int n, const int* ks, float* dst, char* err, int err_len) {
    for (int i = 0; i < n; ++i)
        if (ks[i] < 0 || ks[i] >= e->last_n_out) {
            sn_set_err(err, err_len, "output row out of range");
            return -1;
        }
    for (int i = 0; i < n; ++i)
        SN_HIP_TRY(hipMemcpy(dst + (size_t) i * e->V, e->logits + (size_t) ks[i] * e->V, (size_t) e->V * 4,
                             hipMemcpyDeviceToHost),
                   -1);
    return 0;
}
extern "C" int sn_logits(sn_engine* e, int k, float* dst, char* err, int err_len) {
    return sn_logits_rows(e, 1, &k, dst, err, err_len);
}

extern "C" void sn_want_probs(sn_engine* e, int on) { e->want_probs = on != 0; }
extern "C" int sn_probs(sn_engine* e, int n_out, float* dst, char* err, int err_len) {
    if (n_out < 0 || n_out > e->last_pn) {
        sn_set_err(err, err_len, "the last step has no token probabilities for these rows");
        return -1;
    }
    memcpy(dst, e->last_probs.data(), (size_t) n_out * 32);
    return 0;
}

extern "C" int sn_set_eog(sn_engine* e, const int32_t* ids, int n) {
    if (n < 0 || n > 8) return -1;
    e->eog.assign(ids, ids + n);
    if (n > 0 && hipMemcpy(e->d_ban, ids, (size_t) n * 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
    return 0;
}
extern "C" void sn_no_end(sn_engine* e, int slot, int on) {
    if (slot >= 0 && slot < e->slots) e->no_end[slot] = on != 0;
}

// ---------------------------------------------------------------------------------------------------------------------
// cache calls (sn_seq.inc.h)

extern "C" int sn_copy(sn_engine* e, int from, int to, int n, char* err, int err_len) {
    if (!slot_ok(e, from, 0, n) || !slot_ok(e, to, 0, n) || from == to) {
        sn_set_err(err, err_len, "sn_copy: bad slots or cells");
        return -1;
    }
    int32_t *tf = e->seq_pages(from), *tt = e->seq_pages(to);
    for (int c = 0; c < e->max_pages; ++c) {  // what `to` held goes
        page_drop(e, tt[c]);
        tt[c] = -1;
    }
    const int pc = e->page_cells;
    for (int c = 0; c < n / pc; ++c) {
        if (tf[c] < 0) {
            sn_set_err(err, err_len, "sn_copy: the source has no cells there");
            return -1;
        }
        tt[c] = tf[c];
        ++e->ref[tf[c]];
    }
    if (n % pc) {
        const int c = n / pc, np = page_new(e);
        if (np < 0) {
            sn_set_err(err, err_len, "out of cache pages");
            e->pt_dirty = true;
            return -2;
        }
        tt[c] = np;
        if (tf[c] >= 0) kv_page_op(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, pc, tf[c], np, 0, n % pc, e->st);
    }
    e->pt_dirty = true;
    SN_HIP_TRY(hipStreamSynchronize(e->st), -1);
    return 0;
}

extern "C" int sn_clear(sn_engine* e, int slot, int from, int to, char* err, int err_len) {
    if (!slot_ok(e, slot, from, to)) {
        sn_set_err(err, err_len, "sn_clear: bad slot or cells");
        return -1;
    }
    const int pc = e->page_cells;
    int32_t* t = e->seq_pages(slot);
    const int c1 = (from + pc - 1) / pc;  // every chunk from the first wholly at or past `from` goes
    for (int c = c1; c < e->max_pages; ++c) {
        page_drop(e, t[c]);
        t[c] = -1;
    }
    e->pt_dirty = true;
    const int c = from / pc, p = from % pc ? t[c] : -1;
    if (p >= 0 && from != to) {
        if (e->ref[p] > 1) {  // shared: a private copy of the cells kept
            const int np = page_new(e);
            if (np < 0) {
                sn_set_err(err, err_len, "out of cache pages");
                return -2;
            }
            --e->ref[p];
            t[c] = np;
            kv_page_op(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, pc, p, np, 0, from % pc, e->st);
        } else {
            kv_page_op(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, pc, -1, p, from % pc,
                       std::min(pc, to - c * pc), e->st);
        }
    }
    SN_HIP_TRY(hipStreamSynchronize(e->st), -1);
    return 0;
}

extern "C" size_t sn_kv_bytes(const sn_engine* e, int n) { return (size_t) e->L * 2 * n * e->KD * 2; }

static int kv_xfer(sn_engine* e, int slot, int n, void* host, int save, char* err, int err_len) {
    if (!slot_ok(e, slot, 0, n)) {
        sn_set_err(err, err_len, "sn_kv_save / sn_kv_load: bad slot or cells");
        return -1;
    }
    if (n == 0) return 0;
    int32_t* t = e->seq_pages(slot);
    const int np = (n + e->page_cells - 1) / e->page_cells;
    for (int c = 0; c < np; ++c)
        if (t[c] < 0) {
            if (save) {
                sn_set_err(err, err_len, "sn_kv_save: the slot has no cells there");
                return -1;
            }
            if ((t[c] = page_new(e)) < 0) {
                sn_set_err(err, err_len, "out of cache pages");
                return -2;
            }
            e->pt_dirty = true;
        }
    const size_t bytes = sn_kv_bytes(e, n);
    uint16_t* stg = nullptr;
    int32_t* dp = nullptr;
    SN_HIP_TRY(hipMalloc(&stg, bytes), -1);
    if (hipMalloc(&dp, (size_t) np * 4) != hipSuccess) {
        hipFree(stg);
        sn_set_err(err, err_len, "hipMalloc failed");
        return -1;
    }
    hipMemcpy(dp, t, (size_t) np * 4, hipMemcpyHostToDevice);
    if (!save) hipMemcpy(stg, host, bytes, hipMemcpyHostToDevice);
    kv_stage(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, e->page_cells, dp, n, stg, save, e->st);
    hipStreamSynchronize(e->st);
    if (save) hipMemcpy(host, stg, bytes, hipMemcpyDeviceToHost);
    const hipError_t ke = hipGetLastError();
    hipFree(stg);
    hipFree(dp);
    if (ke != hipSuccess) {
        sn_set_err(err, err_len, "KV transfer failed: %s", hipGetErrorString(ke));
        return -1;
    }
    return 0;
}
extern "C" int snx_fill_kv(sn_engine* e, int slot, int n, uint64_t seed, char* err, int err_len) {
    if (!slot_ok(e, slot, 0, n)) {
        sn_set_err(err, err_len, "snx_fill_kv: bad slot or cells");
        return -1;
    }
    if (n == 0) return 0;
    int32_t* t = e->seq_pages(slot);
    const int np = (n + e->page_cells - 1) / e->page_cells;
    for (int c = 0; c < np; ++c)
        if (t[c] < 0) {
            if ((t[c] = page_new(e)) < 0) {
                sn_set_err(err, err_len, "out of cache pages");
                return -2;
            }
            e->pt_dirty = true;
        }
    int32_t* dp = nullptr;
    SN_HIP_TRY(hipMalloc(&dp, (size_t) np * 4), -1);
    hipMemcpy(dp, t, (size_t) np * 4, hipMemcpyHostToDevice);
    kv_fill_normal(e->kbase, e->vbase, e->layer_halves, e->L, e->KVH, e->page_cells, dp, n,
                   seed ^ (0x9E3779B97F4A7C15ull * (uint64_t) (slot + 1)), e->st);
    hipStreamSynchronize(e->st);
    const hipError_t ke = hipGetLastError();
    hipFree(dp);
    if (ke != hipSuccess) {
        sn_set_err(err, err_len, "snx_fill_kv failed: %s", hipGetErrorString(ke));
        return -1;
    }
    return 0;
}

extern "C" int sn_kv_save(sn_engine* e, int slot, int n, void* dst, char* err, int err_len) {
    return kv_xfer(e, slot, n, dst, 1, err, err_len);
}
extern "C" int sn_kv_load(sn_engine* e, int slot, int n, const void* src, char* err, int err_len) {
    return kv_xfer(e, slot, n, (void*) src, 0, err, err_len);
}

// ---------------------------------------------------------------------------------------------------------------------
// queries and the calls this engine answers trivially

extern "C" int sn_n_vocab(const sn_engine* e) { return e->V; }
extern "C" int sn_n_ctx_train(const sn_engine* e) { return e->n_ctx_train; }
extern "C" const char* sn_arch(const sn_engine* e) { return e->arch.c_str(); }
extern "C" int sn_n_embd(const sn_engine* e) { return e->E; }
extern "C" int sn_pages_total(const sn_engine* e) { return e->n_pages; }
extern "C" int sn_pages_free(const sn_engine* e) { return (int) e->freel.size(); }
extern "C" size_t sn_page_bytes(const sn_engine* e) { return (size_t) e->page_cells * e->KD * 2 * 2 * e->L; }
extern "C" int sn_seq_pages(const sn_engine* e, int seq, int* own) {
    if (seq < 0 || seq >= e->slots) return 0;
    int n = 0, o = 0;
    const int32_t* t = e->pt.data() + (size_t) seq * e->max_pages;
    for (int c = 0; c < e->max_pages; ++c)
        if (t[c] >= 0) {
            ++n;
            o += e->ref[t[c]] == 1;
        }
    if (own) *own = o;
    return n;
}
extern "C" size_t sn_mem_used(const sn_engine* e) {
    return (size_t) (e->n_pages - (int) e->freel.size()) * sn_page_bytes(e);
}
extern "C" int sn_cut_ok(const sn_engine* e, int slot, int n) { return slot_ok(e, slot, 0, n) ? 1 : 0; }
extern "C" int sn_cut_best(const sn_engine* e, int slot, int n) {
    (void) e;
    (void) slot;
    return n;
}
extern "C" int sn_recurrent(const sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" int sn_draft_rows(sn_engine* e, int seq, int want) {
    (void) e;
    (void) seq;
    return want;
}
extern "C" int sn_small_rows(const sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" int sn_chat_exact(const sn_engine* e) {
    (void) e;
    return 1;
}
extern "C" int sn_mark(sn_engine* e, int slot) {
    (void) e;
    (void) slot;
    return 0;
}
extern "C" int sn_state_take(sn_engine* e, int seq) {
    (void) e;
    (void) seq;
    return -1;
}
extern "C" int sn_win_need(const sn_engine* e, int n) {
    (void) e;
    (void) n;
    return 0;
}
extern "C" int sn_win_room(const sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" int sn_win_pages(const sn_engine* e, int seq) {
    (void) e;
    (void) seq;
    return 0;
}
extern "C" size_t sn_trim(sn_engine* e, int spare) {
    (void) e;
    (void) spare;
    return 0;
}
extern "C" int sn_trim_pending(sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" size_t sn_state_bytes(const sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" int sn_state_entries(const sn_engine* e, int seq) {
    (void) e;
    (void) seq;
    return 0;
}
extern "C" int sn_latent(sn_engine* e, int n, const int32_t* rows, const float* vec, float* hid, char* err,
                         int err_len) {
    (void) e; (void) n; (void) rows; (void) vec; (void) hid;
    sn_set_err(err, err_len, "sn_latent: latent rows are not served by this engine");
    return -1;
}
extern "C" int sn_soft_config(sn_engine* e, float temp, int k, const int32_t* eog, int n_eog, char* err, int err_len) {
    (void) e; (void) temp; (void) k; (void) eog; (void) n_eog;
    sn_set_err(err, err_len, "soft words on the GPU: not served by this engine");
    return -1;
}
extern "C" int sn_soft_rows(sn_engine* e, int n_in, const int32_t* in_rows, int n_out, const int32_t* out_ks,
                            char* err, int err_len) {
    (void) e; (void) n_in; (void) in_rows; (void) n_out; (void) out_ks;
    sn_set_err(err, err_len, "soft words on the GPU: not served by this engine");
    return -1;
}
extern "C" int sn_embed_rows(sn_engine* e, int n, const int32_t* ids, float* dst, char* err, int err_len) {
    if (n < 0 || n > 1024) {
        sn_set_err(err, err_len, "sn_embed_rows: 0 .. 1024 ids");
        return -1;
    }
    for (int i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= e->V) {
            sn_set_err(err, err_len, "sn_embed_rows: id out of range");
            return -1;
        }
        SN_HIP_TRY(hipMemcpy(dst + (size_t) i * e->E, e->tok_embd + (size_t) ids[i] * e->E, (size_t) e->E * 4,
                             hipMemcpyDeviceToHost),
                   -1);
    }
    return 0;
}
extern "C" float sn_embd_norm(sn_engine* e) {
    (void) e;
    return 0.0f;
}

// guess head: declared here, served once the nextn layer is loaded (see sn_guess_head)
extern "C" int sn_guess_head(const sn_engine* e) {
    (void) e;
    return 0;
}
extern "C" int sn_guess_on(sn_engine* e, int on) {
    (void) on;
    e->guess_on = 0;
    return 0;
}
extern "C" int sn_guess(sn_engine* e, int seq, int32_t tok, int pos, int k, int32_t* out_tok, char* err, int err_len) {
    (void) e; (void) seq; (void) tok; (void) pos; (void) k; (void) out_tok;
    sn_set_err(err, err_len, "sn_guess: no guess head, or guessing is off (sn_guess_on)");
    return -1;
}
