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
#include <thread>
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
    // a MoE layer: fp32 router [NE][E]; per expert, gate/up stripes interleaved in pairs [2 FE][E] and down [E][FE]
    float* router = nullptr;
    uint8_t *egu = nullptr, *ed = nullptr;
};

}  // namespace

// The buffers a step in flight owns: its staging copy, output tokens, probability records, logits and its start / end
// events. Two sets alternate when a step is queued behind another (sn_step's chain); the engine's fields are the set
// of the step the caller last received, `alt` the other one.
#define GRAPH_CACHE 6  // step shapes whose graphs are kept
struct StepSet {
    uint8_t *d_stage = nullptr, *h_stage = nullptr;
    int32_t *d_otok = nullptr, *h_otok = nullptr;
    float *d_rec = nullptr, *h_rec = nullptr, *logits = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
};

struct sn_engine {
    GgufFile gg;
    std::string arch;
    int E = 0, L = 0, CL = 0, H = 0, KVH = 0, D = 128, F = 0, V = 0, QD = 0, KD = 0, NQKV = 0, n_ctx_train = 0;
    float eps = 1e-6f, rope_base = 1e6f, theta_scale = 1.0f;
    int slots = 0, ctx = 0, max_rows = 0, n_pages = 0, page_cells = 64, max_pages = 0, max_out = 0;
    bool has_nextn = false;
    // qwen3moe: experts, experts a token uses, an expert's FFN width; the tile bound of a step's expert rows
    int NE = 0, NEU = 0, FE = 0, moe_tiles = 0;
    int wt = WT_Q4_0;  // the block type of every layer matrix: WT_Q4_0 or WT_Q8_0 (GGUF Q4_0 / Q8_0)
    int head_t = WT_Q4_0;  // the LM head's: output.weight's, or token_embd's when tied (GGUF Q4_0, Q8_0 or Q6_K)
    size_t egu_stride = 0, ed_stride = 0;
    float *hn = nullptr, *rlog = nullptr, *mw = nullptr;  // normed rows, router logits, routing weights
    int32_t *mid = nullptr, *prow = nullptr, *rsrc = nullptr, *gitems = nullptr, *gcount = nullptr;

    hipStream_t st = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<void*> allocs;

    float *tok_embd = nullptr, *out_norm = nullptr;
    uint8_t* head = nullptr;
    std::vector<DevLayer> ly;
    // the guess head (MTP): its block, eh_proj stripes [E][2E], enorm, hnorm, the norm before the LM head
    DevLayer mtp;
    uint8_t* mtp_eh = nullptr;
    float *mtp_enorm = nullptr, *mtp_hnorm = nullptr, *mtp_hdnorm = nullptr;
    // its rows' buffers: mhn the step's rows after the output norm, mpend each slot's last one (the next head row's
    // hidden state), mhg the head rows' own output states, mx their residual rows, mcat [enorm(embed); hnorm(h)] rows
    float *mhn = nullptr, *mpend = nullptr, *mhg = nullptr, *mx = nullptr, *mcat = nullptr;
    int32_t* d_gtok = nullptr;  // guesses [4][slots]
    // the last step's run of rows of each slot (first row, its position, rows): sn_clear keeps mpend at the cut
    std::vector<int> run_row, run_pos, run_n;
    uint16_t *kbase = nullptr, *vbase = nullptr;
    size_t layer_halves = 0;  // one layer's K (or V) pool, in fp16 values
    int32_t* d_pt = nullptr;

    float *x = nullptr, *qkv = nullptr, *ao = nullptr, *hb = nullptr, *logits = nullptr, *gemm_ws = nullptr;
    size_t gemm_ws_bytes = 0;
    uint8_t* xa = nullptr;
    uint8_t* xa2 = nullptr;  // the down projection's operand when gate|up writes it (q4_gemm_swiglu, q4_gemm_fused)
    // the streaming matmul's fused epilogues (q4_gemm_fused): on when the open-time probe found the device dealing
    // workgroups to its XCDs in turn (snx_fuse switches them off and on); the arrival counters and the XCD check word
    bool fuse = false, fuse_ok = false;
    int nxcd = 1;
    uint64_t* d_fcnt = nullptr;
    int32_t* d_gcnt = nullptr;  // the one-launch MoE routing's system-scope counter
    // the row kernels read the next matmul's first weight groups into the Infinity Cache (resid_quant's next_w); off
    // with SN_NO_PREFETCH
    bool prefetch = true;
    float2* rope_cs = nullptr;  // a step's rotation table (rope_table) [max_rows][64]
    int32_t* d_xerr = nullptr;
    int fcnt_len = 0;
    // the attention's chunk items and merge in one launch (k_attn_fold): withdrawn, always off. Measured slower (60.2
    // against 53.0 + 5.8 us a layer at configs[2]), and one run of its bitwise test against the two launches differed
    // on one MI355X with no cause found, so no step takes it.
    bool attn_fold = false;
    float* apart = nullptr;
    int max_chunks = 0;
    uint8_t *d_stage = nullptr, *h_stage = nullptr;
    size_t stage_bytes = 0;
    int32_t *d_otok = nullptr, *h_otok = nullptr;
    float *d_rec = nullptr, *h_rec = nullptr;
    int32_t* d_ban = nullptr;
    uint8_t* d_amx = nullptr;  // the argmax's per-chunk partials
    size_t amx_bytes = 0;

    std::vector<int32_t> pt;  // [slots][max_pages], -1: no page
    std::vector<int> ref;     // holders of each page
    std::vector<int> freel;   // free pages
    bool pt_dirty = true;
    std::vector<int32_t> eog;
    std::vector<uint8_t> no_end;
    bool want_probs = false;
    int attn_mode = -1;  // the attention work list's form (snx_attn_mode)
    int last_n_out = 0, last_pn = 0;
    std::vector<float> last_probs;
    double last_ms = 0.0;
    int guess_on = 0;

    // the device work of recent step shapes, captured as HIP graphs and replayed while a shape repeats: a key is every
    // host value a launch of the step takes (the buffer set, row counts, work-list sizes, staging offsets), so a replay
    // issues exactly the launches an eager step would. A few shapes are kept (least recently used first out): chained
    // steps alternate buffer sets.
    bool graphs = true;
    struct GraphEnt {
        std::vector<int64_t> key;
        hipGraphExec_t ex;
    };
    std::vector<GraphEnt> gcache;
    long graph_replays = 0, graph_captures = 0;

    // the other buffer set, and which of the two the engine's fields are (part of every graph key)
    StepSet alt;
    int set_id = 0;
    // the queued step (sn_step's chain, sn_step.inc.h:31-212): R write rows of slots ch_seq at ch_pos (one past the step
    // before), fed that step's tokens ch_tok on the GPU; it runs in `alt` until taken or dropped
    bool ch_on = false;
    int ch_R = 0, ch_fast = 0;
    bool ch_probs = false;
    long ch_cfg = 0;
    std::vector<int32_t> ch_seq, ch_pos, ch_tok;
    long ch_taken = 0, ch_dropped = 0;
    // bumped by the calls that change how a step chooses its tokens (end ids, no-end slots, probability records): a
    // step queued before such a call is not the step asked for after it
    long cfg_gen = 0;

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
        *why = "tensor " + name + " has an unsupported type (Q4_0 or Q8_0 matrices, all of one type, and F32 norms / "
               "embedding are served)";
        t = nullptr;
    }
    return t;
}

// a GGUF Q4_0 / Q8_0 matrix (ne = [K, N]) into tiles at dst (stripe stride / offset for interleaving); Q6_K (the
// head) into its own tiles
bool upload_q4(sn_engine* e, const GgufTensor* t, uint8_t* tmp, uint8_t* dst, int sstride, int soff, char* err,
               int err_len) {
    SN_HIP_TRY(hipMemcpyAsync(tmp, t->data, t->nbytes, hipMemcpyHostToDevice, e->st), false);
    if (t->type == GGML_Q6_K) q6k_repack(tmp, (int) t->ne[1], (int) t->ne[0], dst, e->st);
    else q4_repack(tmp, (int) t->ne[1], (int) t->ne[0], dst, sstride, soff, e->st, t->type == GGML_Q8_0 ? WT_Q8_0 : WT_Q4_0);
    SN_HIP_TRY(hipStreamSynchronize(e->st), false);
    return true;
}

// a GGUF Q4_0 / Q8_0 expert tensor (ne = [K, N, NE]) into per-expert tiles, expert x at dst + x * dst_stride
bool upload_q4_experts(sn_engine* e, const GgufTensor* t, uint8_t* tmp, uint8_t* dst, int NE, int N, int K,
                       size_t dst_stride, int sstride, int soff, char* err, int err_len) {
    SN_HIP_TRY(hipMemcpyAsync(tmp, t->data, t->nbytes, hipMemcpyHostToDevice, e->st), false);
    const size_t src_stride = (size_t) N * ggml_row_bytes(t->type, K);
    for (int x = 0; x < NE; ++x)
        q4_repack(tmp + x * src_stride, N, K, dst + x * dst_stride, sstride, soff, e->st, e->wt);
    SN_HIP_TRY(hipStreamSynchronize(e->st), false);
    return true;
}

// rows [r0, r0 + nr) of a token table as fp32: ggml's dequantize_row_q4_0 (x0 * d), _q8_0 (q * d) and _q6_K
// ((d * scale) * (q - 32)), element for element
void table_rows(const GgufTensor* t, int64_t r0, int64_t nr, float* out) {
    const int64_t K = t->ne[0];
    const size_t rb = ggml_row_bytes(t->type, K);
    auto h2f = [](const uint8_t* p) {
        _Float16 h;
        memcpy(&h, p, 2);
        return (float) h;
    };
    for (int64_t r = 0; r < nr; ++r) {
        const uint8_t* row = t->data + (size_t) (r0 + r) * rb;
        float* y = out + (size_t) r * K;
        if (t->type == GGML_F32) {
            memcpy(y, row, (size_t) K * 4);
        } else if (t->type == GGML_Q4_0) {
            for (int64_t b = 0; b < K / 32; ++b) {
                const uint8_t* blk = row + b * 18;
                const float d = h2f(blk);
                for (int j = 0; j < 16; ++j) {
                    y[32 * b + j] = (float) ((blk[2 + j] & 0x0F) - 8) * d;
                    y[32 * b + j + 16] = (float) ((blk[2 + j] >> 4) - 8) * d;
                }
            }
        } else if (t->type == GGML_Q8_0) {
            for (int64_t b = 0; b < K / 32; ++b) {
                const uint8_t* blk = row + b * 34;
                const float d = h2f(blk);
                for (int j = 0; j < 32; ++j) y[32 * b + j] = (float) (int8_t) blk[2 + j] * d;
            }
        } else {  // Q6_K
            for (int64_t b = 0; b < K / 256; ++b) {
                const uint8_t* blk = row + b * 210;
                const float d = h2f(blk + 208);
                const int8_t* sc = (const int8_t*) (blk + 192);
                for (int e = 0; e < 256; ++e) {
                    const int h = e >> 7, c = (e & 127) >> 5, l = e & 31;
                    const uint8_t lb = blk[64 * h + 32 * (c & 1) + l];
                    const int q = ((c < 2 ? lb & 15 : lb >> 4) | (((blk[128 + 32 * h + l] >> (2 * c)) & 3) << 4)) - 32;
                    y[256 * b + e] = (d * (float) sc[e >> 4]) * (float) q;
                }
            }
        }
    }
}

// the token table on the device as fp32 rows (a quantized table dequantized once here: the gathers read fp32)
float* upload_table(sn_engine* e, const GgufTensor* t, char* err, int err_len) {
    const int64_t K = t->ne[0], V = t->ne[1];
    float* d = e->dalloc<float>((size_t) V * K * 4, err, err_len);
    if (!d) return nullptr;
    const int64_t chunk = std::max<int64_t>(1, (64 << 20) / (K * 4));
    std::vector<float> buf((size_t) std::min(chunk, V) * K);
    const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    for (int64_t r0 = 0; r0 < V; r0 += chunk) {
        const int64_t nr = std::min(chunk, V - r0);
        std::vector<std::thread> th;
        for (unsigned k = 0; k < nt; ++k)
            th.emplace_back([&, k] {
                const int64_t a = nr * k / nt, b = nr * (k + 1) / nt;
                table_rows(t, r0 + a, b - a, buf.data() + (size_t) a * K);
            });
        for (auto& x : th) x.join();
        if (hipMemcpy(d + (size_t) r0 * K, buf.data(), (size_t) nr * K * 4, hipMemcpyHostToDevice) != hipSuccess) {
            sn_set_err(err, err_len, "upload of %s failed", t->name.c_str());
            return nullptr;
        }
    }
    return d;
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
    if (a != "qwen3" && a != "qwen3moe") {
        *why = "architecture '" + a + "': this engine serves qwen3 and qwen3moe models";
        return false;
    }
    if (a == "qwen3moe") {
        const int ne = (int) g.num(a + ".expert_count", 0), nu = (int) g.num(a + ".expert_used_count", 0);
        const int fe = (int) g.num(a + ".expert_feed_forward_length", 0);
        if (ne < 1 || ne > 256 || nu < 1 || nu > 8 || nu > ne || fe <= 0 || fe % 128) {
            *why = "experts: 1 .. 256 experts, 1 .. 8 used, expert FFN width a multiple of 128";
            return false;
        }
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
    // the token table: F32, Q4_0, Q8_0 or Q6_K; the head: output.weight, or the table when tied (sn_load.inc.h:341-352)
    const GgufTensor* te = g.find("token_embd.weight");
    const GgufTensor* to = g.find("output.weight");
    const GgufTensor* tq = g.find("blk.0.attn_q.weight");
    auto qtype = [](int t) { return t == GGML_Q4_0 || t == GGML_Q8_0 || t == GGML_Q6_K; };
    if (!te || !(te->type == GGML_F32 || qtype(te->type))) {
        *why = "token_embd must be F32, Q4_0, Q8_0 or Q6_K";
        return false;
    }
    const GgufTensor* head = to ? to : te;
    if (!qtype(head->type)) {
        *why = to ? "output.weight must be Q4_0, Q8_0 or Q6_K" : "a tied LM head needs a Q4_0, Q8_0 or Q6_K token table";
        return false;
    }
    if ((te->type == GGML_Q6_K || head->type == GGML_Q6_K) && E % 256) {
        *why = "a Q6_K token table or head needs an embedding length that is a multiple of 256";
        return false;
    }
    if (!tq || (tq->type != GGML_Q4_0 && tq->type != GGML_Q8_0)) {
        *why = "the layer matrices must be Q4_0 or Q8_0";
        return false;
    }
    // the row kernels after a layer matrix add its k-slices: every plan must stay within KS_MAX of them
    const int F = (int) g.num(a + ".feed_forward_length", 0), QD = H * D, NQKV = (H + 2 * KVH) * D;
    const int shapes[][2] = {{NQKV, E}, {E, QD}, {2 * F, E}, {E, F}, {E, 2 * E}};
    for (const auto& sh : shapes) {
        if (sh[0] <= 0 || sh[1] <= 0 || sh[1] % 32) continue;  // (absent: a MoE model's dense FFN width)
        const int ks = q4_plan(sh[0], sh[1], tq->type).ks;
        if (ks < 1 || ks > KS_MAX) {
            *why = "matrix " + std::to_string(sh[0]) + " x " + std::to_string(sh[1]) + " would take " + std::to_string(ks) +
                   " k-slices; the row kernels add at most " + std::to_string(KS_MAX);
            return false;
        }
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
    e->CL = e->L + (nextn > 0 ? 1 : 0);  // cache layers: the model's, then the guess head's
    e->E = (int) g.num(a + ".embedding_length", 0);
    e->H = (int) g.num(a + ".attention.head_count", 0);
    e->KVH = (int) g.num(a + ".attention.head_count_kv", 0);
    e->F = (int) g.num(a + ".feed_forward_length", 0);
    if (e->has_nextn && e->E > 4096) return fail("the guess head takes an embedding length of at most 4096");
    if (a == "qwen3moe") {
        e->NE = (int) g.num(a + ".expert_count", 0);
        e->NEU = (int) g.num(a + ".expert_used_count", 0);
        e->FE = (int) g.num(a + ".expert_feed_forward_length", 0);
    }
    e->eps = (float) g.num(a + ".attention.layer_norm_rms_epsilon", 1e-6);
    e->rope_base = (float) g.num(a + ".rope.freq_base", 1e6);
    e->n_ctx_train = (int) g.num(a + ".context_length", 0);
    e->theta_scale = powf(e->rope_base, -2.0f / (float) e->D);
    e->QD = e->H * e->D;
    e->KD = e->KVH * e->D;
    e->NQKV = e->QD + 2 * e->KD;
    const GgufTensor* emb = g.find("token_embd.weight");
    const GgufTensor* head_t = g.find("output.weight") ? g.find("output.weight") : emb;  // no output: tied
    e->wt = g.find("blk.0.attn_q.weight")->type == GGML_Q8_0 ? WT_Q8_0 : WT_Q4_0;  // every layer matrix is this type
    e->head_t = head_t->type;
    e->V = (int) emb->ne[1];
    const char* pe = getenv("SN_PAGE");
    e->page_cells = pe && atoi(pe) == 32 ? 32 : 64;
    e->slots = slots;
    e->ctx = (ctx + e->page_cells - 1) / e->page_cells * e->page_cells;
    e->max_pages = e->ctx / e->page_cells;
    e->n_pages = pages > 0 ? pages : slots * e->max_pages;
    e->max_rows = max_rows;
    // output rows a step may ask for: a write row per slot and a few drafts (sn_step.inc.h:97-99); with a guess head the
    // fused draft-verify step reads every verify row (up to 5 a slot)
    e->max_out = std::max(slots + 4, e->has_nextn ? std::min(max_rows, 5 * slots) : 0);
    e->max_chunks = (e->ctx + ATT_CHUNK - 1) / ATT_CHUNK;
    if (hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&e->ev0) != hipSuccess ||
        hipEventCreate(&e->ev1) != hipSuccess || hipEventCreate(&e->alt.ev0) != hipSuccess ||
        hipEventCreate(&e->alt.ev1) != hipSuccess)
        return fail("HIP stream / event creation failed (no GPU?)");

    // ---- weights
    const int E = e->E, QD = e->QD, KD = e->KD, F = e->F;
    size_t max_t = 0;
    for (const GgufTensor& t : g.tensors) max_t = std::max(max_t, t.nbytes);
    uint8_t* tmp = nullptr;
    if (hipMalloc(&tmp, max_t) != hipSuccess) return fail("hipMalloc of the upload buffer failed");
    bool ok = true;
    auto q4 = [&](const std::string& n, int N, int K) -> const GgufTensor* {
        const GgufTensor* t = need(g, n, e->wt, &why);
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
    if (emb->ne[0] != E || head_t->ne[0] != E || head_t->ne[1] != e->V) {
        hipFree(tmp);
        return fail("token_embd / output.weight have unexpected dimensions");
    }
    e->tok_embd = upload_table(e, emb, err, err_len);
    ok = ok && e->tok_embd;
    e->out_norm = f32("output_norm.weight", E);
    if (ok) {
        e->head = e->dalloc<uint8_t>(e->head_t == GGML_Q6_K ? q6t_bytes(e->V, E) : wt_bytes(e->head_t, e->V, E), err,
                                     err_len);
        ok = e->head && upload_q4(e, head_t, tmp, e->head, 1, 0, err, err_len);
    }
    auto load_layer = [&](int i, DevLayer& l) {
        const std::string p = "blk." + std::to_string(i) + ".";
        l.attn_norm = f32(p + "attn_norm.weight", E);
        l.q_norm = f32(p + "attn_q_norm.weight", e->D);
        l.k_norm = f32(p + "attn_k_norm.weight", e->D);
        l.ffn_norm = f32(p + "ffn_norm.weight", E);
        const GgufTensor *tq = q4(p + "attn_q.weight", QD, E), *tk = q4(p + "attn_k.weight", KD, E),
                         *tv = q4(p + "attn_v.weight", KD, E), *to = q4(p + "attn_output.weight", E, QD);
        if (!ok) return;
        l.wqkv = e->dalloc<uint8_t>(wt_bytes(e->wt, e->NQKV, E), err, err_len);
        l.wo = e->dalloc<uint8_t>(wt_bytes(e->wt, E, QD), err, err_len);
        ok = l.wqkv && l.wo;
        // q, k, v stripes one after another (one matmul for all three)
        ok = ok && upload_q4(e, tq, tmp, l.wqkv, 1, 0, err, err_len) &&
             upload_q4(e, tk, tmp, l.wqkv + wt_bytes(e->wt, QD, E), 1, 0, err, err_len) &&
             upload_q4(e, tv, tmp, l.wqkv + wt_bytes(e->wt, QD + KD, E), 1, 0, err, err_len) &&
             upload_q4(e, to, tmp, l.wo, 1, 0, err, err_len);
        if (!ok) return;
        if (e->NE > 0 && i < e->L) {  // experts (the guess head's block stays dense)
            const int NE = e->NE, FE = e->FE;
            const GgufTensor* tr = need(g, p + "ffn_gate_inp.weight", GGML_F32, &why);
            if (tr && (tr->ne[0] != E || tr->ne[1] != NE)) tr = nullptr, why = "router " + p + " has unexpected dims";
            auto q4e = [&](const std::string& n, int N, int K) -> const GgufTensor* {
                const GgufTensor* t = need(g, n, e->wt, &why);
                if (t && (t->ne[0] != K || t->ne[1] != N || t->ne[2] != NE)) {
                    why = "tensor " + n + " has unexpected dimensions";
                    t = nullptr;
                }
                return t;
            };
            const GgufTensor *tg = q4e(p + "ffn_gate_exps.weight", FE, E), *tu = q4e(p + "ffn_up_exps.weight", FE, E),
                             *td = q4e(p + "ffn_down_exps.weight", E, FE);
            ok = tr && tg && tu && td;
            if (!ok) return;
            l.router = upload_f32(e, tr, err, err_len);
            l.egu = e->dalloc<uint8_t>(e->egu_stride * NE, err, err_len);
            l.ed = e->dalloc<uint8_t>(e->ed_stride * NE, err, err_len);
            ok = l.router && l.egu && l.ed;
            // per expert: gate and up stripes interleaved in pairs, down stripes; experts one after another
            ok = ok && upload_q4_experts(e, tg, tmp, l.egu, NE, FE, E, e->egu_stride, 2, 0, err, err_len) &&
                 upload_q4_experts(e, tu, tmp, l.egu, NE, FE, E, e->egu_stride, 2, 1, err, err_len) &&
                 upload_q4_experts(e, td, tmp, l.ed, NE, E, FE, e->ed_stride, 1, 0, err, err_len);
            return;
        }
        const GgufTensor *tg = q4(p + "ffn_gate.weight", F, E), *tu = q4(p + "ffn_up.weight", F, E),
                         *td = q4(p + "ffn_down.weight", E, F);
        if (!ok) return;
        l.wgu = e->dalloc<uint8_t>(wt_bytes(e->wt, 2 * F, E), err, err_len);
        l.wd = e->dalloc<uint8_t>(wt_bytes(e->wt, E, F), err, err_len);
        ok = l.wgu && l.wd;
        // gate and up stripes interleaved in pairs
        ok = ok && upload_q4(e, tg, tmp, l.wgu, 2, 0, err, err_len) && upload_q4(e, tu, tmp, l.wgu, 2, 1, err, err_len) &&
             upload_q4(e, td, tmp, l.wd, 1, 0, err, err_len);
    };
    if (e->NE > 0) {
        e->egu_stride = wt_bytes(e->wt, 2 * e->FE, E);
        e->ed_stride = wt_bytes(e->wt, E, e->FE);
    }
    e->ly.resize(e->L);
    for (int i = 0; i < e->L && ok; ++i) load_layer(i, e->ly[i]);
    if (e->has_nextn && ok) {
        // the guess head (sn_load.inc.h:134-147): block L, eh_proj [E][2E], its norms; shared_head_norm falls back to
        // the model's output norm
        load_layer(e->L, e->mtp);
        const std::string p = "blk." + std::to_string(e->L) + ".nextn.";
        if (const GgufTensor* t = ok ? q4(p + "eh_proj.weight", E, 2 * E) : nullptr) {
            e->mtp_eh = e->dalloc<uint8_t>(wt_bytes(e->wt, E, 2 * E), err, err_len);
            ok = e->mtp_eh && upload_q4(e, t, tmp, e->mtp_eh, 1, 0, err, err_len);
        }
        if (ok) e->mtp_enorm = f32(p + "enorm.weight", E);
        if (ok) e->mtp_hnorm = f32(p + "hnorm.weight", E);
        if (ok) e->mtp_hdnorm = g.find(p + "shared_head_norm.weight") ? f32(p + "shared_head_norm.weight", E) : e->out_norm;
    }
    hipFree(tmp);
    if (!ok) return fail(why.empty() ? std::string() : why);

    // ---- the KV pool: per layer, K then V, pages of [KVH][page_cells][128] fp16 (K regions chunk-major: kcell_at), zeroed
    e->layer_halves = (size_t) e->n_pages * e->KVH * e->page_cells * e->D;
    e->kbase = e->dalloc<uint16_t>(e->layer_halves * 2 * e->CL * sizeof(uint16_t), err, err_len);
    if (!e->kbase) return fail("");
    e->vbase = e->kbase + e->layer_halves * e->CL;
    if (hipMemset(e->kbase, 0, e->layer_halves * 2 * e->CL * 2) != hipSuccess) return fail("KV pool clear failed");
    e->pt.assign((size_t) slots * e->max_pages, -1);
    e->ref.assign(e->n_pages, 0);
    for (int p = e->n_pages - 1; p >= 0; --p) e->freel.push_back(p);
    e->no_end.assign(slots, 0);

    // ---- step buffers
    const int R = max_rows, MO = e->max_out;
    const int KMAX = std::max(std::max(E, QD), std::max(F, e->has_nextn ? 2 * E : 0));
    e->d_pt = e->dalloc<int32_t>(e->pt.size() * 4, err, err_len);
    e->x = e->dalloc<float>((size_t) R * E * 4, err, err_len);
    e->qkv = e->dalloc<float>((size_t) R * e->NQKV * 4, err, err_len);
    e->ao = e->dalloc<float>((size_t) R * QD * 4, err, err_len);
    e->hb = e->dalloc<float>((size_t) R * F * 4, err, err_len);
    e->logits = e->dalloc<float>((size_t) MO * e->V * 4, err, err_len);
    // MoE: a step's (row, expert) pairs in expert-major tiles of 16 rows: at most one partial tile per expert used
    const int RK = R * e->NEU;
    if (RK > 4096) return fail("a MoE model's steps take at most 4096 / experts-used rows (max_rows)");
    e->moe_tiles = e->NE > 0 ? std::min(e->NE, RK) + (RK + 15) / 16 : 0;
    const int P = e->moe_tiles * 16;
    // xa also holds the Q6_K head's Q8_K records
    e->xa = e->dalloc<uint8_t>(std::max({xa_bytes(R, KMAX), e->NE > 0 ? xa_bytes(P, std::max(E, e->FE)) : 0,
                                         e->head_t == GGML_Q6_K ? xk_bytes(MO, E) : 0}),
                               err, err_len);
    if (e->NE == 0 && F > 0) e->xa2 = e->dalloc<uint8_t>(xa_bytes(R, F), err, err_len);
    if (e->NE > 0) e->xa2 = e->dalloc<uint8_t>(xa_bytes(P, e->FE), err, err_len);  // (grouped gate|up + SwiGLU)
    // the fused epilogues' arrival counters (sets x row-tile groups of any decode-sized launch; zero between launches:
    // each set's last workgroup resets its own) and the XCD check word
    e->fcnt_len = 1 << 16;
    e->d_fcnt = e->dalloc<uint64_t>((size_t) e->fcnt_len * 8, err, err_len);
    e->d_xerr = e->dalloc<int32_t>(4, err, err_len);
    e->d_gcnt = e->dalloc<int32_t>(4, err, err_len);
    if (!e->d_fcnt || !e->d_xerr || !e->d_gcnt || hipMemset(e->d_fcnt, 0, (size_t) e->fcnt_len * 8) != hipSuccess ||
        hipMemset(e->d_xerr, 0, 4) != hipSuccess || hipMemset(e->d_gcnt, 0, 4) != hipSuccess)
        return fail("fused-epilogue counters");
    e->rope_cs = e->dalloc<float2>((size_t) std::max(R, slots) * 64 * sizeof(float2), err, err_len);
    if (!e->rope_cs) return fail("");
    e->fuse_ok = xcd_round_robin(e->st, &e->nxcd);
    e->fuse = e->fuse_ok && !getenv("SN_NO_FUSE");
    e->prefetch = !getenv("SN_NO_PREFETCH");
    e->attn_fold = false;  // (withdrawn: see attn_fold)
    size_t ws = 0;
    ws = std::max(ws, q4_workspace_bytes(R, e->NQKV, E, e->wt));
    ws = std::max(ws, q4_workspace_bytes(R, E, QD, e->wt));
    if (F > 0) {
        ws = std::max(ws, q4_workspace_bytes(R, 2 * F, E, e->wt));
        ws = std::max(ws, q4_workspace_bytes(R, E, F, e->wt));
    }
    if (e->head_t != GGML_Q6_K) ws = std::max(ws, q4_workspace_bytes(MO, e->V, E, e->head_t));
    if (e->NE > 0) {
        ws = std::max(ws, (size_t) P * 2 * e->FE * 4);  // grouped expert matmuls: one slice
        ws = std::max(ws, (size_t) P * E * 4);
        const int NU = e->NEU;
        e->hn = e->dalloc<float>((size_t) R * E * 4, err, err_len);
        e->rlog = e->dalloc<float>((size_t) R * e->NE * 4, err, err_len);
        e->mw = e->dalloc<float>((size_t) R * NU * 4, err, err_len);
        e->mid = e->dalloc<int32_t>((size_t) R * NU * 4, err, err_len);
        e->prow = e->dalloc<int32_t>((size_t) R * NU * 4, err, err_len);
        e->rsrc = e->dalloc<int32_t>((size_t) P * 4, err, err_len);
        e->gitems = e->dalloc<int32_t>((size_t) e->moe_tiles * 2 * 4, err, err_len);
        e->gcount = e->dalloc<int32_t>(4, err, err_len);
        if (!e->hn || !e->rlog || !e->mw || !e->mid || !e->prow || !e->rsrc || !e->gitems || !e->gcount) return fail("");
    }
    if (e->has_nextn) {
        ws = std::max(ws, q4_workspace_bytes(R, E, 2 * E, e->wt));    // eh_proj
        ws = std::max(ws, q4_workspace_bytes(R, 2 * KD, E, e->wt));   // the head's k|v (its cache fill)
    }
    e->gemm_ws_bytes = ws;
    e->gemm_ws = e->dalloc<float>(ws, err, err_len);
    e->apart = e->dalloc<float>((size_t) R * e->H * e->max_chunks * (e->D + 2) * 4, err, err_len);
    // staging: tok, seq, pos (R each), out_rows (MO), skip (MO bytes, padded), groups (R), items (R * max_chunks), pt
    // (+ with a guess head: 4 rounds of head rows, one a slot, their groups and items; row sources and keep lists)
    e->stage_bytes = (size_t) 3 * R * 4 + (size_t) MO * 4 + ((MO + 15) / 16 * 16) + (size_t) R * sizeof(AttnGroup) +
                     (size_t) R * e->max_chunks * sizeof(AttnItem) + (size_t) R * 4 + e->pt.size() * 4 + 256 + 64;
    if (e->has_nextn)
        e->stage_bytes += (size_t) 4 * slots * (sizeof(AttnGroup) + e->max_chunks * sizeof(AttnItem) + 4 + 64) +
                          (size_t) 16 * R * 4 + 4096;
    e->d_stage = e->dalloc<uint8_t>(e->stage_bytes, err, err_len);
    e->d_otok = e->dalloc<int32_t>((size_t) MO * 4, err, err_len);
    e->d_rec = e->dalloc<float>((size_t) MO * 32, err, err_len);
    e->alt.d_stage = e->dalloc<uint8_t>(e->stage_bytes, err, err_len);
    e->alt.d_otok = e->dalloc<int32_t>((size_t) MO * 4, err, err_len);
    e->alt.d_rec = e->dalloc<float>((size_t) MO * 32, err, err_len);
    e->alt.logits = e->dalloc<float>((size_t) MO * e->V * 4, err, err_len);
    if (!e->alt.d_stage || !e->alt.d_otok || !e->alt.d_rec || !e->alt.logits) return fail("");
    e->d_ban = e->dalloc<int32_t>(8 * 4, err, err_len);
    e->amx_bytes = argmax_workspace_bytes(MO, e->V);
    e->d_amx = e->dalloc<uint8_t>(e->amx_bytes, err, err_len);
    if (!e->d_pt || !e->x || !e->qkv || !e->ao || !e->hb || !e->logits || !e->xa || !e->gemm_ws || !e->apart ||
        !e->d_stage || !e->d_otok || !e->d_rec || !e->d_ban || !e->d_amx)
        return fail("");
    if (e->has_nextn) {
        const int RS = std::max(R, slots);
        e->mhn = e->dalloc<float>((size_t) R * E * 4, err, err_len);
        e->mpend = e->dalloc<float>((size_t) slots * E * 4, err, err_len);
        e->mhg = e->dalloc<float>((size_t) RS * E * 4, err, err_len);
        e->mx = e->dalloc<float>((size_t) RS * E * 4, err, err_len);
        e->mcat = e->dalloc<float>((size_t) RS * 2 * E * 4, err, err_len);
        e->d_gtok = e->dalloc<int32_t>((size_t) 4 * slots * 4, err, err_len);
        if (!e->mhn || !e->mpend || !e->mhg || !e->mx || !e->mcat || !e->d_gtok) return fail("");
        if (hipMemset(e->mpend, 0, (size_t) slots * E * 4) != hipSuccess) return fail("guess-head state clear failed");
        e->run_row.assign(slots, -1);
        e->run_pos.assign(slots, 0);
        e->run_n.assign(slots, 0);
    }
    if (hipHostMalloc((void**) &e->h_stage, e->stage_bytes, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->h_otok, (size_t) MO * 4, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->h_rec, (size_t) MO * 32, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->alt.h_stage, e->stage_bytes, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->alt.h_otok, (size_t) MO * 4, 0) != hipSuccess ||
        hipHostMalloc((void**) &e->alt.h_rec, (size_t) MO * 32, 0) != hipSuccess)
        return fail("pinned host buffers failed");
    return e;
}

namespace {
void swap_sets(sn_engine* e);
int settle(sn_engine* e);
}  // namespace

extern "C" void sn_close(sn_engine* e) {
    if (!e) return;
    if (e->st) hipStreamSynchronize(e->st);  // (a queued step ends; its cells go with the pool)
    for (void* p : e->allocs) hipFree(p);
    for (int k = 0; k < 2; ++k) {  // both buffer sets
        if (e->h_stage) hipHostFree(e->h_stage);
        if (e->h_otok) hipHostFree(e->h_otok);
        if (e->h_rec) hipHostFree(e->h_rec);
        if (e->ev0) hipEventDestroy(e->ev0);
        if (e->ev1) hipEventDestroy(e->ev1);
        e->h_stage = nullptr, e->h_otok = nullptr, e->h_rec = nullptr, e->ev0 = nullptr, e->ev1 = nullptr;
        swap_sets(e);
    }
    for (auto& ev : e->prof_ev) hipEventDestroy(ev);
    for (auto& g : e->gcache) hipGraphExecDestroy(g.ex);
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
        kv_page_op(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, e->page_cells, -1, p, 0, e->page_cells, e->st);
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

namespace {

// One staging copy of a step's inputs: pieces 16-byte aligned in the pinned host buffer, copied to the device at once.
struct Stage {
    sn_engine* e;
    size_t off = 0;
    bool over = false;
    size_t put(const void* src, size_t n) {
        const size_t at = off;
        if (at + n > e->stage_bytes) {
            over = true;
            return 0;
        }
        if (n) memcpy(e->h_stage + at, src, n);
        off = (off + n + 15) / 16 * 16;
        return at;
    }
    template <class T>
    size_t put(const std::vector<T>& v) { return put(v.data(), v.size() * sizeof(T)); }
    template <class T>
    T* dev(size_t at) const { return (T*) (e->d_stage + at); }
};

// The attention work of R rows (attn_plan: run items for prompt rows, then whole groups or per-chunk items and the
// rows to merge). bytes (the algorithmic bytes of the attention launches): each (sequence, KV head) reads its cells
// once, q in, page-table entries, and for the rows of run items and whole groups the outputs and the o-projection
// operand out (the chunk partials, an intermediate, are not counted); merge_bytes: the partials in, the outputs and
// the operand out (the rows of chunk items).
struct AttnList {
    size_t o_grp = 0, o_itm = 0, o_mrow = 0, o_run = 0;
    int n_items = 0, n_mrows = 0, n_runs = 0;
    bool whole = false;
    // plain chunk items (no shared chunks, runs or whole groups: every group's chunks 0 .. nc - 1, one item each), the
    // group count and the most chunks of a group: the form the fold launch takes
    bool plain = false;
    int n_groups = 0, max_nc = 0;
    double bytes = 0.0, merge_bytes = 0.0;
    // every value of the list the attention launches take, for a graph key: the form (whole groups launch another
    // kernel and no merge), the item, merge-row and run-item counts (grid sizes) and the staging offsets of the arrays
    void key(std::vector<int64_t>& k) const {
        k.insert(k.end(), {(int64_t) whole, (int64_t) n_items, (int64_t) n_mrows, (int64_t) o_grp, (int64_t) o_itm,
                           (int64_t) o_mrow, (int64_t) n_runs, (int64_t) o_run, (int64_t) plain, (int64_t) n_groups,
                           (int64_t) max_nc});
    }
};

AttnList attn_list(sn_engine* e, Stage& S, int R, const int32_t* seq, const int32_t* pos) {
    AttnPlan p;
    attn_plan(R, seq, pos, e->H, e->KVH, e->page_cells, p, e->attn_mode, e->pt.empty() ? nullptr : e->pt.data(),
              e->max_pages);
    AttnList al;
    al.o_grp = S.put(p.groups);
    al.o_itm = S.put(p.items);
    al.o_mrow = S.put(p.mrows);
    al.o_run = S.put(p.runs);
    al.n_items = (int) p.items.size();
    al.n_mrows = (int) p.mrows.size();
    al.n_runs = (int) p.runs.size();
    al.whole = p.whole;
    al.n_groups = (int) p.groups.size();
    al.plain = !p.whole && p.runs.empty() && !p.items.empty();
    int nct = 0;
    for (const AttnGroup& g : p.groups) {
        const int nc = (g.pos0 + g.nrows - 1) / ATT_CHUNK + 1;
        al.max_nc = std::max(al.max_nc, nc);
        nct += nc;
    }
    for (const AttnItem& it : p.items) al.plain = al.plain && it.share[0] < 0;
    al.plain = al.plain && nct == al.n_items;
    // chunk partials: (acc[128], m, l) per (row, head, chunk of the row), for the rows the merge folds
    double part = 0.0;
    for (const AttnGroup& g : p.groups)
        for (int i = 0; i < g.nrows; ++i)
            if (std::find(p.mrows.begin(), p.mrows.end(), g.row0 + i) != p.mrows.end())
                part += (double) ((g.pos0 + i) / ATT_CHUNK + 1) * e->H * (e->D + 2) * 4;
    const double row_out = (double) e->QD * 4 + (double) e->QD / 32 * 76;  // a row's output and operand (76 B a block)
    const double merged = (double) p.mrows.size();
    al.bytes = (double) R * e->QD * 4 + (R - merged) * row_out;
    al.merge_bytes = merged > 0 ? part + merged * row_out : 0.0;
    std::vector<int> seen;
    for (const AttnGroup& g : p.groups) {
        if (std::find(seen.begin(), seen.end(), g.seq) != seen.end()) continue;
        seen.push_back(g.seq);
        int last = 0;
        for (const AttnGroup& h : p.groups)
            if (h.seq == g.seq) last = std::max(last, h.pos0 + h.nrows - 1);
        al.bytes += (double) (last + 1) * e->KD * 2 * 2 + 4.0 * (last / e->page_cells + 1);
    }
    return al;
}

// A page for every cell the rows read or write: the attention reads cells 0 .. pos of every row, and a chunk a
// sequence never wrote is a zero page. Out of pages: -2 with nothing taken.
int take_pages(sn_engine* e, int R, const int32_t* seq, const int32_t* pos) {
    std::vector<std::pair<int, int>> fresh;
    for (int r = 0; r < R; ++r)
        for (int c = 0; c <= pos[r] / e->page_cells; ++c) {
            int32_t* t = e->seq_pages(seq[r]) + c;
            if (*t >= 0) continue;
            const int p = page_new(e);
            if (p < 0) {
                for (auto& f : fresh) {  // give back what this call took (never written, so still zero)
                    int32_t* tp = e->seq_pages(f.first) + f.second;
                    e->ref[*tp] = 0;
                    e->freel.push_back(*tp);
                    *tp = -1;
                }
                return -2;
            }
            *t = p;
            fresh.push_back({seq[r], c});
            e->pt_dirty = true;
        }
    return 0;
}

// the staged inputs to the device (and the page table when it changed); starts the step's GPU clock
// exchange the engine's buffer set with the other one
void swap_sets(sn_engine* e) {
    std::swap(e->d_stage, e->alt.d_stage);
    std::swap(e->h_stage, e->alt.h_stage);
    std::swap(e->d_otok, e->alt.d_otok);
    std::swap(e->h_otok, e->alt.h_otok);
    std::swap(e->d_rec, e->alt.d_rec);
    std::swap(e->h_rec, e->alt.h_rec);
    std::swap(e->logits, e->alt.logits);
    std::swap(e->ev0, e->alt.ev0);
    std::swap(e->ev1, e->alt.ev1);
    e->set_id ^= 1;
}

int stage_copy(sn_engine* e, Stage& S) {
    const bool send_pt = e->pt_dirty;
    const size_t o_pt = send_pt ? S.put(e->pt) : 0;
    if (S.over) return -1;
    if (hipEventRecord(e->ev0, e->st) != hipSuccess ||
        hipMemcpyAsync(e->d_stage, e->h_stage, S.off, hipMemcpyHostToDevice, e->st) != hipSuccess)
        return -1;
    if (send_pt) {
        if (hipMemcpyAsync(e->d_pt, e->d_stage + o_pt, e->pt.size() * 4, hipMemcpyDeviceToDevice, e->st) != hipSuccess)
            return -1;
        e->pt_dirty = false;
    }
    return 0;
}

// algorithmic bytes of a matmul: the weights (18 or 34 bytes a block) + fp32 input rows + fp32 output rows
double gemm_bytes(int wt, int M, int N, int K) {
    return (double) N * (K / 32) * (wt == WT_Q8_0 ? 34 : 18) + (double) M * K * 4 + (double) M * N * 4;
}

// Device work of a step, all on the engine's stream. Matmuls leave their k-slice sums in the workspace; the next row
// kernel adds them in slice order and applies the epilogue (RoPE for q|k|v, residual add + RMSNorm + Q8_0 for o and
// down, SwiGLU + Q8_0 for gate/up).
struct Dev {
    sn_engine* e;
    hipStream_t st;
    const int32_t* cs_pos = nullptr;  // the positions whose rotation table e->rope_cs holds in this step
    int cs_R = 0;
    int ks = 0;  // k-slices of the last matmul
    bool moe_pending = false;  // x awaits a MoE layer's weighted expert rows (added by the next resid)
    int rc = 0;

    void gemm(const uint8_t* w, int M, int N, int K, const uint8_t* xa = nullptr) {
        rc |= e->launch(SNX_K_GEMM, gemm_bytes(e->wt, M, N, K), [&] {
            ks = q4_gemm_raw(w, xa ? xa : e->xa, M, N, K, e->gemm_ws, e->gemm_ws_bytes, st, e->wt);
            return ks < 0 ? -1 : 0;
        });
    }
    // prompt rows: gate|up with its SwiGLU + Q8_0 as the epilogue (the rows h and the down projection's operand in
    // xa2); false when the shape does not take it
    bool gemm_swiglu(const uint8_t* w, int M) {
        const int F = e->F, E = e->E;
        if (!e->xa2 || !q4_gemm_swiglu_fits(M, 2 * F, E, e->wt)) return false;
        rc |= e->launch(SNX_K_GEMM, gemm_bytes(e->wt, M, 2 * F, E) - (double) M * F * 4 + (double) M * F * 6, [&] {
            return q4_gemm_swiglu(w, e->xa, M, 2 * F, E, e->hb, e->xa2, st, e->wt) == 1 ? 0 : -1;
        });
        return true;
    }
    // decode-sized rows: a matmul whose last workgroup of each set runs the set's epilogue (the split path's row
    // kernel, same bits); false when the engine or the shape has no fused launch (nothing launched)
    bool gemm_fused(const uint8_t* w, int M, int N, int K, int fe, GemmArgs& ea, double extra_bytes) {
        if (!e->fuse || !q4_gemm_fused_fits(M, N, K, e->wt, fe, e->nxcd, e->fcnt_len)) return false;
        ea.cnt = e->d_fcnt, ea.xerr = e->d_xerr, ea.nxcd = e->nxcd;
        int r = 0;
        rc |= e->launch(SNX_K_GEMM, gemm_bytes(e->wt, M, N, K) + extra_bytes, [&] {
            r = q4_gemm_fused(w, e->xa, M, N, K, e->gemm_ws, e->gemm_ws_bytes, st, e->wt, fe, ea, e->fcnt_len);
            return r < 0 ? -1 : 0;
        });
        return r == 1;
    }
    // the rotation table of R rows at positions d_pos (formed by one small launch when the step has not formed it)
    const float2* cs_for(int R, const int32_t* d_pos) {
        if (cs_pos != d_pos || cs_R < R) {
            rc |= e->launch(SNX_K_OTHER, (double) R * 64 * 8, [&] {
                rope_table(d_pos, R, e->theta_scale, e->rope_cs, st);
                return 0;
            });
            cs_pos = d_pos, cs_R = R;
        }
        return e->rope_cs;
    }
    // q|k|v with QK-norm + RoPE + the cache write fused (H query heads; 0 for the guess head's k|v)
    bool gemm_rope(const uint8_t* w, const DevLayer& l, int R, int N, int H, const int32_t* d_seq,
                   const int32_t* d_pos, uint16_t* kp, uint16_t* vp) {
        GemmArgs ea{};
        ea.qkv = e->qkv, ea.ldqkv = e->NQKV, ea.qw = l.q_norm, ea.kw = l.k_norm, ea.eps = e->eps;
        ea.theta_scale = e->theta_scale, ea.seq = d_seq, ea.pos = d_pos, ea.pt = e->d_pt, ea.max_pages = e->max_pages;
        ea.page_cells = e->page_cells, ea.kpool = kp, ea.vpool = vp, ea.H = H, ea.KVH = e->KVH;
        if (!e->fuse || !q4_gemm_fused_fits(R, N, e->E, e->wt, FE_ROPE, e->nxcd, e->fcnt_len)) return false;
        ea.rope_cs = cs_for(R, d_pos);
        return gemm_fused(w, R, N, e->E, FE_ROPE, ea, (double) R * (H * e->D * 4 + 2 * e->KD * 2));
    }
    // gate|up with SwiGLU + Q8_0 fused: the down projection's operand in xa2, the rows in hb
    bool gemm_swiglu_dec(const uint8_t* w, int R) {
        if (!e->xa2) return false;
        GemmArgs ea{};
        ea.h = e->hb, ea.xo = e->xa2;
        return gemm_fused(w, R, 2 * e->F, e->E, FE_SWIGLU, ea, (double) R * e->F * 6);
    }
    void quant(const float* x, const int32_t* rows, int M, int K, const float* nw, float* xn = nullptr) {
        rc |= e->launch(SNX_K_QUANT, (double) M * K * 8, [&] {
            quant_act(x, rows, M, K, K, nw, e->eps, e->xa, xn, K, st);
            return 0;
        });
    }
    // x (R rows of E) += the last matmul's sums (add false: x = the sums); then the Q8_0 operand of norm(x) when asked
    // (next_w: the next matmul's N x E matrix, whose first weight groups the launch reads into the Infinity Cache)
    void resid(float* x, int R, const float* nw, bool quantize, bool add = true, const uint8_t* next_w = nullptr,
               int next_N = 0) {
        const int E = e->E;
        if (moe_pending) {  // x += the MoE output (the grouped down matmul's rows, weighted), then the operand
            moe_pending = false;
            rc |= e->launch(SNX_K_QUANT, (double) R * e->NEU * E * 4 + (double) R * E * 8 +
                                             (quantize ? (double) R * E * 2 : 0.0), [&] {
                return moe_resid_quant(x, e->gemm_ws, e->prow, e->mw, e->NEU, R, E, nw, e->eps,
                                       quantize ? e->xa : nullptr, st);
            });
            return;
        }
        rc |= e->launch(SNX_K_QUANT, (double) R * E * (8 + 4 * ks) + (quantize ? (double) R * E * 2 : 0.0), [&] {
            return resid_quant(x, e->gemm_ws, ks, R, E, nw, e->eps, quantize ? e->xa : nullptr, st, add, nullptr,
                               e->prefetch ? next_w : nullptr, next_N, E, e->wt);
        });
    }
    void swiglu(int R) {
        const int F = e->F;
        rc |= e->launch(SNX_K_QUANT, (double) R * 2 * F * 4 * ks + (double) R * F * 6, [&] {
            return swiglu_quant(e->gemm_ws, ks, R, F, e->hb, e->xa, st);
        });
    }
    void rope(const DevLayer& l, int R, int H, const int32_t* d_seq, const int32_t* d_pos, uint16_t* kp, uint16_t* vp) {
        const int N = (H + 2 * e->KVH) * e->D;
        rc |= e->launch(SNX_K_ROPE, (double) R * (N * 4.0 * (ks + 1) + H * e->D * 4 + 2 * e->KD * 2), [&] {
            return qk_norm_rope_kv(e->qkv, e->NQKV, e->gemm_ws, ks, R, H, e->KVH, l.q_norm, l.k_norm, e->eps,
                                   e->theta_scale, d_seq, d_pos, e->d_pt, e->max_pages, e->page_cells, kp, vp, st,
                                   cs_pos == d_pos && cs_R >= R ? e->rope_cs : nullptr);
        });
    }
    void attention(const Stage& S, const AttnList& al, int R, const int32_t* d_pos, uint16_t* kp, uint16_t* vp) {
        AttnArgs aa{};
        aa.q = e->qkv;
        aa.ldq = e->NQKV;
        aa.kpool = kp;
        aa.vpool = vp;
        aa.pt = e->d_pt;
        aa.max_pages = e->max_pages;
        aa.page_cells = e->page_cells;
        aa.groups = S.dev<const AttnGroup>(al.o_grp);
        aa.items = S.dev<const AttnItem>(al.o_itm);
        aa.n_items = al.n_items;
        aa.runs = S.dev<const AttnItem>(al.o_run);
        aa.n_runs = al.n_runs;
        aa.part = e->apart;
        aa.max_chunks = e->max_chunks;
        aa.out = e->ao;
        aa.ldo = e->QD;
        aa.xa = e->xa;  // the merge writes the o-projection's Q8_0 operand itself
        aa.H = e->H;
        aa.KVH = e->KVH;
        aa.scale = 1.0f / sqrtf((float) e->D);
        aa.n_rows = R;
        aa.row_pos = d_pos;
        aa.whole = al.whole ? 1 : 0;
        aa.mrows = S.dev<const int32_t>(al.o_mrow);
        aa.n_mrows = al.n_mrows;
        // the merge folded into the chunk launch where the list is plain chunk items (one launch, the same bits)
        if (e->fuse && e->attn_fold && al.plain && al.max_nc <= 127 &&
            (long) al.n_groups * e->KVH * CNT_STRIDE <= e->fcnt_len) {
            aa.fold = 1, aa.n_groups = al.n_groups, aa.fold_chunks = al.max_nc, aa.nxcd = e->nxcd;
            aa.cnt = e->d_fcnt, aa.xerr = e->d_xerr;
        }
        if (al.n_runs > 0)  // (the class's bytes go with its first launch of the step)
            rc |= e->launch(SNX_K_ATTN, al.bytes, [&] { return attention_runs(aa, st); });
        if (al.n_items > 0)
            rc |= e->launch(SNX_K_ATTN, (al.n_runs > 0 ? 0.0 : al.bytes) + (aa.fold ? al.merge_bytes : 0.0),
                            [&] { return attention_items(aa, st); });
        if (!al.whole && al.n_mrows > 0 && !aa.fold)
            rc |= e->launch(SNX_K_MERGE, al.merge_bytes, [&] { return attention_merge(aa, st); });
    }
    uint16_t* kp(int layer) { return e->kbase + (size_t) layer * e->layer_halves; }
    uint16_t* vp(int layer) { return e->vbase + (size_t) layer * e->layer_halves; }

    // one block over R rows whose Q8_0 operand of attn_norm(x) is in xa. Returns whether x still awaits its down
    // projection's sums (left in the workspace: a dense FFN's k-slices, a MoE layer's expert rows); the next resid adds
    // them.
    bool block(const DevLayer& l, int layer, float* x, int R, const Stage& S, const AttnList& al, const int32_t* d_seq,
               const int32_t* d_pos) {
        const int E = e->E, F = e->F;
        if (!gemm_rope(l.wqkv, l, R, e->NQKV, e->H, d_seq, d_pos, kp(layer), vp(layer))) {
            gemm(l.wqkv, R, e->NQKV, E);
            rope(l, R, e->H, d_seq, d_pos, kp(layer), vp(layer));
        }
        attention(S, al, R, d_pos, kp(layer), vp(layer));
        gemm(l.wo, R, E, e->QD);
        if (l.egu) {
            moe(l, x, R);
            return true;
        }
        resid(x, R, l.ffn_norm, true, true, l.wgu, 2 * F);
        if (gemm_swiglu(l.wgu, R) || gemm_swiglu_dec(l.wgu, R)) {
            gemm(l.wd, R, E, F, e->xa2);
            return true;
        }
        gemm(l.wgu, R, 2 * F, E);
        swiglu(R);
        gemm(l.wd, R, E, F);
        return true;
    }

    // MoE FFN (moe_ffn, sn_layers.inc.h:129-144): x += o's sums, ffn norm (the rows kept as hn, their Q8_0 operand in
    // row order); router, top-k and renormalised weights; the (row, expert) pairs in expert-major 16-row tiles;
    // grouped gate/up (its operand rows gathered from hn's, SwiGLU + Q8_0) and down matmuls over the used experts; the
    // weighted sum in slot order into x
    void moe(const DevLayer& l, float* x, int R) {
        const int E = e->E, NE = e->NE, NU = e->NEU, FE = e->FE, T = e->moe_tiles, P = T * 16;
        rc |= e->launch(SNX_K_QUANT, (double) R * E * (8 + 4 * ks) + (double) R * E * 6, [&] {
            return resid_quant(x, e->gemm_ws, ks, R, E, l.ffn_norm, e->eps, e->xa, st, true, e->hn);
        });
        rc |= e->launch(SNX_K_OTHER, (double) NE * E * 4 + (double) R * E * 4, [&] {
            if (e->fuse && E <= MOE_ROUTE_EMAX)  // (one launch: the same results)
                return moe_route(e->hn, l.router, R, E, NE, NU, P, e->rlog, e->mid, e->mw, e->prow, e->rsrc, e->gitems,
                                 e->gcount, e->d_fcnt, e->fcnt_len, e->d_gcnt, e->d_xerr, e->nxcd, st);
            moe_router(e->hn, l.router, R, E, NE, e->rlog, st);
            return moe_select(e->rlog, R, NE, NU, P, e->mid, e->mw, e->prow, e->rsrc, e->gitems, e->gcount, st);
        });
        // the experts used (a host read only while profiling: the matmuls' algorithmic bytes)
        double used = std::min(NE, R * NU);
        if (e->prof_on) {
            std::vector<int32_t> it(2 * (size_t) T);
            int32_t n = 0;
            if (hipMemcpyAsync(&n, e->gcount, 4, hipMemcpyDeviceToHost, st) == hipSuccess &&
                hipMemcpyAsync(it.data(), e->gitems, it.size() * 4, hipMemcpyDeviceToHost, st) == hipSuccess &&
                hipStreamSynchronize(st) == hipSuccess) {
                std::vector<bool> seen(NE, false);
                used = 0;
                for (int i = 0; i < n && i < T; ++i)
                    if (!seen[it[2 * i]]) seen[it[2 * i]] = true, used += 1;
            }
        }
        // (the expert tiles' rows gathered from hn's Q8_0 operand, which the resid above wrote in row order)
        // gate|up with its SwiGLU + Q8_0 in one launch (into xa2) where the shape takes it; else the sums, then the
        // row kernel (into xa)
        const bool gsw = e->fuse && q4_gemm_grouped_swiglu_fits(2 * FE, E, e->wt);
        const uint8_t* xd = gsw ? e->xa2 : e->xa;  // the down projection's operand
        if (gsw) {
            rc |= e->launch(SNX_K_GEMM, used * e->egu_stride + (double) R * NU * E * 4 + (double) R * NU * FE * 1.0625,
                            [&] {
                                return q4_gemm_grouped_swiglu(l.egu, e->egu_stride, e->gitems, e->gcount, T, e->xa, P,
                                                              2 * FE, E, e->xa2, st, e->wt, e->rsrc, e->rsrc, R) == 1
                                           ? 0 : -1;
                            });
        } else {
            rc |= e->launch(SNX_K_GEMM, used * e->egu_stride + (double) R * NU * E * 4 + (double) R * NU * 2 * FE * 4,
                            [&] {
                                return q4_gemm_grouped(l.egu, e->egu_stride, e->gitems, e->gcount, T, e->xa, P, 2 * FE,
                                                       E, e->gemm_ws, e->gemm_ws_bytes, st, e->wt, e->rsrc, e->rsrc,
                                                       R) < 0 ? -1 : 0;
                            });
            rc |= e->launch(SNX_K_QUANT, (double) R * NU * FE * 14, [&] {
                return swiglu_quant(e->gemm_ws, 1, P, FE, nullptr, e->xa, st, e->rsrc);
            });
        }
        rc |= e->launch(SNX_K_GEMM, used * e->ed_stride + (double) R * NU * FE * 4 + (double) R * NU * E * 4, [&] {
            return q4_gemm_grouped(l.ed, e->ed_stride, e->gitems, e->gcount, T, xd, P, E, FE, e->gemm_ws,
                                   e->gemm_ws_bytes, st, e->wt, e->rsrc) < 0 ? -1 : 0;
        });
        moe_pending = true;  // x += the weighted expert rows: the next resid, fused with its norm and operand
    }

    // the model's layers over R rows (qwen_layers, sn_attn.inc.h:216-231); leaves x = the final residual rows
    void model(int R, const int32_t* d_tok, const int32_t* d_seq, const int32_t* d_pos, const Stage& S,
               const AttnList& al) {
        const int E = e->E;
        rc |= e->launch(SNX_K_OTHER, (double) R * E * 8, [&] { embed_rows(e->tok_embd, e->V, E, d_tok, R, e->x, st); return 0; });
        bool pending = false;  // x awaits the previous layer's down projection sums
        for (int i = 0; i < e->L && rc == 0; ++i) {
            if (pending) resid(e->x, R, e->ly[i].attn_norm, true, true, e->ly[i].wqkv, e->NQKV);  // x += them, then the attn_norm operand
            else quant(e->x, nullptr, R, E, e->ly[i].attn_norm);
            pending = block(e->ly[i], i, e->x, R, S, al, d_seq, d_pos);
        }
        if (rc == 0 && pending) resid(e->x, R, nullptr, false);  // x += the last layer's down projection
    }

    // output stage (sn_encode.inc.h:304-317): final norm of rows d_rows (n of them) of `x`, LM head, optional forced
    // drafts, greedy argmax into d_otok (and the probability records when on)
    void outputs(const float* x, int n, const int32_t* d_rows, const uint8_t* d_skip, const uint8_t* d_force = nullptr,
                 const int32_t* d_ftok = nullptr, int32_t* d_otok = nullptr, const float* hdnorm = nullptr) {
        const int V = e->V;
        head_logits(n, x, d_rows, hdnorm ? hdnorm : e->out_norm);
        if (d_force) force_rows(e->logits, V, n, d_force, d_ftok, st);
        const int nban = (int) e->eog.size();
        int32_t* out = d_otok ? d_otok : e->d_otok;
        rc |= e->launch(SNX_K_OTHER, (double) n * V * 4, [&] {
            return argmax_rows(e->logits, V, n, e->d_ban, nban, d_skip, out, e->want_probs && !d_otok ? e->d_rec : nullptr,
                               e->d_amx, e->amx_bytes, st);
        });
    }
    // the LM head over rows `rows` (n of them; null: the first n) of x after the norm nw (null: x is normed): a Q4_0 /
    // Q8_0 head from Q8_0 activations, a Q6_K head from Q8_K records (ggml's CPU operand for each type)
    void head_logits(int n, const float* x, const int32_t* rows, const float* nw) {
        const int E = e->E, V = e->V, ht = e->head_t;
        if (ht == GGML_Q6_K) {
            rc |= e->launch(SNX_K_QUANT, (double) n * E * 8, [&] {
                quant_q8k(x, rows, n, E, E, nw, e->eps, e->xa, st);
                return 0;
            });
            rc |= e->launch(SNX_K_GEMM, (double) V * (E / 256) * 210 + (double) n * E * 4 + (double) n * V * 4, [&] {
                return q6k_gemm(e->head, e->xa, n, V, E, e->logits, V, st);
            });
            return;
        }
        quant(x, rows, n, E, nw);
        head_logits_q(n);
    }
    // a Q4_0 / Q8_0 head over the xa operand's n rows
    void head_logits_q(int n) {
        const int E = e->E, V = e->V, ht = e->head_t;
        rc |= e->launch(SNX_K_GEMM, gemm_bytes(ht, n, V, E), [&] {
            if (q4_plan(V, E, ht).ks == 1)  // one slice: the sums are the logits
                return q4_gemm_raw(e->head, e->xa, n, V, E, e->logits, (size_t) n * V * 4, st, ht) < 0 ? -1 : 0;
            return q4_gemm(e->head, e->xa, n, V, E, e->logits, V, EPI_STORE, e->gemm_ws, e->gemm_ws_bytes, st, ht);
        });
    }

    // the guess head's cache cells of R rows (mtp_fill, sn_state.inc.h:283-313): mhn = the rows after the output norm;
    // row r pairs its token with src[r]'s hidden state (an earlier row of mhn, its slot's mpend, or none); eh_proj, the
    // head block's attn_norm, its k (QK-norm, RoPE) and v into the head's cache layer. keep: (slot, row) pairs whose
    // mhn row becomes the slot's mpend.
    void head_fill(int R, const int32_t* d_tok, const int32_t* d_seq, const int32_t* d_pos, const int32_t* d_src,
                   int nkeep, const int32_t* d_keep) {
        const int E = e->E;
        quant(e->x, nullptr, R, E, e->out_norm, e->mhn);
        rc |= e->launch(SNX_K_OTHER, (double) R * E * 16, [&] {
            mtp_cat(e->tok_embd, e->V, E, d_tok, e->mhn, e->mpend, d_src, d_seq, e->mtp_enorm, e->mtp_hnorm, e->eps,
                    e->mcat, R, st);
            return 0;
        });
        quant(e->mcat, nullptr, R, 2 * E, nullptr);
        gemm(e->mtp_eh, R, E, 2 * E);
        resid(e->mx, R, e->mtp.attn_norm, true, false);
        // the head's k|v stripes (rows QD .. QD + 2 KD of its q|k|v matrix)
        const uint8_t* wkv = e->mtp.wqkv + wt_bytes(e->wt, e->QD, E);
        if (!gemm_rope(wkv, e->mtp, R, 2 * e->KD, 0, d_seq, d_pos, kp(e->L), vp(e->L))) {
            gemm(wkv, R, 2 * e->KD, E);
            rope(e->mtp, R, 0, d_seq, d_pos, kp(e->L), vp(e->L));
        }
        if (nkeep > 0) rows_keep(e->mhn, d_keep, nkeep, E, e->mpend, st);
    }

    // n head rows (sn_cache.inc.h:357-369), row r at position d_pos[r] of slot d_seq[r], token d_tok[r], paired with its
    // slot's mpend (first) or with mhg row r (the head's previous output state): the head block (writing its cell),
    // the head norm (mhg), the LM head and argmax into d_gout
    void head_rows(int n, const int32_t* d_tok, const int32_t* d_seq, const int32_t* d_pos, bool first, const Stage& S,
                   const AttnList& al, int32_t* d_gout) {
        const int E = e->E;
        rc |= e->launch(SNX_K_OTHER, (double) n * E * 16, [&] {
            mtp_cat(e->tok_embd, e->V, E, d_tok, first ? nullptr : e->mhg, e->mpend, nullptr, d_seq, e->mtp_enorm,
                    e->mtp_hnorm, e->eps, e->mcat, n, st);
            return 0;
        });
        quant(e->mcat, nullptr, n, 2 * E, nullptr);
        gemm(e->mtp_eh, n, E, 2 * E);
        resid(e->mx, n, e->mtp.attn_norm, true, false);
        if (block(e->mtp, e->L, e->mx, n, S, al, d_seq, d_pos)) resid(e->mx, n, nullptr, false);
        quant(e->mx, nullptr, n, E, e->mtp_hdnorm, e->mhg);  // mhg: the head's output state (the next row's input)
        if (e->head_t == GGML_Q6_K) head_logits(n, e->mhg, nullptr, nullptr);
        else head_logits_q(n);
        rc |= e->launch(SNX_K_OTHER, (double) n * e->V * 4, [&] {
            return argmax_rows(e->logits, e->V, n, e->d_ban, 0, nullptr, d_gout, nullptr, e->d_amx, e->amx_bytes, st);
        });
    }
};

// the row sources of the guess head's fill (sn_state.inc.h:292): the row before in the step (same slot, position
// before), else the slot's kept state, none at position 0; and each run's last row kept as its slot's state
void head_sources(const sn_engine* e, int R, const int32_t* seq, const int32_t* pos, std::vector<int32_t>& src,
                  std::vector<int32_t>& keep) {
    (void) e;
    src.resize(R);
    keep.clear();
    for (int r = 0; r < R; ++r) {
        src[r] = r > 0 && seq[r] == seq[r - 1] && pos[r] == pos[r - 1] + 1 ? r - 1 : pos[r] == 0 ? -2 : -1;
        if (r + 1 == R || !(seq[r + 1] == seq[r] && pos[r + 1] == pos[r] + 1)) {
            keep.push_back(seq[r]);
            keep.push_back(r);
        }
    }
}

// the runs of the last step, for sn_clear's cut of the guess head's state
void note_runs(sn_engine* e, int R, const int32_t* seq, const int32_t* pos) {
    for (int r = 0; r < R;) {
        int n = 1;
        while (r + n < R && seq[r + n] == seq[r] && pos[r + n] == pos[r] + n) ++n;
        e->run_row[seq[r]] = r;
        e->run_pos[seq[r]] = pos[r];
        e->run_n[seq[r]] = n;
        r += n;
    }
}

// waits for the step; the GPU time and profiling records
int finish(sn_engine* e, int rc, char* err, int err_len, bool recorded = false) {
    if (!recorded) SN_HIP_TRY(hipEventRecord(e->ev1, e->st), -1);
    SN_HIP_TRY(hipEventSynchronize(e->ev1), -1);
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
    return 0;
}

// Run a step's device work on the engine's stream: replayed from the cached graph when the key matches, else captured
// into a new graph (replacing the cached one) and launched; run eagerly while profiling (events around each launch)
// or if capture is not available. The work issues kernels only: no copies, memsets or waits. Returns the work's rc.
template <class Work>
int run_device(sn_engine* e, std::vector<int64_t>&& key, Work work) {
    if (e->graphs && !e->prof_on) {
        key.insert(key.begin(), e->set_id);  // a set's graph holds that set's buffers
        for (size_t i = 0; i < e->gcache.size(); ++i)
            if (e->gcache[i].key == key) {
                std::rotate(e->gcache.begin() + i, e->gcache.begin() + i + 1, e->gcache.end());  // most recent last
                ++e->graph_replays;
                return hipGraphLaunch(e->gcache.back().ex, e->st) == hipSuccess ? 0 : -1;
            }
        if (hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal) == hipSuccess) {
            Dev d{e, e->st};
            work(d);
            hipGraph_t g = nullptr;
            const bool ok = hipStreamEndCapture(e->st, &g) == hipSuccess && g != nullptr;
            if (ok && d.rc != 0) {
                hipGraphDestroy(g);
                return d.rc;
            }
            hipGraphExec_t ex = nullptr;
            if (ok && hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) == hipSuccess) {
                hipGraphDestroy(g);
                if (e->gcache.size() >= GRAPH_CACHE) {
                    hipGraphExecDestroy(e->gcache.front().ex);
                    e->gcache.erase(e->gcache.begin());
                }
                e->gcache.push_back({std::move(key), ex});
                ++e->graph_captures;
                return hipGraphLaunch(ex, e->st) == hipSuccess ? 0 : -1;
            }
            if (g) hipGraphDestroy(g);
        }
        (void) hipGetLastError();  // capture unavailable: eager from now on
        e->graphs = false;
    }
    Dev d{e, e->st};
    work(d);
    return d.rc;
}

bool rows_bad(const sn_engine* e, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos) {
    for (int r = 0; r < R; ++r)
        if (seq[r] < 0 || seq[r] >= e->slots || pos[r] < 0 || pos[r] >= e->ctx || tok[r] < 0 || tok[r] >= e->V)
            return true;
    return false;
}

}  // namespace

namespace {

// The host half of a step: its inputs placed in the staging buffer (tokens, slots, positions, output rows, no-end
// flags, the attention work list, the guess head's row sources) and the key of its device work, which holds every host
// value the step's launches take, so that a cached graph is replayed only for a step that would launch exactly the
// same kernels with the same arguments.
struct StepStage {
    size_t o_tok = 0, o_seq = 0, o_pos = 0, o_out = 0, o_skip = 0, o_src = 0, o_keep = 0;
    int nkeep = 0;  // (slot, row) pairs whose head state is kept
    bool fill = false;
    AttnList al;
    std::vector<int64_t> key;
};

void stage_step(sn_engine* e, Stage& S, StepStage& ss, int R, const int32_t* tok, const int32_t* seq,
                const int32_t* pos, int n_out, const int32_t* out_rows) {
    ss.fill = e->has_nextn && e->guess_on;
    std::vector<int32_t> tz;
    if (!tok) tz.assign(R, 0);
    ss.o_tok = S.put(tok ? tok : tz.data(), (size_t) R * 4);
    ss.o_seq = S.put(seq, (size_t) R * 4);
    ss.o_pos = S.put(pos, (size_t) R * 4);
    ss.o_out = S.put(out_rows, (size_t) n_out * 4);
    std::vector<uint8_t> skip(n_out + 1, 0);
    for (int j = 0; j < n_out; ++j) skip[j] = e->no_end[seq[out_rows[j]]];
    ss.o_skip = S.put(skip);
    ss.al = attn_list(e, S, R, seq, pos);
    if (ss.fill) {
        std::vector<int32_t> src, keep;
        head_sources(e, R, seq, pos, src, keep);
        ss.o_src = S.put(src);
        ss.o_keep = S.put(keep);
        ss.nkeep = (int) keep.size() / 2;
    }
    ss.key = {1, R, n_out, ss.fill, e->want_probs, (int64_t) e->eog.size(), ss.nkeep, (int64_t) ss.o_tok,
              (int64_t) ss.o_seq, (int64_t) ss.o_pos, (int64_t) ss.o_out, (int64_t) ss.o_skip, (int64_t) ss.o_src,
              (int64_t) ss.o_keep};
    ss.al.key(ss.key);
}

// One step's device work, staged into the engine's buffer set and enqueued on the stream with the tokens'
// device-to-host copy; the set's end event recorded, nothing waited for. tok_dev: the rows' tokens are that device
// array (a queued step is fed the step before's outputs), else tok. Returns the device work's code (0, or -1 when a
// launch was refused), or -2 when the staging failed (nothing enqueued).
int enqueue_step(sn_engine* e, int R, const int32_t* tok, const int32_t* tok_dev, const int32_t* seq, const int32_t* pos,
                 int n_out, const int32_t* out_rows) {
    Stage S{e};
    StepStage ss;
    stage_step(e, S, ss, R, tok, seq, pos, n_out, out_rows);
    e->prof_recs.clear();
    if (stage_copy(e, S) != 0) return -2;
    if (tok_dev && hipMemcpyAsync(e->d_stage + ss.o_tok, tok_dev, (size_t) R * 4, hipMemcpyDeviceToDevice, e->st) != hipSuccess)
        return -2;
    const int32_t* d_tok = S.dev<const int32_t>(ss.o_tok);
    const int32_t* d_seq = S.dev<const int32_t>(ss.o_seq);
    const int32_t* d_pos = S.dev<const int32_t>(ss.o_pos);
    const AttnList& al = ss.al;
    const int drc = run_device(e, std::move(ss.key), [&](Dev& d) {
        d.model(R, d_tok, d_seq, d_pos, S, al);
        if (ss.fill && d.rc == 0)
            d.head_fill(R, d_tok, d_seq, d_pos, S.dev<const int32_t>(ss.o_src), ss.nkeep, S.dev<const int32_t>(ss.o_keep));
        if (n_out > 0 && d.rc == 0)
            d.outputs(e->x, n_out, S.dev<const int32_t>(ss.o_out), S.dev<const uint8_t>(ss.o_skip));
    });
    int rc = drc;
    if (drc == 0 && n_out > 0) {
        if (hipMemcpyAsync(e->h_otok, e->d_otok, (size_t) n_out * 4, hipMemcpyDeviceToHost, e->st) != hipSuccess ||
            (e->want_probs &&
             hipMemcpyAsync(e->h_rec, e->d_rec, (size_t) n_out * 32, hipMemcpyDeviceToHost, e->st) != hipSuccess))
            rc = -1;
    }
    return hipEventRecord(e->ev1, e->st) == hipSuccess ? rc : -2;  // the step's end, before anything queued behind it
}

// The step in the engine's buffer set (its end event recorded): wait for it, take its tokens and probability records
int take_step(sn_engine* e, int rc, int R, const int32_t* seq, const int32_t* pos, int n_out, int32_t* out_tok,
              char* err, int err_len) {
    if (rc == -2) {
        sn_set_err(err, err_len, "step staging failed");
        return -1;
    }
    if (finish(e, rc, err, err_len, true) != 0) return -1;
    if (e->has_nextn && e->guess_on) note_runs(e, R, seq, pos);
    if (n_out > 0) memcpy(out_tok, e->h_otok, (size_t) n_out * 4);
    e->last_n_out = n_out;
    e->last_pn = e->want_probs ? n_out : 0;
    if (e->want_probs) e->last_probs.assign(e->h_rec, e->h_rec + (size_t) n_out * 8);
    return 0;
}

// A write step that samples each row in order (sn_step.inc.h:137-142) can have the next one queued behind it; not
// while the guess head fills its cells (a dropped step would have moved the slots' kept head state) or profiling.
bool chain_shape(const sn_engine* e, int R, int n_write, int n_out, const int32_t* out_rows) {
    if ((e->has_nextn && e->guess_on) || e->prof_on || R != n_write || n_out != R || n_out > e->slots) return false;
    for (int j = 0; j < n_out; ++j)
        if (out_rows[j] != j) return false;
    return true;
}

// Queue the step after the one just enqueued (sn_step.inc.h:67-78): the same rows one position on, fed that step's
// outputs on the GPU, staged into the other buffer set and enqueued behind it, so it runs while the caller takes this
// step's tokens. Not when a row would pass the context or the cache is out of pages.
void queue_next(sn_engine* e, int R, const int32_t* seq, const int32_t* pos, int n_fast) {
    std::vector<int32_t> p1(R), rows(R);
    for (int r = 0; r < R; ++r) {
        p1[r] = pos[r] + 1;
        rows[r] = r;
        if (p1[r] >= e->ctx) return;
    }
    if (take_pages(e, R, seq, p1.data()) != 0) return;
    const int32_t* fed = e->d_otok;  // this step's tokens, on the device
    swap_sets(e);
    const int rc = enqueue_step(e, R, nullptr, fed, seq, p1.data(), R, rows.data());
    swap_sets(e);
    e->ch_on = true;
    e->ch_R = R;
    e->ch_fast = n_fast;
    e->ch_probs = e->want_probs;
    e->ch_cfg = e->cfg_gen;
    e->ch_seq.assign(seq, seq + R);
    e->ch_pos = p1;
    e->ch_tok.clear();  // known when this step's tokens are
    if (rc != 0) settle(e);  // nothing usable queued: let what was enqueued end, zero its cells
}

// whether the step asked for is the queued one (sn_step.inc.h:145-169): its rows, positions and tokens, and the same
// way of choosing tokens
bool queued_same(const sn_engine* e, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos, int n_fast,
                 bool shape) {
    if (!shape || R != e->ch_R || n_fast != e->ch_fast || e->want_probs != e->ch_probs || e->cfg_gen != e->ch_cfg ||
        (int) e->ch_tok.size() != R)
        return false;
    for (int r = 0; r < R; ++r)
        if (seq[r] != e->ch_seq[r] || pos[r] != e->ch_pos[r] || tok[r] != e->ch_tok[r]) return false;
    return true;
}

// The queued step is not the step asked for, or a cache call comes first (sn_step.inc.h:31-47): let it end and zero
// the cells it wrote in every layer (clear_cells, sn_cache.inc.h:252-262). Its pages stay, as the reference's do.
int settle(sn_engine* e) {
    if (!e->ch_on) return 0;
    e->ch_on = false;
    ++e->ch_dropped;
    const int pc = e->page_cells;
    for (int r = 0; r < e->ch_R; ++r) {
        const int p = e->seq_pages(e->ch_seq[r])[e->ch_pos[r] / pc];
        if (p >= 0)
            kv_page_op(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, pc, -1, p, e->ch_pos[r] % pc,
                       e->ch_pos[r] % pc + 1, e->st);
    }
    return hipStreamSynchronize(e->st) == hipSuccess ? 0 : -1;
}

}  // namespace

extern "C" int sn_step(sn_engine* e, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos, int n_write,
                       int n_fast, int n_out, const int32_t* out_rows, int32_t* out_tok, int chain, char* err,
                       int err_len) {
    if (step_shape_bad(e, R, n_write, n_fast, n_out)) {
        sn_set_err(err, err_len, "bad step shape");
        return -1;
    }
    if (rows_bad(e, R, tok, seq, pos)) {
        sn_set_err(err, err_len, "a row is out of range (slot, position or token)");
        return -1;
    }
    for (int j = 0; j < n_out; ++j)
        if (out_rows[j] < 0 || out_rows[j] >= R) {
            sn_set_err(err, err_len, "an output row is outside the step");
            return -1;
        }
    // (sn_step.inc.h:187-213) the step asked for may be the queued one, whether or not the caller chains on from it
    const bool shape = chain_shape(e, R, n_write, n_out, out_rows), next = chain && shape;
    int rc;
    if (e->ch_on && queued_same(e, R, tok, seq, pos, n_fast, shape)) {
        e->ch_on = false;
        ++e->ch_taken;
        swap_sets(e);  // its buffer set becomes the engine's
        rc = 0;
    } else {
        if (settle(e) != 0) {
            sn_set_err(err, err_len, "the queued step failed on the GPU");
            return -1;
        }
        if (take_pages(e, R, seq, pos) != 0) {
            sn_set_err(err, err_len, "out of cache pages");
            return -2;
        }
        rc = enqueue_step(e, R, tok, nullptr, seq, pos, n_out, out_rows);
    }
    if (next && rc == 0) queue_next(e, R, seq, pos, n_fast);
    const int trc = take_step(e, rc, R, seq, pos, n_out, out_tok, err, err_len);
    if (e->ch_on) {
        if (trc == 0) e->ch_tok.assign(out_tok, out_tok + R);  // the queued step was fed these
        else settle(e);
    }
    return trc;
}

// k guesses of one sequence (sn_guess, sn_cache.inc.h:357-388): k head rows, each fed the guess before it on the GPU
extern "C" int sn_guess(sn_engine* e, int seq, int32_t tok, int pos, int k, int32_t* out_tok, char* err, int err_len) {
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
    if (!e->has_nextn || !e->guess_on) {
        sn_set_err(err, err_len, "sn_guess: no guess head, or guessing is off (sn_guess_on)");
        return -1;
    }
    if (seq < 0 || seq >= e->slots || pos < 0 || k < 1 || k > 4 || pos + k > e->ctx || tok < 0 || tok >= e->V) {
        sn_set_err(err, err_len, "sn_guess: slot, position, token or count out of range");
        return -1;
    }
    std::vector<int32_t> sq(k, seq), ps(k);
    for (int j = 0; j < k; ++j) ps[j] = pos + j;
    if (take_pages(e, k, sq.data(), ps.data()) != 0) {
        sn_set_err(err, err_len, "out of cache pages");
        return -2;
    }
    Stage S{e};
    const size_t o_tok = S.put(&tok, 4), o_seq = S.put(&seq, 4), o_pos = S.put(ps);
    std::vector<AttnList> al;
    for (int j = 0; j < k; ++j) al.push_back(attn_list(e, S, 1, &seq, &ps[j]));
    e->prof_recs.clear();
    if (stage_copy(e, S) != 0) {
        sn_set_err(err, err_len, "sn_guess: staging failed");
        return -1;
    }
    Dev d{e, e->st};
    for (int j = 0; j < k && d.rc == 0; ++j)
        d.head_rows(1, j ? e->d_gtok + (j - 1) * e->slots : S.dev<const int32_t>(o_tok), S.dev<const int32_t>(o_seq),
                    S.dev<const int32_t>(o_pos) + j, j == 0, S, al[j], e->d_gtok + j * e->slots);
    for (int j = 0; j < k; ++j)
        SN_HIP_TRY(hipMemcpyAsync(e->h_otok + j, e->d_gtok + j * e->slots, 4, hipMemcpyDeviceToHost, e->st), -1);
    if (finish(e, d.rc, err, err_len) != 0) return -1;
    memcpy(out_tok, e->h_otok, (size_t) k * 4);
    return 0;
}

// The fused draft-verify step (sn_ext.h): drafts, verify rows, acceptance and the cut, in one submission.
extern "C" int snx_spec_step(sn_engine* e, int n, const int32_t* seq, const int32_t* last, const int32_t* pos, int k,
                             const uint8_t* force, int32_t* out_n, int32_t* out_tok, char* err, int err_len) {
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
    if (!e->has_nextn || !e->guess_on) {
        sn_set_err(err, err_len, "snx_spec_step: no guess head, or guessing is off (sn_guess_on)");
        return -1;
    }
    const int R = n * (k + 1);
    if (n < 1 || n > e->slots || k < 1 || k > 4 || R > e->max_rows || R > e->max_out) {
        sn_set_err(err, err_len, "snx_spec_step: bad sequence count or draft length");
        return -1;
    }
    std::vector<int32_t> vtok(R), vseq(R), vpos(R), rows(R), hpos((size_t) k * n);
    for (int s = 0; s < n; ++s) {
        if (seq[s] < 0 || seq[s] >= e->slots || pos[s] < 0 || pos[s] + k >= e->ctx || last[s] < 0 || last[s] >= e->V) {
            sn_set_err(err, err_len, "snx_spec_step: a sequence is out of range (slot, position or token)");
            return -1;
        }
        for (int t = 0; t < s; ++t)
            if (seq[t] == seq[s]) {
                sn_set_err(err, err_len, "snx_spec_step: a slot appears twice");
                return -1;
            }
        for (int i = 0; i <= k; ++i) {
            const int r = s * (k + 1) + i;
            vtok[r] = i == 0 ? last[s] : 0;  // the drafts are filled in on the GPU
            vseq[r] = seq[s];
            vpos[r] = pos[s] + i;
            rows[r] = r;
        }
        for (int j = 0; j < k; ++j) hpos[(size_t) j * n + s] = pos[s] + j;
    }
    if (take_pages(e, R, vseq.data(), vpos.data()) != 0) {
        sn_set_err(err, err_len, "out of cache pages");
        return -2;
    }
    Stage S{e};
    const size_t o_vtok = S.put(vtok), o_vseq = S.put(vseq), o_vpos = S.put(vpos), o_rows = S.put(rows);
    std::vector<uint8_t> skip(R + 1, 0), frc(R + 1, 0);
    for (int r = 0; r < R; ++r) skip[r] = e->no_end[vseq[r]];
    if (force)
        for (int s = 0; s < n; ++s)
            for (int i = 0; i < k; ++i) frc[s * (k + 1) + i] = force[s * k + i] != 0;
    const size_t o_skip = S.put(skip), o_force = S.put(frc);
    const size_t o_last = S.put(last, (size_t) n * 4), o_hseq = S.put(seq, (size_t) n * 4), o_hpos = S.put(hpos);
    std::vector<AttnList> hal;
    for (int j = 0; j < k; ++j) hal.push_back(attn_list(e, S, n, seq, &hpos[(size_t) j * n]));
    const AttnList al = attn_list(e, S, R, vseq.data(), vpos.data());
    std::vector<int32_t> src, keep;
    head_sources(e, R, vseq.data(), vpos.data(), src, keep);
    const size_t o_src = S.put(src);
    // device scratch in the staging buffer: draft checks, results, kept rows, accepted counts
    std::vector<int32_t> zeros((size_t) R + 2 * n + R + 2 * n + n, 0);
    const size_t o_ftok = S.put(zeros.data(), (size_t) R * 4), o_outn = S.put(zeros.data(), (size_t) n * 4),
                 o_outt = S.put(zeros.data(), (size_t) R * 4), o_keep = S.put(zeros.data(), (size_t) 2 * n * 4),
                 o_acc = S.put(zeros.data(), (size_t) n * 4);
    e->prof_recs.clear();
    if (stage_copy(e, S) != 0) {
        sn_set_err(err, err_len, "snx_spec_step: staging failed");
        return -1;
    }
    hipStream_t st = e->st;
    int32_t* d_vtok = S.dev<int32_t>(o_vtok);
    const int32_t* d_vseq = S.dev<const int32_t>(o_vseq);
    const int32_t* d_vpos = S.dev<const int32_t>(o_vpos);
    int32_t* d_ftok = S.dev<int32_t>(o_ftok);
    int32_t* d_outn = S.dev<int32_t>(o_outn);
    int32_t* d_outt = S.dev<int32_t>(o_outt);
    int32_t* d_keep = S.dev<int32_t>(o_keep);
    int32_t* d_acc = S.dev<int32_t>(o_acc);
    // the key of the device work: the step's shape, how tokens are chosen, every staging offset, every attention list
    std::vector<int64_t> key = {2, n, k, R, force != nullptr, e->want_probs, (int64_t) e->eog.size()};
    for (size_t o : {o_vtok, o_vseq, o_vpos, o_rows, o_skip, o_force, o_last, o_hseq, o_hpos, o_src, o_ftok, o_outn,
                     o_outt, o_keep, o_acc})
        key.push_back((int64_t) o);
    for (const AttnList& h : hal) h.key(key);
    al.key(key);
    const int drc = run_device(e, std::move(key), [&](Dev& d) {
        // drafts: k rounds of n head rows (one a sequence), each round fed the guesses before it
        for (int j = 0; j < k && d.rc == 0; ++j)
            d.head_rows(n, j ? e->d_gtok + (j - 1) * e->slots : S.dev<const int32_t>(o_last),
                        S.dev<const int32_t>(o_hseq), S.dev<const int32_t>(o_hpos) + (size_t) j * n, j == 0, S, hal[j],
                        e->d_gtok + j * e->slots);
        // verify rows [last, d1 .. dk] of every sequence through the model; the head's cells of those rows
        spec_rows(n, k, e->slots, e->d_gtok, d_vtok, d_ftok, d.st);
        d.model(R, d_vtok, d_vseq, d_vpos, S, al);
        if (d.rc == 0) d.head_fill(R, d_vtok, d_vseq, d_vpos, S.dev<const int32_t>(o_src), 0, nullptr);
        if (d.rc == 0)
            d.outputs(e->x, R, S.dev<const int32_t>(o_rows), S.dev<const uint8_t>(o_skip),
                      force ? S.dev<const uint8_t>(o_force) : nullptr, d_ftok);
        // acceptance, the refused rows' cells cut in every layer, the head's state at the last kept row
        accept_rows(n, k, e->slots, e->d_gtok, e->d_otok, d_vseq, d_outn, d_outt, d_keep, d_acc, d.st);
        cut_cells(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, e->page_cells, e->d_pt, e->max_pages, n, k,
                  d_vseq, d_vpos, d_acc, d.st);
        rows_keep(e->mhn, d_keep, n, e->E, e->mpend, d.st);
    });
    SN_HIP_TRY(hipMemcpyAsync(e->h_otok, d_outt, (size_t) R * 4, hipMemcpyDeviceToHost, st), -1);
    SN_HIP_TRY(hipMemcpyAsync(e->h_rec, d_outn, (size_t) n * 4, hipMemcpyDeviceToHost, st), -1);
    if (finish(e, drc, err, err_len) != 0) return -1;
    memcpy(out_tok, e->h_otok, (size_t) R * 4);
    memcpy(out_n, e->h_rec, (size_t) n * 4);
    for (int s = 0; s < n; ++s) {  // the run each sequence keeps (sn_clear's cut of the head state)
        e->run_row[seq[s]] = s * (k + 1);
        e->run_pos[seq[s]] = pos[s];
        e->run_n[seq[s]] = out_n[s];
    }
    e->last_n_out = 0;  // the verify rows' logits are not kept for sn_logits
    return 0;
}

extern "C" double sn_last_gpu_ms(const sn_engine* e) { return e->last_ms; }

extern "C" long snx_graph_count(const sn_engine* e, int replays) { return replays ? e->graph_replays : e->graph_captures; }

extern "C" long snx_chain_count(const sn_engine* e, int dropped) { return dropped ? e->ch_dropped : e->ch_taken; }

extern "C" void snx_graphs(sn_engine* e, int on);
extern "C" void snx_attn_mode(sn_engine* e, int mode) {
    e->attn_mode = mode < -1 || mode > 2 ? -1 : mode;
    snx_graphs(e, e->graphs);  // captured graphs hold the old form's launches
}

extern "C" int snx_fuse(sn_engine* e, int on) {
    e->fuse = on != 0 && e->fuse_ok;
    snx_graphs(e, e->graphs);  // captured graphs hold the other path's launches
    return e->fuse ? 1 : 0;
}

extern "C" int snx_xcd_faults(sn_engine* e) {
    if (settle(e) != 0) return -1;
    int32_t v = 0;
    if (hipStreamSynchronize(e->st) != hipSuccess || hipMemcpy(&v, e->d_xerr, 4, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return v;
}

extern "C" void snx_graphs(sn_engine* e, int on) {
    e->graphs = on != 0;
    for (auto& g : e->gcache) hipGraphExecDestroy(g.ex);
    e->gcache.clear();
}

extern "C" int snx_step_key(int H, int KVH, int page_cells, int mode, int R, const int32_t* seq, const int32_t* pos,
                            int64_t* key, int cap, int* whole) {
    if (H <= 0 || KVH <= 0 || H % KVH || 16 % (H / KVH) || (page_cells != 32 && page_cells != 64) || R <= 0 ||
        mode < -1 || mode > 2)
        return -1;
    int slots = 0, cells = 0;
    for (int r = 0; r < R; ++r) {
        if (seq[r] < 0 || pos[r] < 0) return -1;
        slots = std::max(slots, seq[r] + 1);
        cells = std::max(cells, pos[r] + 1);
    }
    sn_engine e;  // the fields the host half of a step reads; nothing on the device
    e.H = H, e.KVH = KVH, e.D = 128, e.QD = H * 128, e.KD = KVH * 128;
    e.page_cells = page_cells, e.attn_mode = mode, e.slots = slots, e.max_rows = R;
    e.max_chunks = (cells + ATT_CHUNK - 1) / ATT_CHUNK;
    e.no_end.assign(slots, 0);
    e.stage_bytes = (size_t) R * (64 + sizeof(AttnGroup) + (size_t) e.max_chunks * sizeof(AttnItem)) + 4096;
    std::vector<uint8_t> host(e.stage_bytes);
    e.h_stage = host.data();
    std::vector<int32_t> tok(R, 0), rows(R);
    for (int r = 0; r < R; ++r) rows[r] = r;
    Stage S{&e};
    StepStage ss;
    stage_step(&e, S, ss, R, tok.data(), seq, pos, R, rows.data());
    e.h_stage = nullptr;
    if (S.over) return -1;
    if (whole) *whole = ss.al.whole ? 1 : 0;
    for (int i = 0; i < (int) ss.key.size() && i < cap; ++i) key[i] = ss.key[i];
    return (int) ss.key.size();
}

extern "C" void snx_prof(sn_engine* e, int on) {
    settle(e);
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
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
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

extern "C" void sn_want_probs(sn_engine* e, int on) {
    if (e->want_probs != (on != 0)) ++e->cfg_gen;
    e->want_probs = on != 0;
}
extern "C" int sn_probs(sn_engine* e, int n_out, float* dst, char* err, int err_len) {
    if (n_out < 0 || n_out > e->last_pn) {
        sn_set_err(err, err_len, "the last step has no token probabilities for these rows");
        return -1;
    }
    memcpy(dst, e->last_probs.data(), (size_t) n_out * 32);
    return 0;
}

extern "C" int sn_set_eog(sn_engine* e, const int32_t* ids, int n) {
    if (n < 0 || n > 8 || n >= e->V) return -1;
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= e->V) return -1;
    if (settle(e) != 0) return -1;  // the queued step reads the ban list
    ++e->cfg_gen;
    e->eog.assign(ids, ids + n);
    if (n > 0 && hipMemcpy(e->d_ban, ids, (size_t) n * 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
    return 0;
}
extern "C" void sn_no_end(sn_engine* e, int slot, int on) {
    if (slot >= 0 && slot < e->slots && e->no_end[slot] != (on != 0)) {
        e->no_end[slot] = on != 0;
        ++e->cfg_gen;
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// cache calls (sn_seq.inc.h)

extern "C" int sn_copy(sn_engine* e, int from, int to, int n, char* err, int err_len) {
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
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
        if (tf[c] >= 0) kv_page_op(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, pc, tf[c], np, 0, n % pc, e->st);
    }
    e->pt_dirty = true;
    SN_HIP_TRY(hipStreamSynchronize(e->st), -1);
    return 0;
}

extern "C" int sn_clear(sn_engine* e, int slot, int from, int to, char* err, int err_len) {
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
    if (!slot_ok(e, slot, from, to)) {
        sn_set_err(err, err_len, "sn_clear: bad slot or cells");
        return -1;
    }
    const int pc = e->page_cells;
    int32_t* t = e->seq_pages(slot);
    if (e->has_nextn && e->guess_on) {
        // the guess head's state of the slot: the hidden state of its last kept cell when the last step's run holds
        // it (sn_seq.inc.h:72), none at 0
        const size_t EB = (size_t) e->E * 4;
        if (from == 0) {
            SN_HIP_TRY(hipMemsetAsync(e->mpend + (size_t) slot * e->E, 0, EB, e->st), -1);
        } else if (e->run_row[slot] >= 0 && from - 1 >= e->run_pos[slot] && from - 1 < e->run_pos[slot] + e->run_n[slot]) {
            const int row = e->run_row[slot] + (from - 1 - e->run_pos[slot]);
            SN_HIP_TRY(hipMemcpyAsync(e->mpend + (size_t) slot * e->E, e->mhn + (size_t) row * e->E, EB,
                                      hipMemcpyDeviceToDevice, e->st), -1);
        }
    }
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
            kv_page_op(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, pc, p, np, 0, from % pc, e->st);
        } else {
            kv_page_op(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, pc, -1, p, from % pc,
                       std::min(pc, to - c * pc), e->st);
        }
    }
    SN_HIP_TRY(hipStreamSynchronize(e->st), -1);
    return 0;
}

extern "C" size_t sn_kv_bytes(const sn_engine* e, int n) { return (size_t) e->CL * 2 * n * e->KD * 2; }

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
    kv_stage(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, e->page_cells, dp, n, stg, save, e->st);
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
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
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
    kv_fill_normal(e->kbase, e->vbase, e->layer_halves, e->CL, e->KVH, e->page_cells, dp, n,
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
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
    return kv_xfer(e, slot, n, dst, 1, err, err_len);
}
extern "C" int sn_kv_load(sn_engine* e, int slot, int n, const void* src, char* err, int err_len) {
    if (settle(e) != 0) return -1;  // a cache call drops the queued step first (sn.h:36-38)
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
extern "C" size_t sn_page_bytes(const sn_engine* e) { return (size_t) e->page_cells * e->KD * 2 * 2 * e->CL; }
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
// the most cells of the slot's first n it can be cut back to (sn_cache.inc.h:448-452): n when sn_cut_ok takes it (no
// recurrent state here), 0 for a bad slot or n <= 0
extern "C" int sn_cut_best(const sn_engine* e, int slot, int n) {
    if (!e || slot < 0 || slot >= e->slots || n <= 0) return 0;
    return sn_cut_ok(e, slot, n) ? n : 0;
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

// the guess head (sn_cache.inc.h:288-298): there when the GGUF carries a nextn block the engine loaded
extern "C" int sn_guess_head(const sn_engine* e) { return e->has_nextn ? 1 : 0; }
extern "C" int sn_guess_on(sn_engine* e, int on) {
    if (!e->has_nextn) return 0;
    settle(e);
    e->guess_on = on != 0;
    return e->guess_on;
}
