// Kernel launchers shared by the engine (engine.cpp) and the kernel-level C ABI (snk.cpp). Host-side only.
#pragma once
#include "sn_common.h"

#include <vector>

enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

struct GemmArgs {
    const uint8_t* w;
    const uint8_t* xa;
    float* y;
    float* part;  // k-slice partial sums [ks][M][N]
    // grouped (experts): z-block i runs item (expert, row tile) items[2i], items[2i + 1] for i < *count, its weights at
    // w + expert * wstride; one slice, one row tile a workgroup
    const int32_t* items;
    const int32_t* count;
    size_t wstride;
    const int32_t* rmask;  // (optional) rows p with rmask[p] < 0 are not stored
    // (optional, grouped) the activation gathered: tile row p is row gsrc[p] (< 0: zeros) of a row-ordered operand of
    // gM rows, instead of row p of a tile-ordered one
    const int32_t* gsrc;
    int gM;
    // (prompt gate|up, q4_gemm_swiglu) SwiGLU of the sums as fp32 rows h [M][N / 2] and as the Q8_0 operand xo
    float* h;
    uint8_t* xo;
    int M, N, K, ldy, epi;
    int nstripes, ngroups, ks, gps, mtiles;
    // The streaming kernel's fused epilogues (decode rows, q4_gemm_fused): a workgroup that has stored its slice's sums
    // counts itself in cnt[set + gridDim.x * z] (zero between launches), and the set's last one adds the set's slices in
    // slice order and applies the epilogue itself. The hardware deals a launch's workgroups to the device's nxcd XCDs
    // in turn by linear id (from where the queue's last launch left off), and the grid's sets are padded to a multiple
    // of nxcd, so every workgroup of a set runs on one XCD and the sums reach the last one through that XCD's L2. Each
    // workgroup also adds 1 to its XCD's 5-bit field of the 64-bit count: a last workgroup that finds the count's
    // workgroups on more than one XCD sets *xerr (its epilogue may have read stale sums).
    uint64_t* cnt;
    int32_t* xerr;
    int nxcd;
    // FE_ROPE: the rows' q|k|v heads normed, rotated, and k, v written to their cells (qk_norm_rope_kv's arguments)
    float* qkv;
    int ldqkv;
    const float *qw, *kw;
    float eps, theta_scale;
    const int32_t *seq, *pos, *pt;
    int max_pages, page_cells;
    uint16_t *kpool, *vpool;
    int H, KVH;
    const float2* rope_cs;  // the rows' rotation table (rope_table), or null (each head forms its angles)
};
// the streaming kernel's fused epilogues: none (the k-slice sums for the row kernels), the SwiGLU + Q8_0 of a
// stripe-interleaved gate|up matrix (k_swiglu_quant's arithmetic), the q|k|v heads' QK-norm + RoPE + cache write
// (k_qk_rope's arithmetic)
// (the kernel's instances: FE + i, i = 0..7, whose KM = fe_slice_bound(i) bounds the slices the epilogue loads)
enum { FE_NONE = 0, FE_SWIGLU = 8, FE_ROPE = 16, FE_GSWIGLU = 32 };  // (FE_GSWIGLU: grouped, one slice; no counters)
// the epilogue instances' slice bounds (the exact counts of the common plans: 3 gate|up, 5 q|k|v at K = 2560, 10 ...)
__host__ __device__ constexpr int fe_slice_bound(int i) {
    return i == 0 ? 1 : i == 1 ? 2 : i == 2 ? 3 : i == 3 ? 4 : i == 4 ? 5 : i == 5 ? 8 : i == 6 ? 10 : 16;
}
// the index of the least bound that holds ks slices (1 <= ks <= 16)
static inline int fe_slice_index(int ks) {
    int i = 0;
    while (i < 7 && fe_slice_bound(i) < ks) ++i;
    return i;
}

// Launch shape of one matrix: a workgroup owns 4 spw stripes (a "set": spw per wavefront) and gps consecutive 4-block
// groups (a slice). Layer-sized matrices at decode row counts run the streaming kernel (sspw stripes a wavefront,
// smt row tiles a workgroup); LM-head-wide matrices and prompt-sized row counts the ring kernel (spw, sets). The
// slices are the same for both, so a row's sums do not depend on the kernel.
struct GemmPlan {
    int nstripes, ngroups, spw, sets, ks, gps;
    bool stream;    // the streaming kernel serves this matrix below Q4_PAIR_ROWS rows
    int sspw, smt;  // its stripes a wavefront and row tiles a workgroup
    int sd;         // its ring depth (groups of weights in flight a wavefront)
};

// Depends on (N, K) only, never on the rows.
GemmPlan q4_plan(int N, int K, int wt = WT_Q4_0);
// the raw matmul with an explicit plan (tuning): mt row tiles a workgroup, spw stripes a wavefront, G groups a slice
// loaded at once (G 0: the default plan); the slice count, or -1
// part[ks][M][N] added in slice order into y [M][N]
// The prompt rows' gate|up matmul with its SwiGLU: from Q4_PAIR_ROWS rows, a Q4_0 stripe-interleaved matrix of
// N = 2F (F a multiple of 128) walked whole (k_q4_gemm_w2, FK) with silu(gate) * up written as fp32 rows h [M][F] and
// as the Q8_0 operand xo (K = F), the same bits as the matmul's slices through k_swiglu_quant. xo must not be xa.
// Returns 1, or 0 when the shape does not qualify (nothing launched: use the matmul and swiglu_quant).
int q4_gemm_swiglu(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* h, uint8_t* xo, hipStream_t st,
                   int wt);
bool q4_gemm_swiglu_fits(int M, int N, int K, int wt);  // whether q4_gemm_swiglu takes this shape
void q4_reduce_slices(const float* part, int ks, int M, int N, float* y, hipStream_t st);
int q4_gemm_raw_plan(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                     hipStream_t st, int wt, int mt, int spw, int G);
// The k-slice sums of a matmul of M rows: ks * M * N floats.
size_t q4_workspace_bytes(int M, int N, int K, int wt = WT_Q4_0);
// Raw matmul: part[slice][M][N] = the slice's sums (the consumer adds the slices in order). Returns the slice count,
// or -1 when part_bytes is too small. wt: the weight type of w (WT_Q4_0 or WT_Q8_0 tiles).
int q4_gemm_raw(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                hipStream_t st, int wt = WT_Q4_0);
// The raw matmul of decode-sized rows with a fused epilogue fe (FE_SWIGLU: a.h, a.xo; FE_ROPE: the rope fields of a)
// through the streaming kernel: the same sums in the same order as q4_gemm_raw followed by swiglu_quant (xo must not be
// xa) or qk_norm_rope_kv, so the same bits. `a` carries the epilogue's fields and the counters (a.cnt, cnt_len of
// them, a set's every CNT_STRIDE), a.xerr and a.nxcd. Returns 1 when launched, 0 when the shape or weight type has no fused launch
// (nothing launched: use the split path), -1 on bad arguments.
int q4_gemm_fused(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                  hipStream_t st, int wt, int fe, const GemmArgs& a, int cnt_len);
// whether q4_gemm_fused launches this shape (host only)
bool q4_gemm_fused_fits(int M, int N, int K, int wt, int fe, int nxcd, int cnt_len);
// Whether the current device deals a launch's workgroups to its XCDs in turn by linear id: a probe launch on `st`
// (synchronous) of 8192 workgroups, each recording its XCD id; true when workgroups i and i mod nxcd ran on the same
// XCD for every i, with nxcd the number of XCD ids seen (at most 8). The condition of the fused epilogues.
bool xcd_round_robin(hipStream_t st, int* nxcd);
// Grouped raw matmul of expert matrices (moe: qmm_grouped, sn_attn.inc.h:352-359): up to max_items (expert, row tile)
// items, the device count in `count`; part[M][N] rows of each item's tile (one slice).
// gsrc (optional): the operand's tile row p is row gsrc[p] of the row-ordered operand xa of gM rows (gathered while
// loading; gsrc[p] < 0 reads zeros), as if the rows had been quantized into expert-tile order.
// The grouped gate|up matmul (q4_gemm_grouped's arguments, N = 2F interleaved as swiglu_quant reads it) with SwiGLU +
// Q8_0 of its rows into the operand xo [M][F] (rows with rmask < 0 not written), in one launch: the same bits as
// q4_gemm_grouped followed by swiglu_quant(ks 1). 1 when launched, 0 when the shape has no such launch (Q4_0, K of at
// most 16 groups, F a multiple of 128; nothing launched), -1 on bad arguments.
bool q4_gemm_grouped_swiglu_fits(int N, int K, int wt);
int q4_gemm_grouped_swiglu(const uint8_t* w, size_t wstride, const int32_t* items, const int32_t* count, int max_items,
                           const uint8_t* xa, int M, int N, int K, uint8_t* xo, hipStream_t st, int wt,
                           const int32_t* rmask, const int32_t* gsrc, int gM);
int q4_gemm_grouped(const uint8_t* w, size_t wstride, const int32_t* items, const int32_t* count, int max_items,
                    const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes, hipStream_t st,
                    int wt = WT_Q4_0, const int32_t* rmask = nullptr, const int32_t* gsrc = nullptr, int gM = 0);
// one plain streaming read of `bytes` (a multiple of 16) from buf (a calibration launch; sink: 1 KB, never written
// in practice)
void read_floor(const void* buf, size_t bytes, float* sink, hipStream_t st);
// GGUF Q4_0 (wt = WT_Q4_0) or Q8_0 (WT_Q8_0) rows -> tiles; source stripe s lands at destination stripe
// s * sstride + soff.
void q4_repack(const uint8_t* src, int N, int K, uint8_t* dst, int sstride, int soff, hipStream_t st,
               int wt = WT_Q4_0);
// rows (optional): row m of the operand is row rows[m] of x (rows[m] < 0: a zero row). nw (optional): RMSNorm weight
// applied first.
// xn (optional): the normed fp32 rows, ldn apart.
void quant_act(const float* x, const int32_t* rows, int M, int K, int ldx, const float* nw, float eps, uint8_t* xa,
               float* xn, int ldn, hipStream_t st);
// Raw matmul into the workspace, then the slices added in order with an epilogue into y (ldy apart): store, add, or
// SwiGLU of the stripe-interleaved gate/up pair (output column 16p + n = silu(column 32p + n) * column 32p + 16 + n).
// x[m] += the k-slice sums part[ks][M][K] (added in slice order; add false: x[m] = the sums); then, with xa, the Q8_0
// operand of the new rows (RMS-normed by nw when given). K <= 8192. 0, or -1 (shape).
// next_w (optional): the next matmul's N x K matrix (weight type wt), whose first weight groups extra workgroups read
// into the Infinity Cache meanwhile (decode-sized rows).
int resid_quant(float* x, const float* part, int ks, int M, int K, const float* nw, float eps, uint8_t* xa,
                hipStream_t st, bool add = true, float* xn = nullptr, const uint8_t* next_w = nullptr, int next_N = 0,
                int next_K = 0, int wt = 2);
// h (optional) and the Q8_0 operand of silu(gate) * up from a stripe-interleaved gate/up matmul's k-slice sums
// part[ks][M][2F]. 0, or -1 (more than KS_MAX slices, F not a multiple of 32: nothing launched).
int swiglu_quant(const float* part, int ks, int M, int F, float* h, uint8_t* xa, hipStream_t st,
                  const int32_t* rows = nullptr);
int q4_gemm(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* y, int ldy, int epi, float* ws,
            size_t ws_bytes, hipStream_t st, int wt = WT_Q4_0);

// ---- Q6_K weights (csrc/q6k.hip) ----
// GGUF Q6_K rows [N][K / 256 x 210 bytes] -> tiles (K % 256 == 0); the tiles back to fp32 [N][K] (bit-exact check)
void q6k_repack(const uint8_t* src, int N, int K, uint8_t* dst, hipStream_t st);
void q6k_dequant(const uint8_t* tiles, int N, int K, float* out, hipStream_t st);
// rows of X (source rows[m] when given; ldx floats apart), RMS-normed by nw when given, into Q8_K records (xk_bytes)
void quant_q8k(const float* x, const int32_t* rows, int M, int K, int ldx, const float* nw, float eps, uint8_t* xk,
               hipStream_t st);
// y[m][n] (ldy apart) = the rows of xk . the tiles' rows (ggml vec_dot_q6_K_q8_K); 0, or -1 (K % 256)
int q6k_gemm(const uint8_t* tiles, const uint8_t* xk, int M, int N, int K, float* y, int ldy, hipStream_t st);

// ---- paged attention ----
// One work item = (query group, KV head, chunk of ATT_CHUNK cells). A query group is up to 16/G rows of one
// sequence (G = H/KVH query heads per KV head); its rows' positions rise by one (draft rows, prompt rows).
#define ATT_CHUNK 256
struct AttnGroup {
    int32_t row0;   // first row of the group (rows row0 .. row0 + nrows - 1)
    int32_t nrows;  // 1 .. 16/G
    int32_t seq;    // the sequence (page-table row)
    int32_t pos0;   // position of the first row; row i is at pos0 + i and attends cells 0 .. pos0 + i
};
#define ATT_SHARE_MAX 4  // groups a shared-chunk item serves
struct AttnItem {
    int32_t group;   // index into the group list
    int32_t chunk;   // cells chunk*ATT_CHUNK ..
    int32_t nchunk;  // chunks the item covers (whole-group items: all of the group's; otherwise 1)
    // a shared-chunk item (chunk items only): more groups of one row each whose chunk `chunk` lies wholly below their
    // positions on the very pages of `group`'s: their queries take the MFMA columns after `group`'s (-1: none), so the
    // chunk's K/V cells are read once for all of them
    int32_t share[ATT_SHARE_MAX - 1];
    // a run item (k_attn_run): groups group .. group + nmem - 1, consecutive groups of one sequence at consecutive
    // positions (prompt rows), walked together over the last one's nchunk chunks; 1 for every other item
    int32_t nmem;
    // a copy of groups[group] (attn_plan fills it), so that a chunk or whole-group workgroup's first loads need no
    // load of its group
    AttnGroup g;
};
#define ATT_RUN_MAX 4       // groups a run item holds (their queries staged in LDS, K/V cells read once for all)
#define ATT_RUN_MIN_WG 128  // run items are used when they make at least this many workgroups (items x KV heads)
struct AttnArgs {
    const float* q;          // [rows][H][D] fp32 (normed, roped; the softmax scale is applied inside)
    int ldq;                 // floats between rows of q
    const uint16_t* kpool;   // fp16 cells: page p, kv head h: kpool + ((p * KVH + h) * page_cells) * D (kcell_at)
    const uint16_t* vpool;
    const int32_t* pt;       // [n_seq][max_pages] page table
    int max_pages;
    int page_cells;          // 32 or 64
    const AttnGroup* groups;
    const AttnItem* items;
    int n_items;
    const AttnItem* runs;    // run items (k_attn_run: outputs written directly, no partials), n_runs of them
    int n_runs;
    float* part;             // partials [rows][H][max_chunks][130]: acc[128], m, l
    int max_chunks;
    float* out;              // [rows][ldo] fp32 (merge output), or NULL
    int ldo;
    uint8_t* xa;             // merge output also as the o-projection's xa operand (K = H*D), or NULL
    int H, KVH;
    float scale;
    int n_rows;
    const int32_t* row_pos;  // [rows] position of each row (merge: its chunk count)
    int whole;               // items are whole groups: one kernel writes the outputs, no partials, no merge
    const int32_t* mrows;    // rows the merge folds (chunk items), n_mrows of them
    int n_mrows;
    // (optional) fold: the chunk items and their merge in one launch (k_attn_fold: plain chunk items only, every group's
    // chunks 0 .. nc - 1; the items array is not read). n_groups groups, fold_chunks = the most chunks of a group
    // (<= 127); cnt: n_groups * KVH counters CNT_STRIDE apart, zero between launches; *xerr set when a (group, KV
    // head)'s workgroups ran on two XCDs; nxcd: the XCDs the launch is dealt to in turn (xcd_round_robin).
    int fold, n_groups, fold_chunks, nxcd;
    uint64_t* cnt;
    int32_t* xerr;
};
int paged_attention(const AttnArgs& a, hipStream_t st);  // attention_runs, attention_items, then attention_merge
int attention_runs(const AttnArgs& a, hipStream_t st);   // the run items (nothing without)
int attention_items(const AttnArgs& a, hipStream_t st);  // the partials (chunk items) or whole groups
int attention_merge(const AttnArgs& a, hipStream_t st);  // chunk items: the merge (nothing for whole groups)
// The work list of R rows: consecutive rows of one sequence at consecutive positions share a group (up to 16/G rows:
// their K/V loads are shared). Whole groups (one item each, walked by one workgroup per KV head) when the groups give
// one round of ATT_WHOLE_MIN_WG .. ATT_WHOLE_MAX_WG workgroups, the longest context is at most 9/8 of the mean and the
// contexts are long; otherwise one item per (group, 256-cell chunk), every row merged. Both fold a row's chunk
// partials in the same order with the same arithmetic, so a row's output does not depend on which list it was in.
// Prompt rows: a sequence's consecutive full groups at consecutive positions become run items of up to ATT_RUN_MAX
// groups (one workgroup per (run item, KV head) walks the last group's context once for all of them, folding each
// group's chunk partials in chunk order as the whole-group kernel does) when the run items make at least
// ATT_RUN_MIN_WG workgroups; the other groups follow the rule above.
#define ATT_WHOLE_MIN_WG 240
#define ATT_WHOLE_MAX_WG 256
struct AttnPlan {
    std::vector<AttnGroup> groups;
    std::vector<AttnItem> items;
    std::vector<AttnItem> runs;
    std::vector<int32_t> mrows;
    int max_chunk = 0;  // the most chunks of any group
    bool whole = false;
};
// mode: -1 as above, 0 per-chunk items, 1 whole groups (0 and 1: no run items), 2 run items wherever a sequence has
// two or more such groups, the other groups as -1. pt (optional, host [slots][max_pages]): the page table, from
// which chunk items of one-row groups whose chunk is wholly below their positions on the same pages become shared
// items (a chunk's partial is computed alike in either kind, so a row's output does not depend on the sharing).
void attn_plan(int R, const int32_t* seq, const int32_t* pos, int H, int KVH, int page_cells, AttnPlan& p,
               int mode = -1, const int32_t* pt = nullptr, int max_pages = 0);

// ---- elementwise / row kernels ----
// (a token id outside [0, V) gives a zero row)
void embed_rows(const float* table, int V, int E, const int32_t* tok, int R, float* x, hipStream_t st);
// q|k|v rows: from qkv (part NULL) or from the q|k|v matmul's k-slice sums part[ks][R][(H + 2 KVH) 128], which are
// then also written to qkv (k and v as summed, q after QK-norm and RoPE); k and v go to the rows' cache cells.
// cs (optional): the rows' rotation table (rope_table of the same positions), else each head forms its angles.
// 0, or -1 (more than KS_MAX slices: nothing launched).
int qk_norm_rope_kv(float* qkv, int ldqkv, const float* part, int ks, int R, int H, int KVH, const float* qw,
                    const float* kw, float eps, float theta_scale, const int32_t* seq, const int32_t* pos,
                    const int32_t* pt, int max_pages, int page_cells, uint16_t* kpool, uint16_t* vpool,
                    hipStream_t st, const float2* cs = nullptr);
// the rotation's (cos, sin) of R rows at positions pos (device), 64 lanes each, into cs [R][64]: the values each head's
// QK-RoPE would form itself (rope_cs), formed once for all of a step's heads and layers
void rope_table(const int32_t* pos, int R, float theta_scale, float2* cs, hipStream_t st);
// cells [a, b) of page `dst` in every layer: copied from page `src` (src >= 0) or zeroed (src < 0)
void kv_page_op(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells, int src, int dst,
                int a, int b, hipStream_t st);
// cells [0, n) of a slot (page list on the device) between the pool and a cell-major staging buffer
// [L][K, V][n][KVH][128] (save: pool -> staging; load: staging -> pool)
void kv_stage(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells,
              const int32_t* pages, int n, uint16_t* staging, int save, hipStream_t st);
// seeded N(0, 1) fp16 into cells [0, n) of a slot (page list on the device), every layer, K and V
void kv_fill_normal(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells,
                    const int32_t* pages, int n, uint64_t seed, hipStream_t st);
// greedy argmax of n rows of V scores (first index of the largest; rows with skip[r] never take the nban <= 8 ids in
// ban), with the optional 8-word probability records; ws: argmax_workspace_bytes(n, V) bytes of partials. -1: bad
// arguments or workspace too small (nothing launched).
#define AMX_CHUNK 4096
static inline int argmax_chunks(int V) { return (V + AMX_CHUNK - 1) / AMX_CHUNK; }
size_t argmax_workspace_bytes(int n, int V);
int argmax_rows(const float* logits, int V, int n, const int32_t* ban, int nban, const uint8_t* skip, int32_t* out,
                float* rec, void* ws, size_t ws_bytes, hipStream_t st);

// ---- the guess head (MTP) and the fused draft-verify step
// [enorm(embed(tok)); hnorm(h)] rows into cat [R][2E]; h: src NULL: hrows row r (hrows given) or pend[seq[r]];
// src[r] >= 0: hrows row src[r], -1: pend[seq[r]], -2: zeros
void mtp_cat(const float* table, int V, int E, const int32_t* tok, const float* hrows, const float* pend,
             const int32_t* src, const int32_t* seq, const float* enorm, const float* hnorm, float eps, float* cat,
             int R, hipStream_t st);
// keep [n][2] = (slot, row): dst[slot] = src[row] (E floats); slot < 0 skips
void rows_keep(const float* src, const int32_t* keep, int n, int E, float* dst, hipStream_t st);
// verify rows of n sequences x (k + 1) from the drafts gtok [k][slots]: vtok rows i > 0, ftok (row i < k: draft i)
void spec_rows(int n, int k, int slots, const int32_t* gtok, int32_t* vtok, int32_t* ftok, hipStream_t st);
void force_rows(float* logits, int V, int R, const uint8_t* force, const int32_t* ftok, hipStream_t st);
void accept_rows(int n, int k, int slots, const int32_t* gtok, const int32_t* otok, const int32_t* seq, int32_t* out_n,
                 int32_t* out_tok, int32_t* keep, int32_t* acc, hipStream_t st);
void cut_cells(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int CL, int KVH, int page_cells, const int32_t* pt,
               int max_pages, int n, int k, const int32_t* seq, const int32_t* pos, const int32_t* acc, hipStream_t st);

// ---- mixture of experts
// router logits lg [R][NE] (fp32) of the normed rows hn [R][E]
void moe_router(const float* hn, const float* router, int R, int E, int NE, float* lg, hipStream_t st);
// each row's k experts ids [R][k] and weights w [R][k] from lg, then the pairs in expert-major 16-row tiles: prow
// [R][k], rsrc [P] (-1 padding), items [2 x tiles] (expert, tile), count. NE <= 256, k <= 8, R * k <= 4096, P at least
// 16 (min(NE, R k) + ceil(R k / 16)); -1 otherwise (nothing launched).
int moe_select(const float* lg, int R, int NE, int k, int P, int32_t* ids, float* w, int32_t* prow, int32_t* rsrc,
               int32_t* items, int32_t* count, hipStream_t st);
// moe_router + moe_select in one launch, the same results: the row blocks' logits, then each block's routing by the
// block's last workgroup (an XCD-local handoff: the launch's workgroups are dealt to nxcd XCDs in turn), then the
// grouping by the last block (a system-coherent handoff). cnt: cnt_len 64-bit counters (a row block's every
// CNT_STRIDE), gcnt one, both zero between
// launches; *xerr set when a row block's workgroups ran on more than one XCD. E <= MOE_ROUTE_EMAX; -1 otherwise
// (nothing launched).
int moe_route(const float* hn, const float* router, int R, int E, int NE, int k, int P, float* lg, int32_t* ids,
              float* w, int32_t* prow, int32_t* rsrc, int32_t* items, int32_t* count, uint64_t* cnt, int cnt_len,
              int32_t* gcnt, int32_t* xerr, int nxcd, hipStream_t st);
// x[r] += sum_j w[r][j] y[prow[r][j]] (slot order)
// x[r] += the MoE output of row r (sum over its k slots, in slot order, of w[r][j] * y[prow[r][j]]: y the grouped down
// matmul's rows) and then, when xa is given, the RMSNorm (nw) + Q8_0 operand of the new rows, in one launch (one
// workgroup a row, the arithmetic of resid_quant); 0, or -1 (bad shape)
int moe_resid_quant(float* x, const float* y, const int32_t* prow, const float* w, int k, int M, int K, const float* nw,
                    float eps, uint8_t* xa, hipStream_t st);
