// sn_kernels.h — kernel-level C ABI of libsn_hip.so: the hot kernels of sn_step on caller-owned device memory, for
// the single-matmul and single-attention configurations, parity tests and roofline timing. Pointers prefixed d_ are
// device pointers; `stream` is a hipStream_t (NULL: the default stream). All calls are asynchronous on `stream`
// unless stated. Each entry names the reference kernel it stands for.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- Q4_0 x Q8_0 matmul: Y[m][n] (+)= sum_k X[m][k] W[n][k] ----------------------------------------------------------
// Replaces the Q4_0 mat-vec / few-row / block matmuls dispatched by mm() (core_mm.inc.h:307-325; kernels.metal:1324-1411,
// :1413-1490, :746-1007) with ggml CPU numerics (Q8_0 activations, integer block sums).
enum { SNK_EPI_STORE = 0, SNK_EPI_ADD = 1, SNK_EPI_SWIGLU = 2 };

// bytes of a matrix of N rows x K (K % 32 == 0) in the stripe layout; GGUF Q4_0 rows -> stripes
size_t snk_q4_stripes_bytes(int N, int K);
int snk_q4_repack(const void* d_q4, int N, int K, void* d_stripes, void* stream);
// the stripes dequantized back to fp32 [N][K] with the matmul's own unpack (d * (q - 8)): for the bit-exactness check
// against ggml's dequantize_row_q4_0
int snk_q4_dequant(const void* d_stripes, int N, int K, float* d_w, void* stream);
// Q8_0 weights (block_q8_0: fp16 d + 32 int8, w = d*q; the reference's mv_q8_0* kernels, kernels.metal:1995-2130,
// and its Q8_0 cv_ks dequant, :597-609), with ggml's CPU numerics (vec_dot_q8_0_q8_0: Q8_0 activations, integer block
// sums): bytes of the tile layout, GGUF Q8_0 rows -> tiles, the tiles dequantized back with the matmul's own unpack
// (d * q, for the bit-exactness check against ggml's dequantize_row_q8_0), and the matmul (arguments as snk_q4_gemm).
size_t snk_q8_tiles_bytes(int N, int K);
int snk_q8_repack(const void* d_q8, int N, int K, void* d_tiles, void* stream);
int snk_q8_dequant(const void* d_tiles, int N, int K, float* d_w, void* stream);
size_t snk_q8_workspace_bytes(int M, int N, int K);
int snk_q8_gemm(const void* d_tiles, const void* d_xa, int M, int N, int K, float* d_y, int ldy, int epi, void* d_ws,
                size_t ws_bytes, void* stream);

// Q6_K weights (block_q6_K: ql[128], qh[64], int8 scales[16], fp16 d per 256 weights; the reference reads them for the
// token table and the LM head, sn_load.inc.h:341-359, kernels.metal:1010-1120), with ggml's CPU numerics
// (vec_dot_q6_K_q8_K: Q8_K activations, integer sums per 16-weight group times its scale): bytes of the tile layout,
// GGUF rows -> tiles (K % 256 == 0), the tiles dequantized back with the matmul's own unpack ((d * scale) * (q - 32),
// for the bit-exactness check against dequantize_row_q6_K), the Q8_K activation records (quantize_row_q8_K_ref; RMS-
// normed by d_norm_w first when not NULL), and the matmul y[m][n] (ldy apart, no workspace). 0, or -1 (bad shape).
size_t snk_q6k_tiles_bytes(int N, int K);
int snk_q6k_repack(const void* d_q6k, int N, int K, void* d_tiles, void* stream);
int snk_q6k_dequant(const void* d_tiles, int N, int K, float* d_w, void* stream);
size_t snk_xk_bytes(int M, int K);
int snk_quant_q8k(const float* d_x, int M, int K, int ldx, const float* d_norm_w, float eps, void* d_xk, void* stream);
int snk_q6k_gemm(const void* d_tiles, const void* d_xk, int M, int N, int K, float* d_y, int ldy, void* stream);

// activation operand: M fp32 rows (ldx apart) quantized to Q8_0 (ggml x86 quantize_row_q8_0), RMS-normed by d_norm_w
// first when it is not NULL (the rmsnorm of kernels.metal:121-140 fused in front)
size_t snk_xa_bytes(int M, int K);
int snk_quant_act(const float* d_x, int M, int K, int ldx, const float* d_norm_w, float eps, void* d_xa, void* stream);
// the matmul; epi: store, add into d_y, or SwiGLU over interleaved gate/up stripe pairs (N = 2F, output F columns).
// d_ws: k-slice partial sums of snk_q4_workspace_bytes(M, N, K) bytes (may be 0). 0, or -1 (workspace too small).
size_t snk_q4_workspace_bytes(int M, int N, int K);
// the launch plan of an N x K matrix of weight type wt (2 Q4_0, 8 Q8_0), which depends on (N, K, wt) alone: 16-row
// stripes per wavefront (*spw: 2 for Q4_0 matrices of LM-head width, at least 6144 stripes; else 1) and k-slices
// (*ks). 0, or -1 (bad shape or type).
int snk_q4_plan(int N, int K, int wt, int* spw, int* ks);
int snk_q4_gemm(const void* d_stripes, const void* d_xa, int M, int N, int K, float* d_y, int ldy, int epi, void* d_ws,
                size_t ws_bytes, void* stream);
// Prompt rows (M >= 256) of a stripe-interleaved gate|up matrix (N = 2F, F a multiple of 128, the wide split plans)
// with its SwiGLU as the epilogue: silu(gate) * up as fp32 rows d_h [M][F] and as the Q8_0 operand d_xo (K = F, not
// d_xa), the same bits as snk_q4_gemm's SwiGLU epilogue and snk_quant_act of its rows (the prompt step's fused
// up-projection epilogue, qmm_epi flag 4, kernels.metal:566-568, with the next block matmul's input written directly
// as its flag 32 does). 0, 1 when the shape does not take it (nothing launched), or -1
int snk_q4_gemm_swiglu(const void* d_stripes, const void* d_xa, int M, int N, int K, float* d_h, void* d_xo,
                       void* stream);
// snk_q4_gemm without a workspace and without allocating: the k-slice partial sums go to a fixed device array of
// 32 MiB that the library holds on each GPU it runs on (until the process ends), so the call makes no hipMalloc,
// hipFree or other allocating call. The same kernels as snk_q4_gemm, so the same bits. A shape whose partials
// (snk_q4_workspace_bytes(M, N, K)) exceed 32 MiB is refused with the reason in err. Calls that overlap on one GPU
// (other streams or threads) share the array and race. 0, or -1 (err; an error state that HIP held before the call is
// left as it was and not reported as this call's).
// No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
int snk_q4_gemm_noalloc(const void* d_stripes, const void* d_xa, int M, int N, int K, float* d_y, int ldy, int epi,
                        void* stream, char* err, int err_len);
// average device time (microseconds) of one raw matmul launch (the k-slice sums into d_ws, as a decode step runs it:
// the step's row kernels add the slices) over `iters` launches timed with HIP events on `stream`, the weights taken
// from n_copies stripe copies in turn (copies beyond the 256 MB Infinity Cache keep the reads in HBM). d_y and ldy are
// not used. Synchronous; -1 when d_ws is too small.
double snk_q4_gemm_time(const void* const* d_stripes, int n_copies, const void* d_xa, int M, int N, int K, float* d_y,
                        int ldy, void* d_ws, size_t ws_bytes, int iters, void* stream);

// Average device time (microseconds) of one plain streaming read of `bytes` (a multiple of 16) over `iters` launches
// back to back on `stream`, from n_copies buffers in turn (d_sink: 1 KB of device memory the kernel could write): the
// floor for launches that move that many bytes, measured beside them. No counterpart in the reference (a calibration
// of this box); -1 for bad arguments.
double snk_read_time(const void* const* d_bufs, int n_copies, size_t bytes, float* d_sink, int iters, void* stream);

// Launch-plan tuning of the matmul (raw k-slice sums of Q4_0 stripes): an explicit plan of mt row tiles a workgroup
// (1, 2), spw stripes a wavefront (1, 2) and G groups a slice with every load of the slice issued at once (G 0: the
// default plan; mt 0, spw 0, G 0: the per-column integer-dot GEMV of M <= 4 rows, with the default plan's slices and
// the same bits). snk_q4_gemm_plan_time: average device time (microseconds) of one launch over `iters` launches on
// `stream`, weights from n_copies stripe copies in turn; -1 for a plan that is not instantiated or too small a
// workspace. snk_q4_gemm_plan_sums: the plan's slices added in order into d_y [M][N], for checking a plan; 0 or -1.
double snk_q4_gemm_plan_time(const void* const* d_stripes, int n_copies, const void* d_xa, int M, int N, int K,
                             void* d_ws, size_t ws_bytes, int mt, int spw, int G, int iters, void* stream);
int snk_q4_gemm_plan_sums(const void* d_stripes, const void* d_xa, int M, int N, int K, float* d_y, void* d_ws,
                          size_t ws_bytes, int mt, int spw, int G, void* stream);

// ---- paged GQA attention (decode and verify rows) -------------------------------------------------------------------
// Replaces attn_part + attn_merge (kernels.metal:1122-1192) and fa2 (kernels.metal:2674-2770). q: [rows][H][128] fp32
// (ldq floats apart); K/V pool fp16, page p of KV head h at pool + ((p * KVH + h) * page_cells) * 128 (a V cell: 128
// contiguous values; a K region: chunk-major, dim d of cell c at 8 * (page_cells * (d / 8) + c) + d % 8); d_pt:
// [sequences][max_pages] int32; out: [rows][ldo] fp32. Row r of sequence seq[r] attends cells 0 .. pos[r].
typedef struct snk_attn snk_attn;
// the work list of a set of rows (host arrays), built once and reused by snk_attn_run; NULL on failure (err)
snk_attn* snk_attn_new(int n_rows, const int32_t* seq, const int32_t* pos, int H, int KVH, int max_pages,
                       int page_cells, char* err, int err_len);
int snk_attn_run(snk_attn* p, const float* d_q, int ldq, const void* d_kpool, const void* d_vpool, const int32_t* d_pt,
                 float scale, float* d_out, int ldo, void* stream);
// average device time (microseconds) of one run (partials + merge) over `iters` runs (HIP events); synchronous
double snk_attn_time(snk_attn* p, const float* d_q, int ldq, const void* d_kpool, const void* d_vpool,
                     const int32_t* d_pt, float scale, float* d_out, int ldo, int iters, void* stream);
// the same with the list's form chosen by the caller: mode -1 as snk_attn_new, 0 one item per 256-cell chunk and the
// merge, 1 whole groups, 2 run items wherever a sequence has two or more consecutive full query groups (prompt rows;
// -1 takes them when they make at least 128 workgroups), the other rows as -1 (for tests and timing; every form gives
// the same bits for a row)
snk_attn* snk_attn_new_mode(int n_rows, const int32_t* seq, const int32_t* pos, int H, int KVH, int max_pages,
                            int page_cells, int mode, char* err, int err_len);
// the same with the host copy of the page table (pt [slots][max_pages], the rows' slots index it): a decode row's
// 256-cell chunk that lies wholly below its position on the very pages of other decode rows' same chunk (a shared
// prefix: sn_copy's pages) is read once for up to 4 such rows (16 / (H / KVH) at most), the engine's plan for every
// step (attn_part's per-chunk items, kernels.metal:1122-1192, with sharers batched). Gives the same bits for a row.
snk_attn* snk_attn_new_pt(int n_rows, const int32_t* seq, const int32_t* pos, int H, int KVH, int max_pages,
                          int page_cells, int mode, const int32_t* pt, char* err, int err_len);
// 1 when the list is whole groups (one workgroup per (group, KV head) walks its whole context and writes the output:
// one launch, no merge; chosen when the groups make one round of 240 .. 256 workgroups, no context is over 9/8 of the
// mean and the contexts are long), 0 when it is one item per 256-cell chunk followed by the merge. Both give the same
// bits for a row.
int snk_attn_whole(const snk_attn* p);
// the list's run items: up to 4 consecutive query groups of one sequence (16 prompt rows at G = 4) walked over their
// context by one workgroup per (item, KV head), which writes their outputs (no partials, no merge); the K/V cells of
// a chunk are read once for all of them (the prompt rows of attn_pre, kernels.metal:1201-1306, sn_attn.inc.h:195-206)
int snk_attn_runs(const snk_attn* p);
// Whether snk_attn_run launches the chunk items and their merge as one kernel (k_attn_fold: the last workgroup of each
// (group, KV head) folds the group's rows itself). Withdrawn: the form is never taken and the call always returns 0
// (it measured slower than the two launches, and one run of its bitwise test against them differed with no cause
// found). Kept so that callers of the entry point keep linking.
int snk_attn_fold(snk_attn* p, int on);
// 1 when a fold launch of this list found a (group, KV head)'s workgroups on two XCDs, 0 if never, -1 (no fold state)
int snk_attn_xcd_faults(const snk_attn* p);
void snk_attn_free(snk_attn* p);

// ---- per-head QK-norm + NEOX RoPE + K/V cache write (qk_rope, kernels.metal:149-197) -------------------------------
// d_qkv: R rows of [q: H*128 | k: KVH*128 | v: KVH*128] fp32, ldqkv floats apart; q is normed and rotated in place, k
// (normed, rotated) and v go to cell pos[r] of sequence seq[r] as fp16, in the pools' layout (snk_attn_run's).
// theta_scale = base^(-2/128) (computed by the caller in fp32, as ggml does); theta_i = pos * theta_scale^i by i
// successive fp32 multiplies.
int snk_qk_rope(float* d_qkv, int ldqkv, int R, int H, int KVH, const float* d_qw, const float* d_kw, float eps,
                float theta_scale, const int32_t* d_seq, const int32_t* d_pos, const int32_t* d_pt, int max_pages,
                int page_cells, void* d_kpool, void* d_vpool, void* stream);

// ---- mixture of experts (moe_ffn, sn_layers.inc.h:129-144) -------------------------------------------------------------
// router logits d_lg [R][NE] = d_hn [R][E] (the fp32 normed rows) x d_router [NE][E] (fp32); E % 4 == 0
int snk_moe_router(const float* d_hn, int R, int E, const float* d_router, int NE, float* d_lg, void* stream);
// rows of the expert-major tile layout of R rows with k of NE experts each: P = 16 (min(NE, R k) + ceil(R k / 16))
int snk_moe_tile_rows(int R, int NE, int k);
// routing and grouping (moe_topk1 + moe_lists, kernels.metal:3419-3497): each row's k experts (softmax of its logits,
// the k largest with ties to the lower id) d_ids [R][k] and weights d_w [R][k] (p / sum p over the k, the sum floored
// at 6.103515625e-5); the (row, slot) pairs in expert-major 16-row tiles, expert x's pairs in (row, slot) order from
// tile toff[x] = the tiles of the experts before it: d_prow [R][k] = the pair's tile row, d_rsrc [P] = the row a tile
// row carries (-1: padding), d_items [2 x P / 16] = (expert, tile) of each tile, *d_count = the tiles used.
// NE <= 256, k <= min(8, NE), R k <= 4096. 0, or -1 (bad arguments, nothing launched).
int snk_moe_select(const float* d_lg, int R, int NE, int k, int32_t* d_ids, float* d_w, int32_t* d_prow,
                   int32_t* d_rsrc, int32_t* d_items, int32_t* d_count, void* stream);
// The routing in one launch (router logits, top-k with renormalised weights, the expert-major tiles), the same results
// as snk_moe_router followed by snk_moe_select: each block of 4 rows is routed by the last of its workgroups to finish,
// whose logits it reads through its XCD's L2, and the last block groups every pair. Allocates and frees its counters
// and probes the XCD dealing (synchronous; for tests). *xerr (optional): 1 when a row block's workgroups ran on more
// than one XCD. E <= 4096 (wider rows: snk_moe_router + snk_moe_select). 0, or -1.
int snk_moe_route(const float* d_hn, int R, int E, const float* d_router, int NE, int k, float* d_lg, int32_t* d_ids,
                  float* d_w, int32_t* d_prow, int32_t* d_rsrc, int32_t* d_items, int32_t* d_count, int* xerr,
                  void* stream);
// the grouped expert matmul (the block matmul's grouped mode, kernels.metal:561-563; sn_attn.inc.h:350-358): for each
// tile i < *d_count, item (x, t) = d_items[2i], d_items[2i + 1]: rows 16t .. 16t + 15 of d_part [P][N] = the
// activation operand's rows (d_xa, P rows of K, snk_quant_act) x expert x's matrix (N x K tiles at d_w + x * wstride;
// Q4_0 stripes, or Q8_0 tiles with wt 8).
// Rows p with d_rmask[p] < 0 are not written (d_rmask may be NULL). max_items: the grid's tile bound (P / 16).
int snk_gemm_grouped(int wt, const void* d_w, size_t wstride, const int32_t* d_items, const int32_t* d_count,
                     int max_items, const void* d_xa, int P, int N, int K, float* d_part, size_t part_bytes,
                     const int32_t* d_rmask, void* stream);

// ---- greedy argmax of logit rows (argmax / argmax_p, kernels.metal:327-442) -------------------------------------------
// d_logits: n rows of V fp32 scores; d_out[r] = the first index of the largest score of row r; rows with d_skip[r] != 0
// (d_skip may be NULL) never take the nban <= 8 ids of d_ban (-1 when every id is banned). d_rec (may be NULL): per row
// 8 words: chosen id, its score, best id, best score, second id, second score (the pair over all ids, ties to the lower
// id), log-sum-exp, 0. d_ws: snk_argmax_workspace_bytes(n, V) bytes. 0, or -1 (bad arguments, workspace too small).
size_t snk_argmax_workspace_bytes(int n, int V);
int snk_argmax(const float* d_logits, int V, int n, const int32_t* d_ban, int nban, const uint8_t* d_skip,
               int32_t* d_out, float* d_rec, void* d_ws, size_t ws_bytes, void* stream);

// ---- MFMA operand layout check: D = A . B for one v_mfma_f32_16x16x32_f16 (A, B as 64 lanes x 8 fp16 each, D as 64
// lanes x 4 fp32), the raw lane contents in and out
int snk_mfma_probe(const void* d_a, const void* d_b, float* d_d, void* stream);

#ifdef __cplusplus
}
#endif
