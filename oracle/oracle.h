// CPU oracle for the batched decode/verify step: a plain-C restatement of the arithmetic the GPU path must reproduce.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product (sonic-llm_amd/) links, imports or calls this code; only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the checker / the CPU baseline.
//
// What it restates (the reference's own path is Objective-C + Metal and cannot be built here; ggml/llama.cpp b11669,
// the north star's CPU reference, is not in /root/reference, only its headers):
//   * ggml b11669 `quantize_row_q4_0_ref`, `dequantize_row_q4_0` (block_q4_0 = fp16 d + 16 nibble bytes, w = d*(q-8));
//     the reference's own CPU copy of the dequant: vendor/sllm-metal-b11669/patches/0001-sllm-qmm-kernel.patch:543-565,
//     and the GPU-side form kernels.metal:21-28, :461-469.
//   * ggml's x86 CPU `quantize_row_q8_0` (activations of a Q4_0 mul_mat: d = amax/127 stored fp16, id = 127/amax,
//     q = round-half-even(x*id)) and the generic `ggml_vec_dot_q4_0_q8_0` (integer block sums, fp32 sumi*dw*dx).
//   * Q8_0 weights: ggml `quantize_row_q8_0_ref` (d = amax/127, q = roundf(x/d)), `dequantize_row_q8_0` (d*q) and the
//     generic `ggml_vec_dot_q8_0_q8_0` (the reference's Q8_0 kernels: kernels.metal:9, :597-609, :1995-2130).
//   * fp32 RMSNorm (kernels.metal:121-140; ggml rms_norm sums squares in double), per-head QK-norm + NEOX RoPE with ggml's
//     iterative theta (kernels.metal:149-197), SwiGLU silu(g)*u (kernels.metal:564-568), greedy argmax with the lowest id on
//     ties (kernels.metal:327-356), paged GQA decode attention (kernels.metal:1122-1192), the Qwen3 layer order
//     (sn_attn.inc.h:216-231) and the output stage (sn_encode.inc.h:248-317).
//   * Q6_K (the token table / tied LM head of real Qwen3 GGUFs; the reference reads them, sn_load.inc.h:341-359,
//     kernels.metal:1010-1120): ggml `dequantize_row_q6_K`, the Q8_K activations of a Q6_K mul_mat
//     (`quantize_row_q8_K_ref`) and the generic `ggml_vec_dot_q6_K_q8_K` (integer sums of scale * (q6 - 32) * q8 per
//     16-element group in 8 lanes, fp32 sums[l] += d6 * d8 * aux32[l]).
//   * MoE routing softmax -> top-k (ties: lower id) -> renormalise with the sum floored at 6.1035e-5 (kernels.metal:3419-3467).
//   * Draft acceptance: rows checked in order, kept while draft == target argmax (next_engine/take.rs:339-357).
//
// How each function is pinned (tests/test_oracle.py, tests/test_golden.py): dequant by the closed form on every nibble
// and fp16 specials; fp16 conversion against numpy; mul_mat against an fp64 product of the dequantized operands and
// against the integer block sum; RMSNorm, RoPE, argmax/top-2, MoE routing and acceptance against closed forms or brute
// force; Q6_K dequant by an independent packer of explicit values, Q8_K by its invariants, vec_dot_q6_K_q8_K by the
// explicit integer block sum and the fp64 product of the dequantized operands; paged attention against an fp64 dense
// softmax over page-gathered cells, chunked == monolithic, page-placement
// and shared-prefix invariance; the model writer's GGUF layout against the reference's own GGUF fixture.
// The composed functions (tests/test_oracle_model.py): or_qwen3_step (dense Q4_0 / Q8_0 and MoE layers, the output
// stage), or_mtp_fill and or_mtp_guess equal, bit for bit (logits, tokens, normed rows, cache cells), tests/ref64.py, a
// numpy restatement written from the reference's layer program, MoE FFN, output stage and guess-head rows with ggml's
// per-operation fp32 arithmetic; and two invariants: one expert copied to every expert gives the dense FFN, a guess
// head whose eh_proj ignores the hidden-state half guesses independently of it.
// Parity unpinned against ggml itself (no ggml vector exists offline): the exact bytes of quantize_row_q4_0_ref and of
// x86 quantize_row_q8_0 (their rounding rules are restated from ggml's published source and checked by invariants
// only), and ggml's fp32 summation order inside mul_mat (checked to tolerance only).
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- fp16 (IEEE binary16, round to nearest even; what ggml's GGML_FP32_TO_FP16 does with F16C) ----
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);

// ---- Q4_0 / Q8_0 blocks ----
// block_q4_0: 18 bytes = fp16 d, qs[16]; element j (<16) = qs[j] & 15, element j+16 = qs[j] >> 4; value d*(q-8).
// block_q8_0: 34 bytes = fp16 d, int8 qs[32]; value d*q.
void or_quantize_row_q4_0(const float* x, uint8_t* y, int64_t k);
void or_dequantize_row_q4_0(const uint8_t* x, float* y, int64_t k);
void or_quantize_row_q8_0(const float* x, uint8_t* y, int64_t k);
void or_dequantize_row_q8_0(const uint8_t* x, float* y, int64_t k);
float or_vec_dot_q4_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq);

// Y[m][n] = sum_k X[m][k] * W[n][k] with ggml CPU semantics: X rows quantized to Q8_0, integer block dots.
// block_q8_0 weights: ggml quantize_row_q8_0_ref (roundf of x / d, d = amax/127); vec_dot_q8_0_q8_0 and the mul_mat of
// Q8_0 weights (activations quantized with or_quantize_row_q8_0)
void or_quantize_row_q8_0_ref(const float* x, uint8_t* y, int64_t k);
float or_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq);
void or_mul_mat_q8_0(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads);
// Test hook: reverse 1 makes or_vec_dot_q4_0_q8_0 and or_vec_dot_q8_0_q8_0 (and so every Q4_0 / Q8_0 mul_mat and model
// step; also the fp32 MoE router's dots) add their terms last first; 0 (the default) is ggml's order. Two implementations of the same
// arithmetic that differ only in summation order: the distance between them over a whole model is the end-to-end
// bound any other implementation (the GPU's) can be held to.
void or_set_sum_order(int reverse);
// W: N rows of K/32 Q4_0 blocks. nthreads <= 0: all cores (OpenMP).
void or_mul_mat_q4_0(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads);
// The same product in fp64 over dequantized W and the fp32 X as given (no activation quantization): the
// self-test reference of patch 0001 (:651-667).
void or_mul_mat_q4_0_f64(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, double* Y, int nthreads);

// ---- elementwise pieces ----
void or_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y);
float or_silu(float x);
// argmax of n scores: the first index of the largest; ban (nban ids) never taken. -1 if n == 0.
int32_t or_argmax(const float* x, int64_t n, const int32_t* ban, int nban);
// the two best (ties: lower id) and the log-sum-exp of a row (argmax_p's record, kernels.metal:358-442)
void or_top2(const float* x, int64_t n, int32_t* i1, float* v1, int32_t* i2, float* v2, float* lse);
// NEOX rope angle table for one position: theta_i = p * s^i computed iteratively in fp32 (ggml_rope_cache_init),
// s = theta_scale (powf(base, -2/D) computed by the caller). cs[2i] = cos, cs[2i+1] = sin, i < D/2.
void or_rope_cache(int32_t pos, float theta_scale, int D, float* cs);
// per-head RMSNorm (weight w[D]) then NEOX rotation of pairs (i, i + D/2); x is one head of D floats, in place
void or_qk_norm_rope(float* x, const float* w, int D, float eps, const float* cs, int do_norm);

// ---- paged GQA decode attention ----
// q: [nq][H][D] fp32 (nq query rows); row r belongs to sequence qseq[r] and attends cells 0..qpos[r] of it.
// K/V pool: fp16, page p of cells holds, for kv head h, cells [page_cells][D] at
//   pool + ((size_t) p * KVH + h) * page_cells * D   (head-major inside a page).
// pt[s * max_pages + c]: the page of sequence s's cells c*page_cells ..; out: [nq][H][D].
// scale: softmax scale applied to the scores. f64: 1 = accumulate in double (closed-form reference), 0 = fp32
// online-free two-pass softmax (max, exp, sum) in fp32.
void or_paged_attn(const float* q, int nq, const int32_t* qseq, const int32_t* qpos, int H, int KVH, int D,
                   const uint16_t* kpool, const uint16_t* vpool, int page_cells, const int32_t* pt, int max_pages,
                   float scale, float* out, int f64, int nthreads);
// the same attention computed in chunks of `chunk` cells with per-chunk (m, l, acc) partials merged in chunk order
// (attn_part / attn_merge, kernels.metal:1122-1192): an invariant check against the monolithic form.
void or_paged_attn_chunked(const float* q, int nq, const int32_t* qseq, const int32_t* qpos, int H, int KVH, int D,
                           const uint16_t* kpool, const uint16_t* vpool, int page_cells, const int32_t* pt,
                           int max_pages, float scale, int chunk, float* out);

// ---- Q6_K weights / Q8_K activations (ggml k-quants, QK_K = 256 elements a block) ----
// block_q6_K: 210 bytes = ql[128] (low 4 bits), qh[64] (high 2 bits), int8 scales[16], fp16 d. Element e of a block:
// half h = e / 128, quarter c = (e % 128) / 32, l = e % 32: the low nibble (c < 2) or high nibble (c >= 2) of
// ql[64h + 32 (c & 1) + l], high bits (qh[32h + l] >> 2c) & 3; value d * scales[e / 16] * (q - 32)
// (ggml dequantize_row_q6_K: (d * scale) * (q - 32), fp32 left to right).
// block_q8_K: fp32 d, int8 qs[256], int16 bsums[16] (292 bytes). quantize_row_q8_K_ref: max = the element of largest
// |x| (the first on ties), iscale = -127 / max, q = min(127, nearest_int(iscale * x)) (round half to even),
// d = 1 / iscale, bsums = the sums of 16 consecutive q; an all-zero block gets d = 0, q = 0.
void or_dequantize_row_q6_K(const uint8_t* x, float* y, int64_t k);
void or_quantize_row_q8_K(const float* x, uint8_t* y, int64_t k);
// ggml_vec_dot_q6_K_q8_K (generic form): per block the integer sums scale * (q6 - 32) * q8 in 8 lanes (aux32), then
// sums[l] += (d6 * d8) * aux32[l]; the result is the sum of the 8 lanes
float or_vec_dot_q6_K_q8_K(int64_t k, const uint8_t* w, const uint8_t* xq);
// Y[M][N] = X[M][K] . W[N][K]^T with Q6_K weights (ggml CPU mul_mat: Q8_K activations, vec_dot_q6_K_q8_K); K % 256 == 0
void or_mul_mat_q6_K(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads);

// ---- a Qwen3 dense model (the GGUF's tensors; Q4_0 or Q8_0 matrices in GGUF block layout, ne = [K, N]) ----
typedef struct {
    const float* attn_norm;  // [E]
    const float* q_norm;     // [D]
    const float* k_norm;     // [D]
    const float* ffn_norm;   // [E]
    const uint8_t* wq;       // [H*D][E]
    const uint8_t* wk;       // [KVH*D][E]
    const uint8_t* wv;       // [KVH*D][E]
    const uint8_t* wo;       // [E][H*D]
    const uint8_t* wg;       // [F][E]
    const uint8_t* wu;       // [F][E]
    const uint8_t* wd;       // [E][F]
    // MoE layer (n_expert > 0): router fp32 [NE][E], experts Q4_0 [NE][FE][E] / [NE][E][FE]
    const float* router;
    const uint8_t* eg;
    const uint8_t* eu;
    const uint8_t* ed;
} or_layer;

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    int n_expert, n_expert_used, n_ff_exp;
    float eps, rope_base;
    const float* tok_embd;     // [V][E] fp32
    const float* output_norm;  // [E]
    const uint8_t* output;     // Q4_0 [V][E]
    const or_layer* layers;    // n_layer
    // the guess head (MTP; NULL when absent): one more block, eh_proj Q4_0 [E][2E], its norms [E]
    const or_layer* mtp;
    const uint8_t* mtp_eh;
    const float *mtp_enorm, *mtp_hnorm, *mtp_head_norm;  // head_norm: shared_head_norm, else output_norm
    int wtype;      // the matrices' block type: 2 Q4_0 (block_q4_0), 8 Q8_0 (block_q8_0)
    int head_type;  // the output matrix's: 2 Q4_0, 8 Q8_0, 14 Q6_K (token_embd's when the head is tied); 0: wtype
} or_qwen3;

// The oracle's KV cache: contiguous per (sequence, layer): K and V fp16 [ctx][KVH][D]. n_layer counts the guess
// head's block too (its cells are layer n_layer - 1 of the model's n_layer + 1).
typedef struct {
    int n_seq, ctx, n_layer, n_kv, head_dim;
    uint16_t* k;  // [n_seq][n_layer][ctx][KVH][D]
    uint16_t* v;
} or_kv;

// One step of R rows (tok, seq, pos): every layer writes each row's K/V at (seq, pos) before any row of that layer
// attends, so rows of one sequence at consecutive positions see each other causally (prompt rows, draft rows).
// logits: [n_out][V] of rows out_rows; hidden (optional): [n_out][E] of those rows after the final norm;
// out_tok: the greedy token of each output row; hn_all (optional): [R][E] every row after the final norm (what the guess
// head pairs with the next position's token). nthreads <= 0: all cores.
void or_qwen3_step(const or_qwen3* m, or_kv* kv, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos,
                   int n_out, const int32_t* out_rows, float* logits, float* hidden, int32_t* out_tok, float* hn_all,
                   int nthreads);

// The guess head's cache cells of R rows (mtp_fill, sn_state.inc.h:283-313): row r's cell at (seq, pos) from its token
// and hprev [R][E], the model's hidden state after the output norm at pos - 1 (zeros at position 0): eh_proj of
// [enorm(embed(tok)); hnorm(hprev)], the head block's attn_norm, k (QK-norm, RoPE) and v.
void or_mtp_fill(const or_qwen3* m, or_kv* kv, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos,
                 const float* hprev, int nthreads);
// k guesses of one sequence (sn_guess / guess_row, sn_cache.inc.h:300-388): row j at position pos + j takes token tok
// (then guess j - 1) and hprev (then the head's own output state), runs the head block (writing its cell), the head
// norm, the LM head and argmax. logits (optional): [k][V].
void or_mtp_guess(const or_qwen3* m, or_kv* kv, int seq, int32_t tok, int pos, int k, const float* hprev,
                  int32_t* out_tok, float* logits, int nthreads);

// MoE FFN routing of one row: softmax over n_expert router logits, the k largest (ties: lower id), weights
// renormalised by their sum floored at 6.103515625e-5 (kernels.metal:3419-3467).
void or_moe_route(const float* logits, int n_expert, int k, int32_t* ids, float* w);

// Test hook: while margins is set, every MoE routing of or_qwen3_step records its margin, the smallest router logit
// chosen minus the largest one not chosen, into margins (at most cap, in call order: layer by layer, row by row);
// or_moe_trace_count() is the number recorded. NULL turns it off.
void or_moe_trace(float* margins, int cap);
int or_moe_trace_count(void);

// Greedy acceptance of one sequence's verify rows: target[i] is row i's argmax (row 0: the last accepted token's
// row, row i: draft i's row), draft[i] (i < k) the i-th draft. Returns the accepted count a in 0..k; the tokens the
// sequence takes are draft[0..a) and then target[a] (the bonus / correction token). (next_engine/take.rs:339-357)
int or_accept(const int32_t* draft, const int32_t* target, int k);

#ifdef __cplusplus
}
#endif
