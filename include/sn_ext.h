// sn_ext.h — engine calls beyond sn.h: per-kernel GPU timing of steps (the role of the reference's SN_PROF switch,
// core.h:232-302 / sn_load.inc.h:49-61, which gives every kernel of a step its own timestamps summed by name) and a
// readback of a step's row buffers for stage-by-stage checks. None of these changes what a step computes.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "sn.h"

#ifdef __cplusplus
extern "C" {
#endif

// kernel classes of a step
enum {
    SNX_K_GEMM = 0,   // Q4_0 x Q8_0 matmuls (q/k/v, o, gate/up, down, LM head) incl. their k-slice reductions
    SNX_K_ATTN = 1,   // paged attention: the chunk partials (per-chunk items), or whole groups (outputs written)
    SNX_K_QUANT = 2,  // Q8_0 activation quantizers (with the RMSNorm fused in front)
    SNX_K_ROPE = 3,   // QK-norm + RoPE + K/V cache write
    SNX_K_OTHER = 4,  // embedding, argmax, copies
    SNX_K_MERGE = 5,  // the attention merge: chunk partials folded into the outputs and the o-projection operand
    SNX_K_COUNT = 6
};

// Profiling on (resets the counters) or off. While on, every launch of a step is bracketed by HIP events on the
// engine's stream, so steps take slightly longer; the tokens are the same.
void snx_prof(sn_engine* e, int on);
// The totals since profiling was turned on for one class: GPU milliseconds, launches, and the algorithmic bytes those
// launches move (matmul: Q4_0 weights + fp32 input rows + fp32 output rows; attention: the fp16 K/V cells each
// (sequence, KV head) reads once + q + output + page-table entries). 0, or -1 for an unknown class.
int snx_prof_read(const sn_engine* e, int kind, double* ms, int* launches, double* bytes);

// Graph replay of steps on (the default) or off. While on, sn_step captures its device work as a HIP graph the first
// time a step shape occurs (rows, outputs, attention work-list size, ...) and replays it while the shape repeats,
// which saves the per-launch cost of ~370 launches a step; the launches and results are the same as with it off.
// Profiling (snx_prof) runs steps without graphs.
void snx_graphs(sn_engine* e, int on);
// Steps captured as a new graph (replays 0) or replayed from the cached one (replays 1) since the engine opened.
long snx_graph_count(const sn_engine* e, int replays);
// Steps taken from the queue (dropped 0: sn_step's chain found the queued step to be the one asked for) or queued and
// dropped (dropped 1: another step or a cache call came first; its cells were zeroed) since the engine opened.
long snx_chain_count(const sn_engine* e, int dropped);
// The attention work list's form: -1 chosen per step (the default), 0 one item per 256-cell chunk and a merge, 1
// whole groups (one workgroup per (group, KV head) walks the whole context: no merge), 2 run items for every
// sequence with two or more consecutive full query groups (prompt rows; -1 takes them when they make at least 128
// workgroups), the other rows as -1. Every form gives the same bits.
void snx_attn_mode(sn_engine* e, int mode);
// The matmul epilogues fused into decode-sized steps' q|k|v (QK-norm, RoPE, cache write) and gate|up (SwiGLU + Q8_0)
// launches, done by each set's last workgroup through its XCD's L2: on when sn_open's probe found the device dealing
// workgroups to its XCDs in turn by linear id (and SN_NO_FUSE is unset). on 0 switches them off (the split path: the
// same bits), 1 back on where the probe allows. Returns whether they are on. Drops captured graphs.
int snx_fuse(sn_engine* e, int on);
// Whether a fused launch ran a workgroup on another XCD than the probe predicted (then its epilogue may have read
// stale sums): 0 never, 1 it did, -1 error. Waits for the engine's work.
int snx_xcd_faults(sn_engine* e);
// The graph key sn_step forms for a step of R rows (slots seq, positions pos; every row sampled in order) on an engine
// of H query heads, KVH KV heads and page_cells-cell pages with attention form `mode` (as snx_attn_mode), computed on
// the host alone (no device): two steps replay one captured graph exactly when their keys are equal. Writes at most
// cap values to key and the attention form chosen to *whole (when given); returns the key's length, or -1 for bad
// arguments. (Host code only; for checks of the replay rule.) The probe has no page table, so it plans the step as
// an engine whose slots share no pages: for an engine with pages shared by sn_copy, the shared-prefix attention items
// its step forms (and so its key) are not covered.
int snx_step_key(int H, int KVH, int page_cells, int mode, int R, const int32_t* seq, const int32_t* pos,
                 int64_t* key, int cap, int* whole);

// Give slot `slot` the cells [0, n) (pages as a step would take them) holding seeded N(0, 1) fp16 K and V in every
// layer: a context "already in the cache" for throughput runs (what the cells hold does not change what a step
// costs). The values depend only on (seed, slot, layer, cell). 0, -2 out of pages, or -1 (err).
int snx_fill_kv(sn_engine* e, int slot, int n, uint64_t seed, char* err, int err_len);

// The last step's row buffers: 0 the residual rows x [R][E], 1 the last layer's q|k|v rows (q after QK-norm and RoPE;
// k, v as the matmul wrote them) [R][H*128 + 2*KVH*128], 2 its attention output [R][H*128], 3 its SwiGLU output
// [R][F]. n floats into dst. 0, or -1.
int snx_debug_read(sn_engine* e, int which, float* dst, size_t n);

// The fused draft-verify step of a guess-head model (guessing on): for each of n sequences (slot seq[s], its pending
// token last[s] at position pos[s], its cells before pos[s] in the cache) the guess head drafts k tokens (1 .. 4;
// sn_guess's rows, batched over the sequences), the model runs the verify rows [last, d1 .. dk] at pos .. pos + k
// (every sequence in one pass), and greedy acceptance keeps the leading drafts equal to their row's argmax
// (next_engine/draft.rs:135-178, take.rs:339-357) — all on the GPU in one submission, one wait. Per sequence: out_n[s]
// = accepted + 1 tokens in out_tok[s * (k + 1) ..]: the accepted drafts, then the correction (bonus) token, which is
// the sequence's next pending token at pos[s] + out_n[s]; the rest of its row is -1. The cells of the refused rows
// are zeroed in every layer (as sn_clear would leave them; their pages stay with the slot) and the head's state moves
// to the last kept row. force (optional, [n][k] bytes): verify row i of sequence s with force[s * k + i] set takes
// draft i + 1 as its argmax (a seeded acceptance rate for benchmarks; the rows still run in full). 0, -2 out of
// pages (nothing ran), or -1 (err).
int snx_spec_step(sn_engine* e, int n, const int32_t* seq, const int32_t* last, const int32_t* pos, int k,
                  const uint8_t* force, int32_t* out_n, int32_t* out_tok, char* err, int err_len);

#ifdef __cplusplus
}
#endif
