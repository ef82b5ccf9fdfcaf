// sn.h — the per-step C ABI of the MI355X decode/verify engine (libsn_hip.so).
//
// Drop-in for the reference's engine/sllm-next/proto/sn.h (its 49 functions, same names, signatures, argument meaning
// and return codes), so the reference's Rust binding engine/sllm-server/src/next_engine/ffi.rs:16-63 links against
// this library unchanged. Each declaration cites the reference declaration it replaces.
//
// Contract kept from the reference:
//   * One thread calls every function; calls are synchronous (sn_step returns after the GPU finished).
//   * A row's result does not depend on the other rows of its step (same tokens at any batch size).
//   * Return codes: 0 ok; -1 with a NUL-terminated reason in err[err_len]; -2 out of cache pages (nothing ran);
//     -3 (sn_copy / sn_clear) the window layers no longer hold the cells (never, for the models served here).
//   * Greedy ties go to the lowest token id.
// What differs: the `kernels` argument of sn_open is ignored (the HIP kernels are compiled into the library).
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sn_engine sn_engine;

// sn.h:16 — load a GGUF (qwen3 / qwen3moe, head_dim 128, Q4_0 matrices, fp32 embedding and norms) for `slots`
// sequences of up to `ctx` cells, `pages` pages of cells (0: every slot its whole ctx), steps of up to max_rows rows.
// Page size: 64 cells (SN_PAGE=32 in the environment selects 32). NULL on failure with the reason in err.
sn_engine* sn_open(const char* gguf_path, const char* kernels, int slots, int ctx, int max_rows, int pages, char* err,
                   int err_len);
// sn.h:22 — whether sn_open can run the file (header and tensor table only); rows: the prompt rows per step to use.
int sn_check(const char* gguf_path, int* rows, char* err, int err_len);
// sn.h:24 — prompt rows for quiet periods (0: the usual).
int sn_quiet_rows(const char* gguf_path);

int sn_n_vocab(const sn_engine* e);      // sn.h:26
int sn_n_ctx_train(const sn_engine* e);  // sn.h:27
const char* sn_arch(const sn_engine* e); // sn.h:29 — "qwen3" or "qwen3moe"

// sn.h:40-41 — one step of R rows (tok, seq, pos). Rows [0, n_write) are write rows (the first n_fast interactive,
// n_fast <= 4; n_fast < 0: a wide draft check of -n_fast <= 8 rows of one sequence), rows [n_write, R) prompt rows
// (consecutive positions of a sequence on consecutive rows). out_tok[j] = greedy token of row out_rows[j].
// chain: the caller will run the same rows next fed these tokens (accepted; the step runs as an ordinary step).
int sn_step(sn_engine* e, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos, int n_write, int n_fast,
            int n_out, const int32_t* out_rows, int32_t* out_tok, int chain, char* err, int err_len);

double sn_last_gpu_ms(const sn_engine* e);  // sn.h:44 — GPU milliseconds of the last step

// sn.h:48 / :50 — scores of output row k (or rows ks) of the last step, n_vocab floats each.
int sn_logits(sn_engine* e, int k, float* dst, char* err, int err_len);
int sn_logits_rows(sn_engine* e, int n, const int* ks, float* dst, char* err, int err_len);

// sn.h:56 / :61 — token probabilities: while on, each output row also gets the record
// {chosen id, chosen score, best id, best score, second id, second score, log-sum-exp, 0}.
void sn_want_probs(sn_engine* e, int on);
int sn_probs(sn_engine* e, int n_out, float* dst, char* err, int err_len);

// sn.h:67 / :75 / :83 / :87-88 — latent rows, soft words, embedding rows: not served by this engine (-1 / 0).
int sn_latent(sn_engine* e, int n, const int32_t* rows, const float* vec, float* hid, char* err, int err_len);
int sn_n_embd(const sn_engine* e);
int sn_soft_config(sn_engine* e, float temp, int k, const int32_t* eog, int n_eog, char* err, int err_len);
int sn_soft_rows(sn_engine* e, int n_in, const int32_t* in_rows, int n_out, const int32_t* out_ks, char* err,
                 int err_len);
int sn_embed_rows(sn_engine* e, int n, const int32_t* ids, float* dst, char* err, int err_len);
float sn_embd_norm(sn_engine* e);

// sn.h:93-94 — end-of-generation ids (at most 8) and the slots whose rows never take them.
int sn_set_eog(sn_engine* e, const int32_t* ids, int n);
void sn_no_end(sn_engine* e, int slot, int on);

// sn.h:99 — slot `to` takes cells [0, n) of `from`: full pages shared, the partly filled last page copied.
int sn_copy(sn_engine* e, int from, int to, int n, char* err, int err_len);
// sn.h:104 — cut a slot to its first `from` cells (cells [from, to) were its last): pages past the cut freed and
// zeroed, the cut page keeps its first cells (a private copy when shared), its cells [from, to) zeroed.
int sn_clear(sn_engine* e, int slot, int from, int to, char* err, int err_len);
int sn_cut_ok(const sn_engine* e, int slot, int n);    // sn.h:108 — always 1 (no window layers)
int sn_recurrent(const sn_engine* e);                  // sn.h:113 — 0

// sn.h:117-126 — the guess (MTP / nextn) head.
int sn_guess_head(const sn_engine* e);
int sn_guess_on(sn_engine* e, int on);
int sn_guess(sn_engine* e, int seq, int32_t tok, int pos, int k, int32_t* out_tok, char* err, int err_len);

int sn_draft_rows(sn_engine* e, int seq, int want);  // sn.h:133 — `want` back (not a recurrent model)
int sn_small_rows(const sn_engine* e);               // sn.h:138 — 0 (one matmul path for every row count)
int sn_chat_exact(const sn_engine* e);               // sn.h:142 — 1 (rows are always exact)
int sn_mark(sn_engine* e, int slot);                 // sn.h:146 — 0
int sn_state_take(sn_engine* e, int seq);            // sn.h:147 — -1
int sn_cut_best(const sn_engine* e, int slot, int n);  // sn.h:151 — n when sn_cut_ok takes it, 0 for a bad slot or n <= 0

// sn.h:155-158 — the page pool.
int sn_pages_total(const sn_engine* e);
int sn_pages_free(const sn_engine* e);
size_t sn_page_bytes(const sn_engine* e);
int sn_seq_pages(const sn_engine* e, int seq, int* own);
// sn.h:163-165 — window pool (none here): 0.
int sn_win_need(const sn_engine* e, int n);
int sn_win_room(const sn_engine* e);
int sn_win_pages(const sn_engine* e, int seq);

// sn.h:168-170 — a slot's first n cells to host memory and back: per layer, K then V, each n cells of
// n_kv * 128 fp16 values (cell-major).
size_t sn_kv_bytes(const sn_engine* e, int n);
int sn_kv_save(sn_engine* e, int slot, int n, void* dst, char* err, int err_len);
int sn_kv_load(sn_engine* e, int slot, int n, const void* src, char* err, int err_len);

size_t sn_trim(sn_engine* e, int spare);      // sn.h:175 — 0 (the pool is one allocation)
int sn_trim_pending(sn_engine* e);            // sn.h:177 — 0
size_t sn_mem_used(const sn_engine* e);       // sn.h:179 — bytes of the pages in use
size_t sn_state_bytes(const sn_engine* e);    // sn.h:182 — 0
int sn_state_entries(const sn_engine* e, int seq);  // sn.h:183 — 0

void sn_close(sn_engine* e);  // sn.h:185

#ifdef __cplusplus
}
#endif
