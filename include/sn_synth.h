// sn_synth.h — synthetic random-init models for the benchmarks and tests (a tool beside the engine, not a hot-path
// entry point). It stands where the reference's tests build a model file with sllm-core's testutil.rs tiny_model
// (engine/sllm-core/src/testutil.rs:22-162); the configs' models are random-init, so the file is generated.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    int n_expert, n_expert_used, n_ff_exp;  // > 0: a qwen3moe model (experts in every layer)
    int nextn;                              // 1: one multi-token-prediction layer after the model's own (blk.<n_layer>)
    float rope_base, eps;
    float w_std;    // std of the matrices before quantization (configs: 0.02)
    float emb_std;  // std of the fp32 embedding table
    int wtype;      // the matrices' block type: 2 (0 too) Q4_0, 8 Q8_0
    int embd_type;  // token_embd's type: 0 F32, 2 Q4_0, 8 Q8_0, 14 Q6_K (seeded valid blocks; n_embd % 256 == 0)
    int tied;       // 1: no output.weight, the LM head is token_embd (which must then be quantized)
} snx_model_cfg;

// Write the model to `path` (GGUF v3; matrices quantized with ggml's quantize_row_q4_0_ref or quantize_row_q8_0_ref;
// norms 1 + N(0, 0.1); a Q6_K token table as seeded blocks: q uniform in 0..63, scales uniform in -15..15, d chosen
// for emb_std). nthreads <= 0: all cores. The bytes depend only on (cfg, seed). 0, or -1 with the reason in err.
int snx_write_model(const char* path, const snx_model_cfg* cfg, uint64_t seed, int nthreads, char* err, int err_len);

// ggml quantize_row_q4_0_ref of k values (k % 32 == 0): 18-byte blocks into y.
void snx_quantize_q4_0(const float* x, uint8_t* y, int64_t k);
// ggml quantize_row_q8_0_ref of k values (k % 32 == 0): 34-byte blocks into y.
void snx_quantize_q8_0(const float* x, uint8_t* y, int64_t k);

#ifdef __cplusplus
}
#endif
