// Shared definitions of the MI355X (gfx950) decode/verify step: vector types, MFMA fragment types, error macro, and the
// device-side layouts every kernel agrees on.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define SN_WAVE 64

// ---- the KV cache: per layer, K and V pools of pages; page p of KV head h is the region of page_cells cells at
// pool + (p * KVH + h) * page_cells * 128 halves. A V cell is 128 contiguous fp16 (cell * 128 + d). A K region holds its
// cells' dims in 16-byte chunks of 8, chunk-major: chunk j of every cell, then chunk j + 1, so chunk j of 16
// consecutive cells is 256 contiguous bytes, the span a quarter-wavefront of an attention score load reads (a K cell
// stored whole, that quarter-wavefront touched 16 cells 16 bytes each: the decode step's attention 8% slower).
__host__ __device__ __forceinline__ size_t kcell_at(int page_cells, int cell, int d) {
    return ((size_t) (d >> 3) * page_cells + cell) * 8 + (d & 7);
}

// ---- raw buffer loads: a per-lane byte offset and a wavefront-uniform one against a resource of `bytes`; a load
// reaching past `bytes` returns zeros and touches no memory
#define RSRC_WORD3 0x00020000  // raw buffer resource, gfx9 data format
#define XA_GATHER_OOB 0x40000000u  // a per-lane offset past any buffer this code makes: the load reads zeros
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short) 0, (int) bytes, RSRC_WORD3);
}
typedef __attribute__((address_space(3))) void* lds_ptr;  // an LDS address (buffer loads straight into LDS)
// Drops this CU's vector L1 lines (buffer_inv sc0). A launch's last-arriving workgroup calls it before reading what
// other workgroups of its XCD stored in the launch: their stores are in the XCD's L2, but a line this CU read earlier
// in the launch (a neighbour's record sharing the line) may still sit in its L1, and a load's sc0 bit does not keep the
// load off it.
__device__ __forceinline__ void l1_drop() { asm volatile("buffer_inv sc0" ::: "memory"); }
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
}
// A 16-byte load with the non-temporal hint (cache-policy bit nt = 2): the attention's K/V cells, read once a step.
// Measured on MI355X: configs[1] 63.3 -> 61.4 us, the decode step's attention 54.3 -> 52.8 us a layer; nt | sc0 the
// same, sc0 alone slower (63.4 us); the nt hint on the matmuls' weight tiles made them slower (gate|up 2203 -> 2095
// GB/s), so they load with the default policy, and so do the prompt rows' run items, whose items of one sequence read
// the same cells in turn (their prompt steps: 52.6 against 47.4 us a launch with the hint).
template <int CPOL = 2>
__device__ __forceinline__ u32x4 bload16nt(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, CPOL));
}
__device__ __forceinline__ u32x2 bload8(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0));
}
__device__ __forceinline__ float bload4f(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
}

// HIP call check for host code: on failure, format the reason into (err, err_len) and return `ret`.
#define SN_HIP_TRY(call, ret)                                                                              \
    do {                                                                                                   \
        hipError_t e_ = (call);                                                                            \
        if (e_ != hipSuccess) {                                                                            \
            sn_set_err(err, err_len, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return ret;                                                                                    \
        }                                                                                                  \
    } while (0)

void sn_set_err(char* err, int err_len, const char* fmt, ...);

// ---- Q4_0 weights in HBM ("stripes") -------------------------------------------------------------------------------
// A GGUF Q4_0 matrix (N rows of K/32 18-byte blocks: fp16 d, 16 nibble bytes) is re-laid at upload into tiles of 16
// rows x 4 blocks, 1152 bytes each, so that one wavefront reads a tile with one 16-byte load per lane:
//   bytes [0, 1024): lane l = n + 16 g (n = row in tile, g = 0..3) holds, for blocks b = 0..3 of the tile, the 4 bytes
//                    qs[4g], qs[4g+2], qs[4g+1], qs[4g+3] of row n (offset 16 l + 4 b: the middle two swapped, so
//                    that the unpack takes 5 instructions, q4_unpack). GGUF byte qs[j]'s low nibble is element j, its
//                    high nibble element j + 16, so lane (n, g) holds elements {4g..4g+3} and {16+4g..16+4g+3}.
//   bytes [1024, 1152): the 16 rows' fp16 scales d, 4 per row (offset 1024 + 8 n + 2 b).
// Tiles of one 16-row stripe follow each other along K, so a stripe is one contiguous stream of K/128 tiles.
// Bytes per weight are those of GGUF (18 per 32); only their order changes. Rows are padded to 16 and blocks to 4
// with zero tiles.
#define Q4T_BYTES 1152
#define Q4T_SCALE_OFF 1024

// ---- Q8_0 weights in HBM ------------------------------------------------------------------------------------------
// A GGUF Q8_0 matrix (N rows of K/32 34-byte blocks: fp16 d, 32 int8 q; value d*q) is re-laid at upload into tiles of
// 16 rows x 4 blocks, 2176 bytes each (= 64 x 34, the GGUF bytes):
//   bytes [0, 2048): lane l = n + 16 g holds 32 bytes, for blocks b = 0..3 of row n: at 32 l + 8 b the int8 q of
//                    elements 4g..4g+3, then of 16+4g..16+4g+3 (the element order of the Q4_0 tile lanes);
//   bytes [2048, 2176): the 16 rows' fp16 scales d, 4 per row (offset 2048 + 8 n + 2 b).
#define Q8T_BYTES 2176
#define Q8T_SCALE_OFF 2048
// weight types (ggml's type ids)
enum { WT_Q4_0 = 2, WT_Q8_0 = 8 };
__host__ __device__ static inline int wt_tile_bytes(int wt) { return wt == WT_Q8_0 ? Q8T_BYTES : Q4T_BYTES; }

// ---- Q6_K weights in HBM (csrc/q6k.hip): tiles of 32 rows x one 256-element block, 6720 bytes (= 32 x 210) --------
#define Q6T_ROWS 32
#define Q6T_BYTES 6720
#define Q6T_SCALE_OFF 6144
#define Q6T_D_OFF 6656
static inline size_t q6t_bytes(int N, int K) { return (size_t) ((N + 31) / 32) * (K / 256) * Q6T_BYTES; }

// ---- Q8_K activation records ("xk", the Q6_K matmul's operand): one 8320-byte record per (32-row tile, 256-block):
//   [G * 512, +512)  group G's fragment: lane l = m + 32 h holds row m's int8 q of elements 16 G + 8 h .. + 7;
//   [8192, +128)     the 32 rows' d (fp32, 1 / iscale of quantize_row_q8_K_ref).
// Row tiles are rounded up to an even count.
#define XK_REC 8320
#define XK_D_OFF 8192
__host__ __device__ static inline int xk_tiles(int M) { return (M + 63) / 64 * 2; }

// ---- activation operand ("xa"): Q8_0-quantized rows as fp16 MFMA fragments -----------------------------------------
// Rows are quantized to Q8_0 exactly as ggml's x86 CPU backend does (per 32-block: d = amax/127 stored fp16,
// q = round-half-even(x * 127/amax)). The operand is a sequence of records, one per (16-row tile mt, 4-block group c),
// tile-major: record (mt, c) starts at (mt * xa_ngroups(K) + c) * XA_REC. A record holds, for blocks 4c + bb:
//   [bb * 1024, +1024)   the fragment of block 4c + bb: lane l = m + 16 g holds row m's elements 4g..4g+3 as q and
//                        16+4g..16+4g+3 as q / 16 (8 fp16, all exact; the order of the weight tile lanes);
//   [4096 + bb * 64, +64) the 16 rows' scales d as fp32 (the fp16 value, exactly);
//   [4352 + bb * 64, +64) the 16 rows' corrections for Q4_0 weights, -(1032 * sum of q over elements 0..15 + 72 * sum
//                        over 16..31), an exact integer;
//   [4608 + bb * 64, +64) the 16 rows' corrections for Q8_0 weights, -1152 * sum of q over all 32 elements.
// The Q4_0 matmul unpacks a weight nibble w to fp16 (1024 + w) for elements 0..15 and (1024 + 16 w) for 16..31; an fp16
// MFMA of a fragment against them, with the Q4_0 correction as its C input, is sum q (w - 8), ggml's integer block sum
// (vec_dot_q4_0_q8_0), exactly: every term and every partial sum is an integer below 2^23 in magnitude. The Q8_0
// matmul unpacks a weight byte w (int8) to fp16 (1024 + (w + 128)) for elements 0..15 and 16 (1024 + (w + 128)) for
// 16..31; with the Q8_0 correction the MFMA is sum q w (vec_dot_q8_0_q8_0), exactly in the same way.
// Row tiles are rounded up to an even count and blocks to whole groups; padding blocks are zero.
#define XA_REC 4864
#define XA_DX_OFF 4096
#define XA_CORR_OFF 4352
#define XA_CORR8_OFF 4608

__host__ __device__ static inline int xa_nbp(int K) { return (K / 32 + 3) / 4 * 4; }
__host__ __device__ static inline int xa_ngroups(int K) { return (K / 32 + 3) / 4; }
__host__ __device__ static inline int xa_mtp(int M) { return (M + 31) / 32 * 2; }
// the record holding row m, block b
__host__ __device__ static inline size_t xa_rec_off(int K, int m, int b) {
    return ((size_t) (m >> 4) * xa_ngroups(K) + (b >> 2)) * XA_REC;
}
__host__ __device__ static inline size_t xa_bytes(int M, int K) { return (size_t) xa_mtp(M) * xa_ngroups(K) * XA_REC; }
__host__ __device__ static inline size_t xk_rec_off(int K, int m, int b) {
    return ((size_t) (m >> 5) * (K / 256) + b) * XK_REC;
}
__host__ __device__ static inline size_t xk_bytes(int M, int K) { return (size_t) xk_tiles(M) * (K / 256) * XK_REC; }
static inline size_t q4t_bytes(int N, int K) { return (size_t) ((N + 15) / 16) * ((K / 32 + 3) / 4) * Q4T_BYTES; }
// bytes of an N x K matrix of weight type wt in the tile layout
static inline size_t wt_bytes(int wt, int N, int K) {
    return (size_t) ((N + 15) / 16) * ((K / 32 + 3) / 4) * wt_tile_bytes(wt);
}

// The sum, in slice order, of ks <= KM k-slices of a matmul (slice k at p + k * stride). Every load is issued before
// any is used (the slice index is clamped, so no load sits behind a branch); the slices past ks are not added.
#define KS_MAX 16
#define MOE_MAX_K 8  // experts used per row
#define MOE_ROUTE_EMAX 4096  // the widest rows (E) of the one-launch routing
// The 64-bit counters by which one launch's workgroups hand work on sit CNT_STRIDE apart (256 bytes): counters that
// share a line serialise each other's atomics (the routing's 8 row blocks of 32 arrivals: 2.6 us for the last
// arrival's atomic with adjacent counters).
#define CNT_STRIDE 32
template <int KM>
__device__ __forceinline__ float4 slices_sum4(const float* p, size_t stride, int ks) {
    float4 v[KM];
    for (int k = 0; k < KM; ++k) v[k] = *(const float4*) (p + (size_t) (k < ks ? k : ks - 1) * stride);
    float4 s = v[0];
    for (int k = 1; k < KM; ++k)
        if (k < ks) s = (float4){s.x + v[k].x, s.y + v[k].y, s.z + v[k].z, s.w + v[k].w};
    return s;
}
template <int KM>
__device__ __forceinline__ float slices_sum1(const float* p, size_t stride, int ks) {
    float v[KM];
    for (int k = 0; k < KM; ++k) v[k] = p[(size_t) (k < ks ? k : ks - 1) * stride];
    float s = v[0];
    for (int k = 1; k < KM; ++k)
        if (k < ks) s += v[k];
    return s;
}
// the smallest slice bound of the kernels' instances that holds ks (0: ks out of range)
static inline int ks_bound(int ks) {
    return ks < 1 ? 0 : ks == 1 ? 1 : ks <= 2 ? 2 : ks <= 4 ? 4 : ks <= 8 ? 8 : ks <= KS_MAX ? 16 : 0;
}
