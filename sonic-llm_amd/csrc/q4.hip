// Q4_0 x Q8_0 matmul for gfx950: Y[m][n] (+)= sum_k X[m][k] W[n][k].
//
// Replaces the reference's Q4_0 mat-vec / few-row / block matmuls (kernels.metal:1324-1411 mv_q4_0_*, :1413-1490
// mvm_q4_0_*, :746-1007 qmm_ks/qmmh_ks_q4_0_*, dispatched by mm() in core_mm.inc.h:307-325), with ggml's CPU numerics
// (Q8_0-quantized activations, integer block sums scaled by dw*dx) instead of the reference's fp16 weights.
//
// How a block's sum is formed: the activation operand holds the Q8_0 integers q as fp16 (exact; q / 16 for the
// elements that pair with high nibbles), the weights are unpacked to fp16 (1024 + w) or (1024 + 16 w), and
// v_mfma_f32_16x16x32_f16 multiplies exactly and accumulates in fp32 with a per-row integer correction as its C input;
// every partial sum is an integer below 2^23, so the MFMA gives ggml's integer block sum isum = sum q (w - 8) exactly.
// One fma per output then adds isum * (dw * dx) (the product of two fp16 values is exact in fp32) to the fp32
// accumulator; the products dw * dx come from a 4 x 4 x 4 fp16 MFMA as well (scale_products), exactly as the VALU
// would form them. The order of the sums of an output is fixed by (N, K) alone, never by the number of rows, so a row's
// result is the same in any step (sn.h:1-3).
#include <stdarg.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "sn_kernels_internal.h"
#include "sn_rows.h"

// ---------------------------------------------------------------------------------------------------------------------
// weight upload: GGUF rows -> stripes (sn_common.h)
// Source stripe s goes to destination stripe s * sstride + soff (sstride 2 interleaves a gate and an up matrix).
__global__ void k_q4_repack(const uint8_t* __restrict__ src, int N, int K, uint8_t* __restrict__ dst, int sstride,
                            int soff) {
    const int nb = K / 32, ngroups = (nb + 3) / 4;
    const int tile = blockIdx.x;  // (stripe, group)
    const int stripe = tile / ngroups, grp = tile % ngroups;
    const int l = threadIdx.x, n = l & 15, g = l >> 4;
    const int row = stripe * 16 + n;
    uint8_t* t = dst + ((size_t) (stripe * sstride + soff) * ngroups + grp) * Q4T_BYTES;
    uint8_t q[16];
    uint16_t d[4];
    for (int b = 0; b < 4; ++b) {
        const int blk = grp * 4 + b;
        const bool ok = row < N && blk < nb;
        const uint8_t* s = src + ((size_t) row * nb + blk) * 18;
        for (int j = 0; j < 4; ++j) q[4 * b + j] = ok ? s[2 + 4 * g + (j == 1 ? 2 : j == 2 ? 1 : j)] : 0;
        d[b] = ok ? (uint16_t) (s[0] | (s[1] << 8)) : 0;
    }
    for (int j = 0; j < 16; ++j) t[16 * l + j] = q[j];
    if (g == 0)
        for (int b = 0; b < 4; ++b) {
            t[Q4T_SCALE_OFF + 8 * n + 2 * b] = (uint8_t) d[b];
            t[Q4T_SCALE_OFF + 8 * n + 2 * b + 1] = (uint8_t) (d[b] >> 8);
        }
}

// GGUF Q8_0 rows (34-byte blocks) -> Q8_0 tiles (sn_common.h); stripe s goes to s * sstride + soff.
__global__ void k_q8_repack(const uint8_t* __restrict__ src, int N, int K, uint8_t* __restrict__ dst, int sstride,
                            int soff) {
    const int nb = K / 32, ngroups = (nb + 3) / 4;
    const int tile = blockIdx.x;
    const int stripe = tile / ngroups, grp = tile % ngroups;
    const int l = threadIdx.x, n = l & 15, g = l >> 4;
    const int row = stripe * 16 + n;
    uint8_t* t = dst + ((size_t) (stripe * sstride + soff) * ngroups + grp) * Q8T_BYTES;
    uint8_t q[32];
    uint16_t d[4];
    for (int b = 0; b < 4; ++b) {
        const int blk = grp * 4 + b;
        const bool ok = row < N && blk < nb;
        const uint8_t* s = src + ((size_t) row * nb + blk) * 34;
        for (int j = 0; j < 4; ++j) {
            q[8 * b + j] = ok ? s[2 + 4 * g + j] : 0;
            q[8 * b + 4 + j] = ok ? s[2 + 16 + 4 * g + j] : 0;
        }
        d[b] = ok ? (uint16_t) (s[0] | (s[1] << 8)) : 0;
    }
    for (int j = 0; j < 32; ++j) t[32 * l + j] = q[j];
    if (g == 0)
        for (int b = 0; b < 4; ++b) {
            t[Q8T_SCALE_OFF + 8 * n + 2 * b] = (uint8_t) d[b];
            t[Q8T_SCALE_OFF + 8 * n + 2 * b + 1] = (uint8_t) (d[b] >> 8);
        }
}

// ---------------------------------------------------------------------------------------------------------------------
// activation quantizer: fp32 rows (optionally RMS-normed by weight nw first) -> xa operand (sn_common.h).
// One workgroup of 256 threads per row. The norm is ggml's: y = (x * scale) * w, scale = 1/sqrt(mean(x^2) + eps).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float block_reduce_sum256(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ void q8_store(const float* v, int g, uint8_t* xa, int K, int m, int b);
__device__ __forceinline__ void q8_zero(int g, uint8_t* xa, int K, int m, int b);

// Four lanes per 32-block: lane part g holds the block's elements {4g..4g+3, 16+4g..16+4g+3}, which is exactly its
// 8-value fragment of the MFMA operand, so each lane writes one 16-byte hi and one 16-byte lo fragment. The block's
// amax is a max over the 4 lanes. Workgroup (row m, block group y): 64 blocks; with a norm weight every workgroup of
// the row first sums the row's squares (the row is read from L2 once per workgroup).
__global__ __launch_bounds__(256) void k_quant_act(const float* __restrict__ X, const int32_t* __restrict__ rows,
                                                   int M, int K, int ldx, const float* __restrict__ nw, float eps,
                                                   uint8_t* __restrict__ xa, float* __restrict__ xn, int ldn) {
    __shared__ float red[4];
    const int m = blockIdx.x, nb = K / 32, t = threadIdx.x;
    const int src = rows ? rows[m] : m;
    // padding of an expert's tile: not written. A row of an MFMA product depends on that row of the operand alone, so
    // whatever the row holds reaches only output rows that nothing reads.
    if (src < 0) return;
    const float* x = X + (size_t) src * ldx;
    float scale = 1.0f;
    if (nw) {
        float s = 0.0f;
        for (int i = t; i < K; i += 256) s += x[i] * x[i];
        s = block_reduce_sum256(s, red);
        scale = 1.0f / sqrtf(s / (float) K + eps);
    }
    const int nbp = xa_nbp(K);
    const int b = blockIdx.y * 64 + (t >> 2), g = t & 3;
    if (b >= nbp) return;  // (whole 4-lane groups leave together: the shuffles below stay within a group)
    if (b >= nb) {  // a padding block of the last 4-block group: zero
        q8_zero(g, xa, K, m, b);
        return;
    }
    const float4 lo4 = *(const float4*) (x + 32 * b + 4 * g), hi4 = *(const float4*) (x + 32 * b + 16 + 4 * g);
    float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
    if (nw) {
        const float4 wl = *(const float4*) (nw + 32 * b + 4 * g), wh = *(const float4*) (nw + 32 * b + 16 + 4 * g);
        const float w[8] = {wl.x, wl.y, wl.z, wl.w, wh.x, wh.y, wh.z, wh.w};
        for (int j = 0; j < 8; ++j) v[j] = (v[j] * scale) * w[j];
    }
    if (xn) {
        float* o = xn + (size_t) m * ldn + 32 * b;
        *(float4*) (o + 4 * g) = (float4){v[0], v[1], v[2], v[3]};
        *(float4*) (o + 16 + 4 * g) = (float4){v[4], v[5], v[6], v[7]};
    }
    q8_store(v, g, xa, K, m, b);
}

// Row m, block b of a Q8_0 operand from its 32 fp32 values (this lane's 8: elements 4g..4g+3, 16+4g..16+4g+3):
// ggml x86 quantize_row_q8_0, d = amax / 127 (stored fp16), q = round-half-even(x * 127 / amax). The 4 lanes of a
// block are adjacent (the shuffles stay within them). Writes the lane's fragment slice (q, and q / 16 for elements
// 16..31) and, from lane part 0, the block's scale and corrections (see sn_common.h).
__device__ __forceinline__ void q8_store(const float* v, int g, uint8_t* xa, int K, int m, int b) {
    float amax = 0.0f;
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float d = amax / 127.f;
    const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    half8 q;
    float slo = 0.0f, shi = 0.0f;  // integer sums (exact in fp32)
    for (int j = 0; j < 8; ++j) {
        const float r = __builtin_rintf(v[j] * id);
        q[j] = (_Float16) (j < 4 ? r : r * 0.0625f);
        if (j < 4) slo += r;
        else shi += r;
    }
    slo += __shfl_xor(slo, 1);
    shi += __shfl_xor(shi, 1);
    slo += __shfl_xor(slo, 2);
    shi += __shfl_xor(shi, 2);
    uint8_t* rec = xa + xa_rec_off(K, m, b);
    *(half8*) (rec + (b & 3) * 1024 + 16 * ((m & 15) + 16 * g)) = q;
    if (g == 0) {
        *(float*) (rec + XA_DX_OFF + (b & 3) * 64 + 4 * (m & 15)) = (float) (_Float16) d;
        *(float*) (rec + XA_CORR_OFF + (b & 3) * 64 + 4 * (m & 15)) = -(1032.0f * slo + 72.0f * shi);
        *(float*) (rec + XA_CORR8_OFF + (b & 3) * 64 + 4 * (m & 15)) = -1152.0f * (slo + shi);
    }
}

// a zero block (padding, or a zero row of an expert's tile)
__device__ __forceinline__ void q8_zero(int g, uint8_t* xa, int K, int m, int b) {
    uint8_t* rec = xa + xa_rec_off(K, m, b);
    *(half8*) (rec + (b & 3) * 1024 + 16 * ((m & 15) + 16 * g)) = (half8){};
    if (g == 0) {
        *(float*) (rec + XA_DX_OFF + (b & 3) * 64 + 4 * (m & 15)) = 0.0f;
        *(float*) (rec + XA_CORR_OFF + (b & 3) * 64 + 4 * (m & 15)) = 0.0f;
        *(float*) (rec + XA_CORR8_OFF + (b & 3) * 64 + 4 * (m & 15)) = 0.0f;
    }
}

__device__ __forceinline__ float4 ld4(const float* p) { return *(const float4*) p; }
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return (float4){a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w}; }

// the workgroup's sum of v, the wavefronts' sums added in wavefront order (at most 16 wavefronts)
__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
    for (int w = 1; w < (int) (blockDim.x >> 6); ++w) s += red[w];
    return s;
}

// The MoE output of row m at elements e .. e + 3: the weighted sum over its k slots of the expert rows y[prow[j]],
// accumulated from zero in slot order (moe_out, kernels.metal:3520-3538; sn_layers.inc.h:129-144)
__device__ __forceinline__ float4 pairs_sum4(const float* y, const int32_t* prow, const float* w, int k, int K, int e) {
    float4 v[MOE_MAX_K];
    float wv[MOE_MAX_K];
    for (int j = 0; j < MOE_MAX_K; ++j)
        if (j < k) {
            wv[j] = w[j];
            v[j] = ld4(y + (size_t) prow[j] * K + e);
        }
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < MOE_MAX_K; ++j)
        if (j < k) {
            acc.x += wv[j] * v[j].x;
            acc.y += wv[j] * v[j].y;
            acc.z += wv[j] * v[j].z;
            acc.w += wv[j] * v[j].w;
        }
    return acc;
}

// The next matmul's first weight groups read by extra workgroups of a row kernel, whose own work leaves HBM idle, so
// that the matmul finds them in the Infinity Cache: for every stripe s and k-slice y of the next matrix, the bytes
// [s sbytes + y gstep, + len) (the groups its workgroups load first), in 128-byte lines, WP_LINES a thread with every
// load in flight (a line past the ranges is an out-of-range buffer load: no access).
#define WP_LINES 4
struct WeightPrefetch {
    const uint8_t* w;
    int nranges, ks, sbytes, gstep, lines;  // ranges = stripes x ks, lines of 128 bytes a range
    uint32_t total;                         // the matrix's bytes
};
__device__ __forceinline__ void weight_prefetch(const WeightPrefetch& pf, int wg, int nwg) {
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(pf.w, pf.total);
    const int nl = pf.nranges * pf.lines;
    uint32_t v[WP_LINES];
    for (int k = 0; k < WP_LINES; ++k) {
        const int L = (k * nwg + wg) * (int) blockDim.x + (int) threadIdx.x;
        const int i = L / pf.lines, ln = L % pf.lines;
        const uint32_t off = L < nl ? (uint32_t) (i / pf.ks) * pf.sbytes + (uint32_t) (i % pf.ks) * pf.gstep + 128u * ln
                                    : pf.total;
        v[k] = __builtin_amdgcn_raw_buffer_load_b32(r, (int) off, 0, 0);
    }
    for (int k = 0; k < WP_LINES; ++k) asm volatile("" ::"v"(v[k]));
}

// Residual rows: x[m] += the k-slice sums of a matmul (part[ks][M][K], slices added in order; add 0: x[m] = the
// sums), or with PAIRS the MoE output (pairs_sum4 over part = the grouped down matmul's rows), written back; then,
// when xa is given, the RMSNorm (weight nw) and Q8_0 operand of the new row. One workgroup per row (the norm needs the
// whole row before any value is quantized), 4 lanes per 32-block: lane t covers blocks t / 4 + (blockDim / 4) i,
// i < IT. Every load (residual, slices, norm weight) is issued before the row's reduction.
template <int IT, int KM, bool PAIRS = false>
__global__ __launch_bounds__(1024) void k_resid_quant(float* __restrict__ X, const float* __restrict__ part, int ks,
                                                      int M, int K, const float* __restrict__ nw, float eps,
                                                      uint8_t* __restrict__ xa, int add, float* __restrict__ xn,
                                                      const int32_t* __restrict__ prow = nullptr,
                                                      const float* __restrict__ pw = nullptr, WeightPrefetch pf = {}) {
    if ((int) blockIdx.x >= M) {  // a prefetch workgroup (WeightPrefetch)
        weight_prefetch(pf, (int) blockIdx.x - M, (int) gridDim.x - M);
        return;
    }
    __shared__ float red[16];
    const int m = blockIdx.x, t = threadIdx.x, g = t & 3, bstep = blockDim.x >> 2;
    const int nb = K / 32, nbp = xa_nbp(K);
    float* x = X + (size_t) m * K;
    float v[IT][8], w[IT][8];
    float ss = 0.0f;
    for (int it = 0; it < IT; ++it) {
        const int b = t / 4 + bstep * it;
        if (b >= nb) continue;
        const int e0 = 32 * b + 4 * g, e1 = e0 + 16;
        if (xa && nw) {
            const float4 wl = ld4(nw + e0), wh = ld4(nw + e1);
            const float w8[8] = {wl.x, wl.y, wl.z, wl.w, wh.x, wh.y, wh.z, wh.w};
            for (int j = 0; j < 8; ++j) w[it][j] = w8[j];
        }
        float4 lo = add ? ld4(x + e0) : (float4){0.f, 0.f, 0.f, 0.f}, hi = add ? ld4(x + e1) : (float4){0.f, 0.f, 0.f, 0.f};
        const float4 slo = PAIRS ? pairs_sum4(part, prow + (size_t) m * ks, pw + (size_t) m * ks, ks, K, e0)
                                 : slices_sum4<KM>(part + (size_t) m * K + e0, (size_t) M * K, ks);
        const float4 shi = PAIRS ? pairs_sum4(part, prow + (size_t) m * ks, pw + (size_t) m * ks, ks, K, e1)
                                 : slices_sum4<KM>(part + (size_t) m * K + e1, (size_t) M * K, ks);
        lo = add4(lo, slo);
        hi = add4(hi, shi);
        *(float4*) (x + e0) = lo;
        *(float4*) (x + e1) = hi;
        const float r8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        for (int j = 0; j < 8; ++j) {
            v[it][j] = r8[j];
            ss += r8[j] * r8[j];
        }
    }
    if (!xa) return;
    const float scale = nw ? 1.0f / sqrtf(block_reduce_sum(ss, red) / (float) K + eps) : 1.0f;
    for (int it = 0; it < IT; ++it) {
        const int b = t / 4 + bstep * it;
        if (b >= nbp) continue;
        if (b >= nb) {  // a padding block of the last 4-block group: zero
            q8_zero(g, xa, K, m, b);
            continue;
        }
        float y[8];
        if (nw) {
            for (int j = 0; j < 8; ++j) y[j] = (v[it][j] * scale) * w[it][j];
        } else {
            for (int j = 0; j < 8; ++j) y[j] = v[it][j];
        }
        if (xn) {  // the normed rows themselves (the MoE router's input)
            float* o = xn + (size_t) m * K + 32 * b;
            *(float4*) (o + 4 * g) = (float4){y[0], y[1], y[2], y[3]};
            *(float4*) (o + 16 + 4 * g) = (float4){y[4], y[5], y[6], y[7]};
        }
        q8_store(y, g, xa, K, m, b);
    }
}

// SwiGLU of a stripe-interleaved gate/up matmul's k-slice sums (part[ks][M][2F]: output column 16p + n is
// silu(column 32p + n) * column 32p + 16 + n), written as fp32 rows h (when given) and as the Q8_0 operand of the next
// matmul. Workgroup (row m, 64 blocks), 4 lanes per block as in k_quant_act. STAGE (many rows): the blocks' 4096
// consecutive sum columns are read 1 KB a wavefront instruction, their slices added, and staged in LDS with 4 floats
// of pad per block, so that the 4-lanes-per-block reads hit distinct banks (Qwen3-4B gate|up at 512 rows: 32 against
// 39 us); otherwise each lane reads its own columns (a wavefront instruction then covers 16 pieces of 64 bytes), the
// shorter path for a few rows (the quantizing kernels of a 32-row step: 0.81 against 0.87 ms with the staged form).
// Both add the slices of a column in slice order. rows (optional): rows m with rows[m] < 0 (padding of an expert's tile) are skipped, as in
// k_quant_act.
template <int KM, bool STAGE>
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ part, int ks, int M, int F,
                                                      float* __restrict__ h, uint8_t* __restrict__ xa,
                                                      const int32_t* __restrict__ rows) {
    __shared__ __attribute__((aligned(16))) float s_v[STAGE ? 64 * 68 : 4];
    const int m = blockIdx.x, t = threadIdx.x;
    if (rows && rows[m] < 0) return;  // the whole workgroup
    const int nb = F / 32, nbp = xa_nbp(F);
    const size_t N = 2 * (size_t) F;
    const int b0 = blockIdx.y * 64;
    if constexpr (STAGE) {
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * (t + 256 * j);  // column 64 b0 + c; a block's 64 columns end at 64 nb = 2F
            if (64 * b0 + c < 64 * nb) {
                const float4 v = slices_sum4<KM>(part + (size_t) m * N + 64 * (size_t) b0 + c, (size_t) M * N, ks);
                *(float4*) &s_v[(c / 64) * 68 + c % 64] = v;
            }
        }
        __syncthreads();
    }
    const int b = b0 + (t >> 2), g = t & 3;
    if (b >= nbp) return;  // (whole 4-lane groups leave together: q8_store's shuffles stay within a group)
    if (b >= nb) {
        q8_zero(g, xa, F, m, b);
        return;
    }
    // elements 32b + 4g + j (pair 2b) and 32b + 16 + 4g + j (pair 2b + 1): gate at 64b + 4g (+32), up 16 further
    float4 g0, u0, g1, u1;
    if constexpr (STAGE) {
        const float* sv = s_v + (t >> 2) * 68;
        g0 = *(const float4*) (sv + 4 * g), u0 = *(const float4*) (sv + 16 + 4 * g);
        g1 = *(const float4*) (sv + 32 + 4 * g), u1 = *(const float4*) (sv + 48 + 4 * g);
    } else {
        auto sum4 = [&](int c) { return slices_sum4<KM>(part + (size_t) m * N + c, (size_t) M * N, ks); };
        g0 = sum4(64 * b + 4 * g), u0 = sum4(64 * b + 16 + 4 * g);
        g1 = sum4(64 * b + 32 + 4 * g), u1 = sum4(64 * b + 48 + 4 * g);
    }
    float v[8] = {silu(g0.x) * u0.x, silu(g0.y) * u0.y, silu(g0.z) * u0.z, silu(g0.w) * u0.w,
                  silu(g1.x) * u1.x, silu(g1.y) * u1.y, silu(g1.z) * u1.z, silu(g1.w) * u1.w};
    if (h) {
        float* o = h + (size_t) m * F + 32 * b;
        *(float4*) (o + 4 * g) = (float4){v[0], v[1], v[2], v[3]};
        *(float4*) (o + 16 + 4 * g) = (float4){v[4], v[5], v[6], v[7]};
    }
    q8_store(v, g, xa, F, m, b);
}

// ---------------------------------------------------------------------------------------------------------------------
// the matmul

// A weight lane's 4 bytes of one block (elements e = 4g + i, i = 0..3: byte 0 holds i = 0, byte 1 i = 2, byte 2 i = 1,
// byte 3 i = 3, each with element e in its low nibble and e + 16 in its high nibble) as the MFMA operand in the lane
// order of the activation fragments: fp16 (1024 + w) for elements 4g..4g+3 and (1024 + 16 w) for 16+4g..16+4g+3
// (0x64 is the high byte of fp16 1024). Bytes 0 and 2 give elements i = 0, 1 by a mask and an OR each (v_and_or_b32),
// bytes 1 and 3 give i = 2, 3 by a byte permute that places them under 0x64 and a mask each: 5 instructions.
// (written as v_and_or_b32 with the mask in a scalar register and 0x64006400 in a vector one: left to the compiler, the
// two literals became a v_and_b32 and a v_or_b32, since a VOP3 instruction here takes no literal)
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t k) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(k));
    return r;
}
__device__ __forceinline__ half8 q4_unpack(uint32_t w) {
    const uint32_t p01 = and_or(w, 0x000F000Fu, 0x64006400u);  // elements 0, 1
    const uint32_t p45 = and_or(w, 0x00F000F0u, 0x64006400u);  // elements 16, 17 (x 16)
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);  // bytes 1, 3 under 0x64
    const uint32_t p23 = h & 0xFF0FFF0Fu, p67 = h & 0xFFF0FFF0u;
    return __builtin_bit_cast(half8, (u32x4){p01, p23, p45, p67});
}

// A Q8_0 weight lane's 8 bytes of one block (int8 q of elements 4g..4g+3 in w_lo, of 16+4g..16+4g+3 in w_hi) as the
// MFMA operand: fp16 (1024 + u) and 16 (1024 + u), u = q + 128 (the sign bit flipped), built by two xors and four byte
// permutes (0x64 and 0x74 are the high bytes of fp16 1024 and 16384; the latter's step is 16).
__device__ __forceinline__ half8 q8_unpack(uint32_t w_lo, uint32_t w_hi) {
    const uint32_t u0 = w_lo ^ 0x80808080u, u1 = w_hi ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x74747474u, u1, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x74747474u, u1, 0x04030402u);
    return __builtin_bit_cast(half8, (u32x4){p0, p1, p2, p3});
}

// The scale products dw * dx of a block on the matrix core, by v_mfma_f32_4x4x4_16b_f16: 16 independent 4 x 4 x 4
// products, lane l holding row l % 4 of block l / 4's A (4 k values), column l % 4 of its B (4 k values) and column
// l % 4 of its D (4 rows). For lane (n, g) that block is (g, n / 4): A = the one-hot dx of row 4 g + n % 4 of the row
// tile (dx_b in k slot b, zeros in the other 3; dx an fp16 value, exact in fp32), B = the 4 blocks' fp16 scales dw of
// stripe row n (the tile's scale word as loaded), so D = dx_b[4 g + v] * dw_b[n] for v = 0..3: the rows and column
// of the block's sums in the 16 x 16 MFMA's layout. Each result is one product of two fp16 values (exact in fp32)
// plus 3 terms 0 * dw (zero for finite scales), so it is the value the VALU would form, for 4 VALU multiplies less a
// (block, stripe, row tile).
__device__ __forceinline__ half4v scale_a(float dx, int b) {
    const uint32_t h = __builtin_bit_cast(uint32_t, b & 1 ? __builtin_amdgcn_cvt_pkrtz(0.0f, dx)
                                                          : __builtin_amdgcn_cvt_pkrtz(dx, 0.0f));
    return __builtin_bit_cast(half4v, b < 2 ? (u32x2){h, 0u} : (u32x2){0u, h});
}
__device__ __forceinline__ floatx4 scale_products(half4v a, u32x2 ws) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, __builtin_bit_cast(half4v, ws), (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0,
                                              0);
}

// One workgroup (4 wavefronts) owns a set of 4 S consecutive 16-row stripes (wavefront w: stripes S w .. S w + S - 1 of
// the set; S = 2, or 1 for narrow matrices), MT row tiles and a k-slice of consecutive 4-block groups, which the 4 wavefronts walk together. Per group:
//   - the activation records of the MT row tiles (MT x 4 KB of fragments, MT x 512 B of scales and corrections) are
//     loaded from global memory once per workgroup, each wavefront a quarter, into a register slot together with the
//     weights of the group before, and staged into an LDS double buffer one group ahead;
//   - each wavefront's S weight tiles go from global memory into a register slot; the ring has D = 2 slots, so the
//     loads of the next group are in flight while a group is summed.
// Every load is a buffer load with a per-lane offset and a wavefront-uniform (scalar) one, issued without a branch:
// groups past the slice repeat its last group and are added with scale 0; stripes past the matrix read as zero (the
// buffer's size stops them) and are not stored. Each block is one MFMA per (row tile, stripe) with the correction as
// its C input, then acc += isum * (dw * dx) (an exact product of two fp16 values), the arithmetic of ggml's
// vec_dot_q4_0_q8_0. Scheduling fences keep the loads of each ring slot in issue order, so the wait before a slot
// leaves the other slot's loads in flight.
//
// The kernel writes each slice's raw fp32 sums, part[slice][M][N]; whoever consumes them adds the slices in slice
// order (k_q4_reduce here; the row kernels of the step), so the order of every sum is fixed by (N, K) alone.
// FK (prompt rows, grid.y = 1): the workgroup walks every slice in turn, each summed into a fresh accumulator exactly
// as its own launch would (the same groups, an odd slice's extra group added with scale 0 as its own ring pads it),
// and adds the slices in slice order as the consumers do ((p0 + p1) + p2 ...), so part[0] holds, bit for bit, what
// the consumers would have made of the split launch's slices: they read it as one slice.
template <int WT, int MT, int S, bool FK, bool SW = false, bool GRP = false>
__device__ __forceinline__ void q4_gemm_ring(const GemmArgs& a) {
    constexpr int D = 2, FPW = MT;  // ring slots, fragments each wavefront stages
    // the loop below stages group i + 1 from register slot j (which holds group i's weights and group i + 1's records)
    // into LDS buffer j ^ 1 and sums group i from buffer j and slot j
    static_assert(D == 2, "the ring is indexed j ^ 1 over the two LDS buffers s_act / s_k");
    constexpr bool Q8 = WT == WT_Q8_0;
    constexpr int TB = Q8 ? Q8T_BYTES : Q4T_BYTES, SO = Q8 ? Q8T_SCALE_OFF : Q4T_SCALE_OFF;
    constexpr int NW = Q8 ? 2 : 1;                               // 16-byte weight loads per lane and tile
    constexpr int CORR = Q8 ? XA_CORR8_OFF : XA_CORR_OFF;         // the record's correction for this weight type
    __shared__ __attribute__((aligned(16))) uint8_t s_act[2][MT * 4][1024];
    __shared__ __attribute__((aligned(16))) float s_k[2][MT][2][64];  // [buffer][row tile][dx, corr][block * 16 + row]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_in = lane & 15, g = lane >> 4;
    const int set = blockIdx.x, slice = blockIdx.y;
    int mt0 = blockIdx.z * MT;
    const uint8_t* wbase = a.w;
    if constexpr (GRP) {  // grouped: this workgroup's (expert, row tile)
        if ((int) blockIdx.z >= *a.count) return;
        wbase = a.w + (size_t) a.items[2 * blockIdx.z] * a.wstride;
        mt0 = a.items[2 * blockIdx.z + 1];
    }
    mt0 = __builtin_amdgcn_readfirstlane(mt0);
    // groups c0 .. c0 + ng - 1 (ng >= 1). FK: every group (the slices hold an even number of groups, so the walk is
    // the groups in order, the last slice padded to an even count as its own launch pads it)
    const int c0 = FK ? 0 : slice * a.gps, ng = FK ? a.ngroups : min(a.gps, a.ngroups - c0);
    const int s0 = set * (4 * S) + wave * S;
    const int sbytes = a.ngroups * TB;  // one stripe
    // one resource for the whole matrix, the wavefront's stripes by scalar offsets (stripes past the matrix read as
    // zeros: the range check covers the scalar offset too)
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(wbase, (uint32_t) (a.nstripes * sbytes));
    // the scales (B of scale_products): a group past the slice (the ring's padding) reads zeros, so it adds nothing
    const int ws_off = SO + 8 * n_in;
    const int rstride = a.ngroups * XA_REC;  // between row tiles' records
    // the activation: the operand's records from row tile mt0 on; or, gathering (a.gsrc, one row tile), each lane's row
    // m = lane % 16 of the tile taken from row gsrc[16 mt0 + m] of a row-ordered operand of a.gM rows (a padding row,
    // gsrc < 0, reads as zeros: its offset is past the buffer). The per-lane offset of a row's piece of a record:
    // fragments 16 (row % 16 + 16 g), scales and corrections 4 (16 b + row % 16), b = lane / 16.
    size_t x0 = (size_t) mt0 * a.ngroups * XA_REC;
    uint32_t xbytes = (uint32_t) (xa_bytes(a.M, a.K) - x0);
    int vf_off = 16 * lane, vk_off = 4 * lane;
    if (GRP && a.gsrc) {
        const int sr = a.gsrc[16 * mt0 + (lane & 15)];
        x0 = 0;
        xbytes = (uint32_t) xa_bytes(a.gM, a.K);
        vf_off = sr < 0 ? (int) XA_GATHER_OOB : (sr >> 4) * rstride + 16 * ((sr & 15) + 16 * g);
        vk_off = sr < 0 ? (int) XA_GATHER_OOB : (sr >> 4) * rstride + 4 * (16 * g + (sr & 15));
    }
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(a.xa + x0, xbytes);
    // what this wavefront stages: fragments f = wave * FPW + j (row tile f / 4, block f % 4); constant block kb =
    // wave (row tile kb / 2; dx or corr) while kb < 2 MT
    const int kb = min(wave, 2 * MT - 1);

    u32x4 wq[D][S][NW];
    u32x2 ws[D][S];
    u32x4 ra[D][FPW];
    float rk[D];
    floatx4 acc[S][MT], tot[S][MT];
    for (int s = 0; s < S; ++s)
        for (int mt = 0; mt < MT; ++mt) acc[s][mt] = tot[s][mt] = (floatx4){0.f, 0.f, 0.f, 0.f};

    // a register slot holds the weights of group i and the activation records of group i + 1: the records are staged
    // into LDS an iteration before their group is summed, so loading them with the weights of the group before keeps
    // a whole iteration between their issue and that use
    auto load_act = [&](u32x4 (&r)[FPW], float& k, int i) {
        const int c = c0 + min(i, ng - 1);
        for (int j = 0; j < FPW; ++j) {
            const int f = wave * FPW + j;
            r[j] = bload16(xr, vf_off, (f / 4) * rstride + c * XA_REC + (f % 4) * 1024);
        }
        k = bload4f(xr, vk_off, (kb / 2) * rstride + c * XA_REC + (kb % 2 ? CORR : XA_DX_OFF));
    };
    auto load = [&](int slot, int i) {
        load_act(ra[slot], rk[slot], i + 1);
        const int c = c0 + min(i, ng - 1);
        for (int s = 0; s < S; ++s) {
            const int so = (s0 + s) * sbytes + c * TB;
            for (int h = 0; h < NW; ++h) wq[slot][s][h] = bload16(wr, 16 * NW * lane + 16 * h, so);
            ws[slot][s] = bload8(wr, ws_off, i < ng ? so : (int) XA_GATHER_OOB);
        }
    };
    auto stage = [&](int buf, const u32x4 (&r)[FPW], float k) {
        for (int j = 0; j < FPW; ++j) *(u32x4*) &s_act[buf][wave * FPW + j][16 * lane] = r[j];
        if (wave < 2 * MT) s_k[buf][kb / 2][kb % 2][lane] = k;
    };
    auto compute = [&](int slot, int buf) {
        for (int b = 0; b < 4; ++b) {
            half8 A[MT];
            half4v da[MT];
            floatx4 cr[MT];
            for (int mt = 0; mt < MT; ++mt) {
                A[mt] = *(const half8*) &s_act[buf][mt * 4 + b][16 * lane];
                da[mt] = scale_a(s_k[buf][mt][0][b * 16 + 4 * g + (n_in & 3)], b);
                cr[mt] = *(const floatx4*) &s_k[buf][mt][1][b * 16 + 4 * g];
            }
            for (int s = 0; s < S; ++s) {
                const half8 bw = Q8 ? q8_unpack(wq[slot][s][b / 2][2 * (b % 2)], wq[slot][s][b / 2][2 * (b % 2) + 1])
                                    : q4_unpack(wq[slot][s][0][b]);
                for (int mt = 0; mt < MT; ++mt) {
                    const floatx4 isum = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], bw, cr[mt], 0, 0, 0);
                    const floatx4 sc = scale_products(da[mt], ws[slot][s]);
                    for (int v = 0; v < 4; ++v) acc[s][mt][v] = __builtin_fmaf(isum[v], sc[v], acc[s][mt][v]);
                }
            }
        }
    };

    {
        u32x4 r0[FPW];
        float k0;
        load_act(r0, k0, 0);
        __builtin_amdgcn_sched_barrier(0);
        for (int j = 0; j < D; ++j) {
            load(j, j);
            __builtin_amdgcn_sched_barrier(0);
        }
        stage(0, r0, k0);
    }
    asm volatile("" ::"s"(a.part), "s"(a.N));  // (the tail's arguments read behind the first loads, as k_q4_gemm_s)
    const int trips = (ng + D - 1) / D;
    int in_slice = 0;  // FK: groups of the current slice summed so far
    bool first = true;
    for (int t = 0; t < trips; ++t)
        for (int j = 0; j < D; ++j) {
            const int i = t * D + j;
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();  // group i is staged in buffer j; everyone is done reading buffer j ^ 1
            stage(j ^ 1, ra[j], rk[j]);  // group i + 1's records (loaded with group i's weights, slot i % D)
            __builtin_amdgcn_sched_barrier(0);
            compute(j, j);
            // the group's sums are complete here: left to the compiler, they sank below the next loads, which then
            // could not reuse the slot's scale registers, and the copy back at the loop's end waited on those loads
            for (int s = 0; s < S; ++s)
                for (int mt = 0; mt < MT; ++mt) asm volatile("" : "+v"(acc[s][mt]));
            if constexpr (FK) {
                if (++in_slice == a.gps || i == D * trips - 1) {  // the slice's last group: add the slice on
                    in_slice = 0;
                    for (int s = 0; s < S; ++s)
                        for (int mt = 0; mt < MT; ++mt) {
                            if (first) tot[s][mt] = acc[s][mt];
                            else
                                for (int v = 0; v < 4; ++v) tot[s][mt][v] = tot[s][mt][v] + acc[s][mt][v];
                            acc[s][mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
                        }
                    first = false;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            load(j, i + D);
        }
    if constexpr (FK)
        for (int s = 0; s < S; ++s)
            for (int mt = 0; mt < MT; ++mt) acc[s][mt] = tot[s][mt];

    if constexpr (SW) {
        // SwiGLU of the tiles, as k_swiglu_quant makes it of the slices (the same sums: silu(gate) * up, Q8_0 blocks of
        // 32 F columns): wavefront w's stripes are gate and up of F columns 64 set + 16 w .. + 15; the workgroup's 2 x 16
        // rows x 64 columns go through LDS to threads (row, block of 32, lane part) for the quantizer
        static_assert(FK && S == 2 && MT == 2, "the SwiGLU epilogue takes the FK walk with gate and up a wavefront");
        __shared__ float s_h[32][64 + 4];
        for (int mt = 0; mt < MT; ++mt)
            for (int v = 0; v < 4; ++v) s_h[16 * mt + 4 * g + v][16 * wave + n_in] = silu(acc[0][mt][v]) * acc[1][mt][v];
        __syncthreads();
        const int t = threadIdx.x, r = t >> 3, blk = (t >> 2) & 1, gq = t & 3;
        const int row = mt0 * 16 + r, F = a.N / 2, b = 2 * set + blk;
        float v8[8];
        for (int j = 0; j < 4; ++j) {
            v8[j] = s_h[r][32 * blk + 4 * gq + j];
            v8[4 + j] = s_h[r][32 * blk + 16 + 4 * gq + j];
        }
        if (row >= a.M || 32 * b >= F) return;  // (a block's 4 lane parts share the row and block: q8_store's shuffles)
        float* o = a.h + (size_t) row * F + 32 * b;
        *(float4*) (o + 4 * gq) = (float4){v8[0], v8[1], v8[2], v8[3]};
        *(float4*) (o + 16 + 4 * gq) = (float4){v8[4], v8[5], v8[6], v8[7]};
        q8_store(v8, gq, a.xo, F, row, b);
        return;
    }

    // lane (n, g) holds rows 4g + v of each row tile, column n of each of its stripes
    for (int s = 0; s < S; ++s) {
        const int stripe = s0 + s, col = stripe * 16 + n_in;
        if (stripe >= a.nstripes || col >= a.N) continue;
        for (int mt = 0; mt < MT; ++mt)
            for (int v = 0; v < 4; ++v) {
                const int row = (mt0 + mt) * 16 + 4 * g + v;
                if (row < a.M && (!GRP || !a.rmask || a.rmask[row] >= 0))
                    a.part[((size_t) slice * a.M + row) * a.N + col] = acc[s][mt][v];
            }
    }
}

// GRP: grouped (expert items, gathered rows, row masks); compiled out of the other launches
// The kernels' hot arguments come first as scalars, which the hardware preloads into SGPRs at wavefront start
// (-amdgpu-kernarg-preload-count): a workgroup issues its first loads without waiting for the argument block; the rest
// of GemmArgs is read from it as before. A launch passes GS_ARGS(a).
// (14 dwords are preloaded: those a workgroup needs before its first loads come first; part, read at the end, last)
#define GS_PARAMS                                                                                                   \
    const uint8_t *w_, const uint8_t *xa_, int M_, int K_, int nstripes_, int ngroups_, int gps_,                   \
        const int32_t *pos_, const int32_t *seq_, int N_, float *part_, GemmArgs a
// (grouped launches, GRP: the item list and its count in the slots of pos and seq, GSG_ARGS)
#define GS_TAKE()                                                                                                   \
    a.w = w_, a.xa = xa_, a.part = part_, a.M = M_, a.N = N_, a.K = K_, a.nstripes = nstripes_,                     \
    a.ngroups = ngroups_, a.gps = gps_;                                                                              \
    if constexpr (GRP) a.items = pos_, a.count = seq_;                                                               \
    else a.pos = pos_, a.seq = seq_
#define GS_ARGS(a) (a).w, (a).xa, (a).M, (a).K, (a).nstripes, (a).ngroups, (a).gps, (a).pos, (a).seq, (a).N, (a).part, (a)
#define GSG_ARGS(a) (a).w, (a).xa, (a).M, (a).K, (a).nstripes, (a).ngroups, (a).gps, (a).items, (a).count, (a).N, (a).part, (a)
template <int WT, int MT, int S, bool FK = false, bool GRP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8))) void k_q4_gemm(GS_PARAMS) {
    GS_TAKE();
    q4_gemm_ring<WT, MT, S, FK, false, GRP>(a);
}
// the FK walk with two stripes a wavefront (prompt rows of the wide matrices): its accumulators and slice sums need
// more than the 168 registers of 3 wavefronts a SIMD. SW: the gate|up matrix's SwiGLU + Q8_0 as its epilogue
template <int WT, int MT, int S, bool SW = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_q4_gemm_fk2(GS_PARAMS) {
    constexpr bool GRP = false;
    GS_TAKE();
    q4_gemm_ring<WT, MT, S, true, SW>(a);
}

// A k-slice sum of the workspace, read by the set's last workgroup from the XCD's L2, where the set's other
// workgroups' stores are (the workgroup has dropped its L1 lines first: l1_drop)
__device__ __forceinline__ float4 part_load4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 1));
}
__device__ __forceinline__ float part_load1(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 1));
}

// The fused epilogue of set `set`, row tiles mt0 .. mt0 + MT - 1, run by the set's last workgroup once every slice's
// sums are in the workspace: the slices of each value added in slice order ((p0 + p1) + p2 ...), as slices_sum4 and
// slices_sum1 add them for the row kernels, then the row kernel's own arithmetic.
//   FE_SWIGLU: the set's 4 S stripes are S Q8_0 blocks of F = N / 2 SwiGLU columns (the gate|up matrix interleaved
//              stripe by stripe): k_swiglu_quant's silu(gate) * up and q8_store, 4 lanes a block (thread: row, block,
//              lane part), into a.h (fp32 rows, when given) and the operand a.xo;
//   FE_ROPE:   the set's 8 stripes are head `set` (128 columns): wavefront w takes rows w, w + 4, ..., lane i the dims
//              (i, i + 64), and qk_head norms, rotates and writes q to a.qkv, k and v to the row's cell (and k, v as
//              summed to a.qkv), as k_qk_rope does.
// (FE_ROPE) the epilogue's row data, loaded by every workgroup while its slice streams (the set's last workgroup is
// known only at the end). Wavefront w of the row tiles mt0 .. mt0 + MT - 1 owns rows mt0 16 + 4 MT w + j, j < 4 MT;
// lane j holds row j's position and page (lanes past the rows, and rows past M, hold row M - 1's), and cs[j] row j's
// rotation of this lane. pos and seq are loaded before the activation is staged, the page entry and the rotation
// after it, so none of them is waited for before the epilogue.
template <int MT>
struct RopeRows {
    int pos, page;
    float2 cs[4 * MT];
};
template <int MT>
__device__ __forceinline__ void rope_rows_begin(const GemmArgs& a, int mt0, int wave, int lane, RopeRows<MT>& rr) {
    const int row = min(mt0 * 16 + 4 * MT * wave + min(lane, 4 * MT - 1), a.M - 1);
    rr.pos = __builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(a.pos, (uint32_t) a.M * 4), row * 4, 0, 0);
    rr.page = __builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(a.seq, (uint32_t) a.M * 4), row * 4, 0, 0);  // (the slot)
}
template <int MT>
__device__ __forceinline__ void rope_rows_end(const GemmArgs& a, int set, int mt0, int wave, int lane, RopeRows<MT>& rr) {
    rr.page = __builtin_amdgcn_raw_buffer_load_b32(
        buf_rsrc(a.pt, 0xfffffff0u), (int) (((size_t) rr.page * a.max_pages + rr.pos / a.page_cells) * 4), 0, 0);
    if (a.rope_cs && set < a.H + a.KVH) {  // (v heads are not rotated)
#pragma unroll
        for (int j = 0; j < 4 * MT; ++j) {
            const int row = min(mt0 * 16 + 4 * MT * wave + j, a.M - 1);
            rr.cs[j] = a.rope_cs[(size_t) row * 64 + lane];
        }
    }
}

template <int FE, int MT, int S, class RR>
__device__ __forceinline__ void q4_epilogue(const GemmArgs& a, int set, int mt0, const RR& rr) {
    const int ks = (int) gridDim.y;
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(a.part, (uint32_t) ((size_t) ks * a.M * a.N * sizeof(float)));
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int KM = fe_slice_bound(FE & 7);  // the slices' bound: every slice's values loaded at once (the index
                                                // clamped, so no load sits behind a branch; slices past ks not added)
    if constexpr (FE >= FE_SWIGLU && FE < FE_ROPE) {
        const int F = a.N / 2;
        for (int it = threadIdx.x; it < 16 * MT * S * 4; it += 256) {
            const int r = it / (4 * S), blk = (it >> 2) % S, g = it & 3;
            const int row = mt0 * 16 + r, b = set * S + blk;
            if (row >= a.M || 32 * b >= F) continue;  // (a block's 4 lane parts together: q8_store's shuffles)
            float4 pv[4][KM];
            for (int q = 0; q < 4; ++q)  // gate, up of pair 2b; gate, up of pair 2b + 1
                for (int k = 0; k < KM; ++k)
                    pv[q][k] = part_load4(pr, (row * a.N + 64 * b + 16 * q + 4 * g) * 4 + min(k, ks - 1) * a.M * a.N * 4);
            float4 v4[4];
            for (int q = 0; q < 4; ++q) {
                float4 acc = pv[q][0];
                for (int k = 1; k < KM; ++k)
                    if (k < ks) acc = (float4){acc.x + pv[q][k].x, acc.y + pv[q][k].y, acc.z + pv[q][k].z, acc.w + pv[q][k].w};
                v4[q] = acc;
            }
            const float4 g0 = v4[0], u0 = v4[1], g1 = v4[2], u1 = v4[3];
            float v[8] = {silu(g0.x) * u0.x, silu(g0.y) * u0.y, silu(g0.z) * u0.z, silu(g0.w) * u0.w,
                          silu(g1.x) * u1.x, silu(g1.y) * u1.y, silu(g1.z) * u1.z, silu(g1.w) * u1.w};
            if (a.h) {
                float* o = a.h + (size_t) row * F + 32 * b;
                *(float4*) (o + 4 * g) = (float4){v[0], v[1], v[2], v[3]};
                *(float4*) (o + 16 + 4 * g) = (float4){v[4], v[5], v[6], v[7]};
            }
            q8_store(v, g, a.xo, F, row, b);
        }
    } else if constexpr (FE >= FE_ROPE && FE < FE_GSWIGLU) {
        // every row of the wavefront (4 MT) in one round of loads: the k-slice sums (the rows' positions, pages and
        // rotations are already in registers, RopeRows)
        constexpr int RN = 4 * MT;
        static_assert(S == 2, "a head is the 8 stripes of a set");
        const int h = set, H = a.H, KVH = a.KVH;
        const bool isq = h < H, isv = h >= H + KVH;
        const float* w = isq ? a.qw : a.kw;
        const float w0 = isv ? 0.0f : w[lane], w1 = isv ? 0.0f : w[lane + 64];
        const int r0 = mt0 * 16 + RN * wave;
        float x0[RN][KM], x1[RN][KM];
#pragma unroll
        for (int j = 0; j < RN; ++j) {
            const int row = min(r0 + j, a.M - 1);  // (past M: the last row again, not written)
            const int off = (row * a.N + h * 128 + lane) * 4;
#pragma unroll
            for (int k = 0; k < KM; ++k) {
                const int o = off + min(k, ks - 1) * a.M * a.N * 4;
                x0[j][k] = part_load1(pr, o);
                x1[j][k] = part_load1(pr, o + 256);
            }
        }
#pragma unroll
        for (int j = 0; j < RN; ++j) {
            const int row = r0 + j;
            float v0 = x0[j][0], v1 = x1[j][0];
#pragma unroll
            for (int k = 1; k < KM; ++k)
                if (k < ks) v0 += x0[j][k], v1 += x1[j][k];
            const int p = __builtin_amdgcn_readlane(rr.pos, j), page = __builtin_amdgcn_readlane(rr.page, j);
            float c = 0.0f, sn = 0.0f;
            if (!isv) {
                if (a.rope_cs) {
                    c = rr.cs[j].x, sn = rr.cs[j].y;
                } else {
                    rope_cs(p, lane, a.theta_scale, c, sn);
                }
            }
            if (row < a.M)
                qk_head(a.qkv + (size_t) row * a.ldqkv + (size_t) h * 128, lane, h, H, KVH, true, v0, v1, c, sn, w0,
                        w1, a.eps, a.kpool, a.vpool, page, a.page_cells, p % a.page_cells);
        }
    }
}

// The streaming form: the slice's activation records (gps groups, up to GMAX) are loaded once per workgroup by the 4
// wavefronts together and staged into LDS behind the kernel's only barrier; each wavefront then streams its own S
// stripes' weights through a ring of D register slots (group i + D's loads issued as soon as group i is summed), with
// no further synchronisation. The activation fragment, scales and corrections read from LDS for a block serve S x MT
// MFMAs. Same arithmetic and order as k_q4_gemm. FE: the fused epilogue run by each set's last workgroup (GemmArgs).
// (the hot arguments as preloaded scalars, GS_PARAMS)
template <int WT, int MT, int S, int D, int GMAX, int FE = FE_NONE, bool GRP = FE == FE_GSWIGLU>
__global__ __launch_bounds__(256) void k_q4_gemm_s(GS_PARAMS) {
    GS_TAKE();
    constexpr bool Q8 = WT == WT_Q8_0;
    constexpr int TB = Q8 ? Q8T_BYTES : Q4T_BYTES, SO = Q8 ? Q8T_SCALE_OFF : Q4T_SCALE_OFF;
    constexpr int NW = Q8 ? 2 : 1;
    constexpr int CORR = Q8 ? XA_CORR8_OFF : XA_CORR_OFF;
    constexpr int NF = GMAX * MT * 4;
    constexpr int NK = GMAX * MT * 2;
    __shared__ __attribute__((aligned(16))) uint8_t s_act[NF][1024];
    __shared__ __attribute__((aligned(16))) float s_k[GMAX][MT][2][64];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_in = lane & 15, g = lane >> 4;
    const int set = blockIdx.x, slice = blockIdx.y;
    if constexpr (FE != FE_NONE) {
        if (set * 4 * S >= a.nstripes) return;  // a padding set (the grid's sets: a multiple of nxcd)
    }
    int mt0 = (int) blockIdx.z * MT;
    const uint8_t* wbase = a.w;
    if constexpr (GRP) {  // grouped (MT = 1): this workgroup's (expert, row tile)
        if ((int) blockIdx.z >= *a.count) return;
        wbase = a.w + (size_t) a.items[2 * blockIdx.z] * a.wstride;
        mt0 = a.items[2 * blockIdx.z + 1];
    }
    mt0 = __builtin_amdgcn_readfirstlane(mt0);
    const int c0 = slice * a.gps, ng = __builtin_amdgcn_readfirstlane(min(a.gps, a.ngroups - c0));
    const int s0 = set * (4 * S) + wave * S;
    const int sbytes = a.ngroups * TB;
    // one resource for the whole matrix (see q4_gemm_ring)
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(wbase, (uint32_t) (a.nstripes * sbytes));
    const int ws_off = SO + 8 * n_in;  // (as in q4_gemm_ring)
    const int rstride = a.ngroups * XA_REC;
    // the activation: the operand's records from row tile mt0 on; or, gathering (a.gsrc, one row tile), lane l's row
    // m = l % 16 of the tile taken from row gsrc[16 mt0 + m] of a row-ordered operand of a.gM rows (a padding row,
    // gsrc < 0, reads as zeros: its offset is past the buffer). Per-lane offsets of a row's piece of a record:
    // fragments 16 (row % 16 + 16 g), scales and corrections 4 (16 b + row % 16), b = l / 16.
    size_t x0 = (size_t) mt0 * a.ngroups * XA_REC;
    uint32_t xbytes = (uint32_t) (xa_bytes(a.M, a.K) - x0);
    int vf_off = 16 * lane, vk_off = 4 * lane;
    if (GRP && a.gsrc) {
        const int sr = a.gsrc[16 * mt0 + (lane & 15)];
        x0 = 0;
        xbytes = (uint32_t) xa_bytes(a.gM, a.K);
        vf_off = sr < 0 ? (int) XA_GATHER_OOB : (sr >> 4) * rstride + 16 * ((sr & 15) + 16 * g);
        vk_off = sr < 0 ? (int) XA_GATHER_OOB : (sr >> 4) * rstride + 4 * (16 * g + (sr & 15));
    }
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(a.xa + x0, xbytes);
    constexpr bool ROPE = FE >= FE_ROPE && FE < FE_GSWIGLU;
    [[maybe_unused]] RopeRows<MT> rr;
    if constexpr (ROPE) rope_rows_begin<MT>(a, mt0, wave, lane, rr);

    // the slice's activation straight into LDS (buffer loads to LDS: lane l's 16 bytes land at 16 l of the fragment,
    // no registers; fragments past the slice repeat its last group: loads stay in bounds, never summed)
    for (int f = wave; f < NF; f += 4) {
        const int c = c0 + min(f / (4 * MT), ng - 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr) &s_act[f][0], 16, vf_off,
                                                 ((f / 4) % MT) * rstride + c * XA_REC + (f % 4) * 1024, 0, 0);
    }
    for (int k = wave; k < NK; k += 4) {
        const int c = c0 + min(k / (2 * MT), ng - 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr) &s_k[k / (2 * MT)][(k / 2) % MT][k % 2][0], 4, vk_off,
                                                 ((k / 2) % MT) * rstride + c * XA_REC + (k % 2 ? CORR : XA_DX_OFF), 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wq[D][S][NW];
    u32x2 ws[D][S];
    auto wload = [&](int slot, int i) {  // group i's weights (i past the slice: its last group again)
        const int c = c0 + min(i, ng - 1);
        for (int t = 0; t < S; ++t) {
            const int so = (s0 + t) * sbytes + c * TB;
            for (int h = 0; h < NW; ++h) wq[slot][t][h] = bload16(wr, 16 * NW * lane + 16 * h, so);
            ws[slot][t] = bload8(wr, ws_off, i < ng ? so : (int) XA_GATHER_OOB);
        }
    };
    for (int j = 0; j < D; ++j) {
        wload(j, j);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the arguments past the preloaded ones that the tail uses, read now (behind the first loads) rather than where
    // the compiler would sink them, at the tail, a round trip after the loop
    asm volatile("" ::"s"(a.part), "s"(a.N));
    // the LDS loads were issued first: waiting until no more than the weights' loads are outstanding waits for them
    constexpr int NWL = D * S * (NW + 1);
    static_assert(NWL < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((NWL & 15) | ((NWL >> 4) << 14) | (7 << 4) | (15 << 8));
    __syncthreads();
    if constexpr (ROPE) {
        rope_rows_end<MT>(a, set, mt0, wave, lane, rr);
        __builtin_amdgcn_sched_barrier(0);
    }

    floatx4 acc[S][MT];
    for (int t = 0; t < S; ++t)
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const int trips = (ng + D - 1) / D;
    for (int tr = 0; tr < trips; ++tr)
        for (int j = 0; j < D; ++j) {
            const int i = tr * D + j;
            const int li = min(i, ng - 1);  // (its LDS group; a group past the slice has zero scales)
            __builtin_amdgcn_sched_barrier(0);
            // block b's MFMAs are issued before block b - 1's scale FMAs (the same FMAs in the same order per output,
            // so the same sums), so a block's matrix-core latency is spent on the previous block's VALU work
            floatx4 is[2][S][MT], sc[2][S][MT];
            for (int b = 0; b < 5; ++b) {
                if (b < 4) {
                    half8 A[MT];
                    half4v da[MT];
                    floatx4 cr[MT];
                    for (int mt = 0; mt < MT; ++mt) {
                        A[mt] = *(const half8*) &s_act[(li * MT + mt) * 4 + b][16 * lane];
                        da[mt] = scale_a(s_k[li][mt][0][b * 16 + 4 * g + (n_in & 3)], b);
                        cr[mt] = *(const floatx4*) &s_k[li][mt][1][b * 16 + 4 * g];
                    }
                    for (int t = 0; t < S; ++t) {
                        const half8 bw = Q8 ? q8_unpack(wq[j][t][b / 2][2 * (b % 2)], wq[j][t][b / 2][2 * (b % 2) + 1])
                                            : q4_unpack(wq[j][t][0][b]);
                        for (int mt = 0; mt < MT; ++mt) {
                            is[b & 1][t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], bw, cr[mt], 0, 0, 0);
                            sc[b & 1][t][mt] = scale_products(da[mt], ws[j][t]);
                        }
                    }
                }
                if (b > 0) {
                    const int pb = (b - 1) & 1;
                    for (int t = 0; t < S; ++t)
                        for (int mt = 0; mt < MT; ++mt)
                            for (int v = 0; v < 4; ++v)
                                acc[t][mt][v] = __builtin_fmaf(is[pb][t][mt][v], sc[pb][t][mt][v], acc[t][mt][v]);
                }
            }
            // the group's sums are complete here (left to the compiler, they sank below the next loads)
            for (int t = 0; t < S; ++t)
                for (int mt = 0; mt < MT; ++mt) asm volatile("" : "+v"(acc[t][mt]));
            __builtin_amdgcn_sched_barrier(0);
            wload(j, i + D);
        }
    // the sums out through LDS (the activation's space, once every wavefront is done with it): each wavefront's
    // [16 MT rows][16 S columns] tile is written back as 16-byte pieces of rows, part[slice][row][col]
    __syncthreads();
    if constexpr (FE == FE_GSWIGLU) {
        // grouped gate|up with its SwiGLU + Q8_0 (one slice: the workgroup's sums are whole). Wavefront w's 4 stripes
        // are gate, up, gate, up of Q8_0 block b = 4 set + w of the F = N / 2 SwiGLU columns (the columns
        // k_swiglu_quant reads: gate at 64 b + 4 g (+32), up 16 further), so silu(gate) * up of its 16 rows goes
        // through its own LDS rows to lanes (row, part) for q8_store, into a.xo (the down matmul's operand)
        static_assert(S == 4 && MT == 1, "a wavefront holds one block of SwiGLU columns");
        constexpr int HW = 36;  // (a row's 32 values, padded)
        float* hw = (float*) &s_act[0][0] + wave * 16 * HW;
        for (int v = 0; v < 4; ++v) {
            const int r = 4 * g + v;
            hw[r * HW + n_in] = silu(acc[0][0][v]) * acc[1][0][v];
            hw[r * HW + 16 + n_in] = silu(acc[2][0][v]) * acc[3][0][v];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the rows are written (this wavefront's own)
        __builtin_amdgcn_wave_barrier();
        const int m = lane >> 2, gq = lane & 3, row = mt0 * 16 + m, b = 4 * set + wave, F = a.N / 2;
        float v8[8];
        for (int j = 0; j < 4; ++j) {
            v8[j] = hw[m * HW + 4 * gq + j];
            v8[4 + j] = hw[m * HW + 16 + 4 * gq + j];
        }
        // (a row's 4 lane parts leave together: q8_store's shuffles stay within them)
        if (row >= a.M || 32 * b >= F || (a.rmask && a.rmask[row] < 0)) return;
        q8_store(v8, gq, a.xo, F, row, b);
        return;
    }
    constexpr int TW = 16 * S + 4;  // (a tile row's floats, padded)
    static_assert(4 * 16 * MT * TW * 4 <= NF * 1024, "the tiles fit the activation's LDS");
    float* tile = (float*) &s_act[0][0] + wave * 16 * MT * TW;
    for (int t = 0; t < S; ++t)
        for (int mt = 0; mt < MT; ++mt)
            for (int v = 0; v < 4; ++v) tile[(mt * 16 + 4 * g + v) * TW + 16 * t + n_in] = acc[t][mt][v];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the tile is written (it is this wavefront's own)
    __builtin_amdgcn_wave_barrier();
    for (int e = lane; e < 16 * MT * 4 * S; e += 64) {
        const int r = e / (4 * S), c4 = (e % (4 * S)) * 4;
        const int row = mt0 * 16 + r, col = s0 * 16 + c4;
        if (row >= a.M || col >= a.N) continue;  // (a stripe past the matrix is not stored)
        if (GRP && a.rmask && a.rmask[row] < 0) continue;
        const float4 v = *(const float4*) &tile[r * TW + c4];
        float* dst = &a.part[((size_t) slice * a.M + row) * a.N + col];
        if (a.N % 4 == 0) {
            *(float4*) dst = v;
        } else {  // (a ragged N: rows are not 16-byte aligned, and the last piece may cross the row's end)
            const float vv[4] = {v.x, v.y, v.z, v.w};
            for (int q = 0; q < 4; ++q)
                if (col + q < a.N) dst[q] = vv[q];
        }
    }
    if constexpr (FE != FE_NONE && FE != FE_GSWIGLU) {
        // this workgroup's sums have reached the L2 (vmcnt counts stores); then it counts itself, and the count's
        // completer (it resets the counter for the next launch) finishes the set
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        __shared__ int s_last;
        uint64_t* c = a.cnt + (size_t) (set + (int) gridDim.x * (int) blockIdx.z) * CNT_STRIDE;
        uint64_t done = 0;  // (the completer's thread 0: the count, taken back once the epilogue is issued)
        if (threadIdx.x == 0) {
            unsigned xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
            const int f = 8 + 5 * (int) (xcc & 7);  // this XCD's field of the count
            const uint64_t add = 1ull + (1ull << f);
            const uint64_t n = __hip_atomic_fetch_add(c, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
            s_last = (int) (n & 255) == (int) gridDim.y;
            if (s_last) {
                if ((int) ((n >> f) & 31) != (int) gridDim.y)  // some workgroup of the set ran on another XCD
                    __hip_atomic_fetch_or(a.xerr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                done = n;
            }
        }
        __syncthreads();
        if (!s_last) return;
        l1_drop();
        q4_epilogue<FE, MT, S>(a, set, mt0, rr);
        // back to zero by an atomic of the same kind, performed where the counts were (a plain store of an atomic
        // compiles to a write-through store, which need not meet the L2's copy); after the epilogue, so that no
        // barrier waits for it (every count of the set has been made: the next launch is the next to count)
        if (threadIdx.x == 0) __hip_atomic_fetch_add(c, (uint64_t) 0 - done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The few-row matmul (M <= 4 rows: the reference's mat-vec rows, mv_q4, kernels.metal:1324-1411). One lane per output
// column: a wavefront takes 4 stripes (64 columns), a workgroup 16, and the plan's k-slices go across workgroups as
// the MFMA kernels split them. The slice's activation rows are staged once into LDS as int8 (from the operand's fp16
// fragments: q, and q / 16 for elements 16..31) with each block's sum of q. A lane loads its column's 64 bytes of a
// tile (its row's 16 bytes at each of the 4 lane positions of the tile: 4 bytes of each of the 4 blocks), unpacks the
// nibbles with a mask and a shift and sums a block with 8 v_dot4 per row: isum = sum q w - 8 sum q = sum q (w - 8),
// the integer the MFMA kernels form; then acc = fma(isum, dw * dx, acc) block by block in the slice's order, a slice
// with an odd group count padded with a zero-scale group as the MFMA kernels' rings pad it. So every sum is the MFMA
// kernels' fp32 bits, and part[slice][M][N] is what their consumers expect. D groups of weights in flight a wavefront.
#define GEMV_GMAX 32  // groups of a slice the staging holds
#define GEMV_ROWS 0   // steps of at most this many rows take the GEMV by default (the MFMA kernels otherwise)
template <int MR, int D>
__global__ __launch_bounds__(256) void k_q4_gemv(GemmArgs a) {
    constexpr int TB = Q4T_BYTES, SO = Q4T_SCALE_OFF;
    constexpr int NIT = MR * GEMV_GMAX * 16 / 256;  // staging items (row, block, lane part) a thread
    constexpr int NDX = (MR * GEMV_GMAX * 4 + 255) / 256;  // block scales a thread stages
    __shared__ __attribute__((aligned(16))) uint32_t s_q[MR][GEMV_GMAX * 4][8];  // int8 q of (row, block)
    __shared__ float s_dx[MR][GEMV_GMAX * 4];
    __shared__ int32_t s_sx[MR][GEMV_GMAX * 4];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, sl = lane >> 4;
    const int set = blockIdx.x, slice = blockIdx.y;
    const int c0 = slice * a.gps, ng = __builtin_amdgcn_readfirstlane(min(a.gps, a.ngroups - c0));
    const int ngp = (ng + 1) & ~1;  // the groups summed: the slice's, an odd count padded with a zero-scale group
    const int nb = 4 * ng;          // blocks of the slice
    const int s0 = set * 16 + wave * 4;
    const int nvalid = __builtin_amdgcn_readfirstlane(max(0, min(4, a.nstripes - s0)));
    const int sbytes = a.ngroups * TB;
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(a.w, (uint32_t) (a.nstripes * sbytes));  // (the whole matrix)
    const int vst = sl * sbytes;  // this lane's stripe, from the wavefront's first
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(a.xa, (uint32_t) xa_bytes(a.M, a.K));
    // the staging loads first (item (m, block, part g): the 8 fp16 of row m's fragment piece g), then the weights
    u32x4 rq[NIT];
    float rdx[NDX];
    for (int j = 0; j < NIT; ++j) {
        const int it = min((int) threadIdx.x + 256 * j, MR * nb * 4 - 1), g = it & 3, b = (it >> 2) % nb, m = (it >> 2) / nb;
        rq[j] = bload16(xr, 16 * (m + 16 * g), (c0 + b / 4) * XA_REC + (b % 4) * 1024);
    }
    for (int j = 0; j < NDX; ++j) {
        const int it = min((int) threadIdx.x + 256 * j, MR * nb - 1), b = it % nb, m = it / nb;
        rdx[j] = bload4f(xr, 4 * m, (c0 + b / 4) * XA_REC + XA_DX_OFF + (b % 4) * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wq[D][4];
    u32x2 ws[D];
    auto load = [&](int slot, int i) {  // group i of the slice (past it: its last group again)
        const int so = s0 * sbytes + (c0 + min(i, ng - 1)) * TB;
        for (int g = 0; g < 4; ++g) wq[slot][g] = bload16(wr, vst + 16 * (n + 16 * g), so);
        ws[slot] = bload8(wr, vst + SO + 8 * n, so);
    };
    for (int j = 0; j < D; ++j) {
        load(j, j);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int j = 0; j < NIT; ++j) {
        const int it = (int) threadIdx.x + 256 * j;  // (the item count is a multiple of 4: the 4 parts of a block
        const bool ok = it < MR * nb * 4;              // are adjacent lanes, all in or all out)
        const int g = it & 3, b = (it >> 2) % nb, m = (it >> 2) / nb;
        const half8 h = __builtin_bit_cast(half8, rq[j]);
        int q[8];
        for (int e = 0; e < 4; ++e) q[e] = (int) (float) h[e];
        for (int e = 4; e < 8; ++e) q[e] = (int) ((float) h[e] * 16.0f);
        int sx = q[0] + q[1] + q[2] + q[3] + q[4] + q[5] + q[6] + q[7];
        sx += __shfl_xor(sx, 1);
        sx += __shfl_xor(sx, 2);
        if (ok) {
            s_q[m][b][g] = (q[0] & 255) | (q[1] & 255) << 8 | (q[2] & 255) << 16 | (uint32_t) (q[3] & 255) << 24;
            s_q[m][b][4 + g] = (q[4] & 255) | (q[5] & 255) << 8 | (q[6] & 255) << 16 | (uint32_t) (q[7] & 255) << 24;
            if (g == 0) s_sx[m][b] = sx;
        }
    }
    for (int j = 0; j < NDX; ++j) {
        const int it = (int) threadIdx.x + 256 * j;
        if (it < MR * nb) s_dx[it / nb][it % nb] = rdx[j];
    }
    __syncthreads();

    const int M = min(a.M, MR);
    float acc[MR];
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    const int trips = (ngp + D - 1) / D;
    for (int tr = 0; tr < trips; ++tr)
        for (int j = 0; j < D; ++j) {
            const int i = tr * D + j;
            const float msc = i < ng ? 1.0f : 0.0f;  // (the padding group adds with scale 0)
            const bool live = i < ngp;               // (groups past the padded count: computed, not added)
            const int lb = 4 * min(i, ng - 1);       // (its blocks in LDS)
            __builtin_amdgcn_sched_barrier(0);
            for (int b = 0; b < 4; ++b) {
                uint32_t wl[4], wh[4];
                for (int g = 0; g < 4; ++g) {  // (the tile's bytes 1 and 2 back in element order)
                    const uint32_t w = __builtin_amdgcn_perm(wq[j][g][b], wq[j][g][b], 0x03010200u);
                    wl[g] = w & 0x0F0F0F0Fu;
                    wh[g] = (w >> 4) & 0x0F0F0F0Fu;
                }
                const float dw = (float) __builtin_bit_cast(half4v, ws[j])[b] * msc;
                for (int m = 0; m < MR; ++m) {
                    const u32x4 q0 = *(const u32x4*) &s_q[m][lb + b][0], q1 = *(const u32x4*) &s_q[m][lb + b][4];
                    int isum = 0;
                    for (int g = 0; g < 4; ++g) isum = __builtin_amdgcn_sdot4((int) q0[g], (int) wl[g], isum, false);
                    for (int g = 0; g < 4; ++g) isum = __builtin_amdgcn_sdot4((int) q1[g], (int) wh[g], isum, false);
                    isum -= 8 * s_sx[m][lb + b];
                    const float v = __builtin_fmaf((float) isum, dw * s_dx[m][lb + b], acc[m]);
                    acc[m] = live ? v : acc[m];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            load(j, i + D);
        }
    const int stripe = s0 + sl, col = stripe * 16 + n;
    if (sl < nvalid && col < a.N)
        for (int m = 0; m < MR; ++m)
            if (m < M) a.part[((size_t) slice * a.M + m) * a.N + col] = acc[m];
}

// k-slice partial sums added in slice order, then the epilogue
__global__ void k_q4_reduce(GemmArgs a) {
    const int outN = a.epi == EPI_SWIGLU ? a.N / 2 : a.N;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.M * outN) return;
    const int row = i / outN, col = i % outN;
    auto sum = [&](int c) {
        float s = 0.0f;
        for (int k = 0; k < a.ks; ++k) s += a.part[((size_t) k * a.M + row) * a.N + c];
        return s;
    };
    if (a.epi == EPI_SWIGLU) {
        // output column 16 p + n: gate column 32 p + n, up column 32 p + 16 + n of the interleaved matrix
        const int p = col / 16, n = col % 16;
        a.y[(size_t) row * a.ldy + col] = silu(sum(32 * p + n)) * sum(32 * p + 16 + n);
    } else if (a.epi == EPI_ADD) {
        a.y[(size_t) row * a.ldy + col] += sum(col);
    } else {
        a.y[(size_t) row * a.ldy + col] = sum(col);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// host side

// The launch shape depends on (N, K) only, never on the rows (row invariance): 4 spw stripes per workgroup (spw = 2
// only for LM-head-wide matrices) and the groups of K in slices across workgroups. A slice holds an even number of groups (the kernel walks groups in
// pairs, one per ring slot; an odd count would add a masked pass), halved from the whole of K while the launch has
// fewer than 768 workgroups, down to 4 groups and at most KS_MAX slices: on MI355X at 32 rows, short slices (a single
// round of loads per workgroup) beat fewer, longer workgroups for the layer-sized matrices, while every slice costs
// the consumer one more partial sum to read.
#define Q4_WIDE (8 * 768)  // stripes of an LM-head-wide matrix
#define Q4_PAIR_ROWS 256   // rows from which every matrix takes its row tiles in pairs
GemmPlan q4_plan(int N, int K, int wt) {
    GemmPlan p;
    p.nstripes = (N + 15) / 16;
    p.ngroups = (K / 32 + 3) / 4;
    auto slices = [&](int gps) { return (p.ngroups + gps - 1) / gps; };
    if (p.nstripes >= Q4_WIDE) {
        // LM-head-wide: the ring kernel, 2 stripes a wavefront (never for Q8_0: twice the weight registers), enough
        // workgroups with no k-split (67 against 77 us for the Q4_0 head at 32 rows)
        p.stream = false;
        p.spw = wt != WT_Q8_0 ? 2 : 1;
        p.sets = (p.nstripes + 4 * p.spw - 1) / (4 * p.spw);
        int gps = (p.ngroups + 1) / 2 * 2;
        while (gps > 4 && p.sets * slices(gps) < 768 && slices(gps - 2) <= KS_MAX) gps -= 2;
        p.gps = gps;
        p.ks = slices(gps);
        p.sspw = p.smt = 1;
        p.sd = 2;
        return p;
    }
    // Layer matrices: slices of 4 groups, or 8 for the wide (gate|up) and the deep (down) ones. Measured at 32 rows on
    // MI355X (streaming kernel, launches back to back): q|k|v 6.2 us (2 stripes a wavefront), o 5.5, gate|up 12.9 (2
    // stripes, both row tiles in one workgroup), down 8.4 (10 slices); the ring kernel with its earlier slices took
    // 7.5, 6.4, 15.0 and 10.8.
    p.stream = true;
    // (8 groups also for the narrow and deep o projection, 4 slices at K = 4096: decode 7,820 -> 7,860 tok/s in the
    // engine, measured against the other plans of the four matrices in one call)
    const bool narrow_deep = p.nstripes < 384 && p.ngroups >= 32;
    p.gps = std::min(p.nstripes >= 1024 || p.ngroups >= 64 || narrow_deep ? 8 : 4, (p.ngroups + 1) / 2 * 2);
    // the slices' consumers (the row kernels) add at most KS_MAX of them: deeper matrices take longer slices (Qwen3-14B's
    // down projection, K = 17408: 10 groups, 14 slices; Qwen3-32B's, K = 25600: 14 groups, 15 slices). The streaming
    // kernel stages at most 8 groups of a slice in LDS; longer slices go to the ring kernel, whose LDS holds two groups.
    while (slices(p.gps) > KS_MAX) p.gps += 2;
    if (p.gps > 8) p.stream = false;
    p.ks = slices(p.gps);
    // two stripes a wavefront for the wide matrices and the deep down projection (whose 8-stripe sets then make 400
    // workgroups at 32 rows: with the o projection's plan above, decode 7,820 -> 7,900 tok/s)
    p.sspw = wt != WT_Q8_0 && (p.nstripes >= 384 || p.ngroups >= 64) ? 2 : 1;
    p.smt = p.nstripes >= 1024 ? 2 : 1;
    // 4 groups in flight a wavefront for the o projection (one stripe a wavefront), 2 for the others. Measured in the
    // step against depth 2, A/B in one call: decode 8,274 -> 8,281 tok/s, Qwen3-30B-A3B 4,827 -> 4,862; depth 4 for
    // the gate|up matrix as well cost decode 0.45%, for q|k|v 0.6% and for down 0.7%
    p.sd = wt == WT_Q4_0 && narrow_deep && p.sspw == 1 ? 4 : 2;
    // the ring kernel (prompt rows) with the same slices: one stripe a wavefront
    p.spw = 1;
    p.sets = (p.nstripes + 3) / 4;
    return p;
}

size_t q4_workspace_bytes(int M, int N, int K, int wt) { return (size_t) q4_plan(N, K, wt).ks * M * N * sizeof(float); }

// (FK: one stripe a wavefront only, the plan of every split layer matrix)
template <int WT, bool FK = false>
static void launch_gemm(int mt, int spw, dim3 grid, const GemmArgs& a, hipStream_t st) {
    if constexpr (WT == WT_Q4_0 && !FK) {
        if (mt == 1) {
            if (spw == 2) hipLaunchKernelGGL((k_q4_gemm<WT, 1, 2, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
            else hipLaunchKernelGGL((k_q4_gemm<WT, 1, 1, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
        } else {
            if (spw == 2) hipLaunchKernelGGL((k_q4_gemm<WT, 2, 2, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
            else hipLaunchKernelGGL((k_q4_gemm<WT, 2, 1, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
        }
    } else {  // Q8_0: one stripe per wavefront (q4_plan); FK likewise
        (void) spw;
        if (mt == 1) hipLaunchKernelGGL((k_q4_gemm<WT, 1, 1, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
        else hipLaunchKernelGGL((k_q4_gemm<WT, 2, 1, FK>), grid, dim3(256), 0, st, GS_ARGS(a));
    }
}

// k_q4_gemm_s launches: ring depth D, gps groups a slice (LDS sized for up to 4 or 8), (MT, S); false when the
// combination is not instantiated. Q8_0 tiles take one stripe a wavefront (their weight registers are twice as many).
template <int WT>
static bool launch_gemm_s(int mt, int spw, int D, int gps, dim3 grid, const GemmArgs& a, hipStream_t st) {
#define GSX(MT_, S_, D_, GM_)                                                                                \
    if (mt == MT_ && spw == S_ && D == D_ && gps <= GM_) {                                                   \
        hipLaunchKernelGGL((k_q4_gemm_s<WT, MT_, S_, D_, GM_>), grid, dim3(256), 0, st, GS_ARGS(a));                  \
        return true;                                                                                         \
    }
    GSX(1, 1, 2, 4) GSX(1, 1, 2, 8) GSX(2, 1, 2, 4) GSX(2, 1, 2, 8)
    if constexpr (WT == WT_Q4_0) {
        GSX(1, 1, 4, 4) GSX(1, 1, 4, 8) GSX(2, 1, 4, 4)
        GSX(1, 2, 2, 4) GSX(1, 2, 2, 8) GSX(1, 2, 4, 8) GSX(2, 2, 2, 4) GSX(2, 2, 2, 8) GSX(2, 2, 4, 4)
    }
#undef GSX
    return false;
}

// The per-column GEMV (k_q4_gemv) of M <= 4 rows with the plan's slices; false when it does not take the shape.
static bool launch_gemv(const GemmPlan& p, const GemmArgs& a, hipStream_t st) {
    if (a.M < 1 || a.M > 4 || p.gps > GEMV_GMAX) return false;
    const dim3 grid((p.nstripes + 15) / 16, p.ks);
    if (a.M == 1) hipLaunchKernelGGL((k_q4_gemv<1, 4>), grid, dim3(256), 0, st, a);
    else if (a.M == 2) hipLaunchKernelGGL((k_q4_gemv<2, 4>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_q4_gemv<4, 4>), grid, dim3(256), 0, st, a);
    return true;
}

int q4_gemm_raw(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                hipStream_t st, int wt) {
    if (M <= 0) return 0;
    if (wt != WT_Q4_0 && wt != WT_Q8_0) return -1;
    const GemmPlan p = q4_plan(N, K, wt);
    if (part == nullptr || part_bytes < (size_t) p.ks * M * N * sizeof(float)) return -1;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.part = part; a.y = nullptr;
    a.M = M; a.N = N; a.K = K; a.ldy = 0; a.epi = EPI_STORE;
    a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps;
    a.mtiles = (M + 15) / 16;
    if (wt == WT_Q4_0 && M <= GEMV_ROWS && launch_gemv(p, a, st)) return p.ks;  // few rows: the per-column GEMV
    if (p.stream && a.M < Q4_PAIR_ROWS) {  // the streaming kernel (ring depth 2)
        const int mt = std::min(p.smt, a.mtiles);
        const dim3 grid((p.nstripes + 4 * p.sspw - 1) / (4 * p.sspw), p.ks, (a.mtiles + mt - 1) / mt);
        const bool ok = wt == WT_Q8_0 ? launch_gemm_s<WT_Q8_0>(mt, p.sspw, 2, p.gps, grid, a, st)
                                      : launch_gemm_s<WT_Q4_0>(mt, p.sspw, p.sd, p.gps, grid, a, st);
        return ok ? p.ks : -1;
    }
    // row tiles of 16 per workgroup (grid z: one per tile) for matrices narrower than 512 stripes: twice the workgroups
    // and loads in flight (q|k|v, o, down: 8.4 against 9.1 us at 32 rows; the two workgroups of a tile pair run on the
    // same XCD, so the second reads the weights from its L2); pairs of tiles for the wider ones (the Q8_0 gate|up and
    // the LM heads were slower with single tiles, the Q4_0 gate|up the same), and for every matrix from Q4_PAIR_ROWS
    // rows on (prompt rows; Qwen3-4B at 512 rows a step: 15.9 ms a step against 16.3 with the narrow ones single and
    // 16.6 all single; 4 tiles, at 2 wavefronts a SIMD for their registers, 17.5). Either way a row's sums are the same
    // (same slices, same order).
    const int mt = a.mtiles == 1 || (p.nstripes < 512 && a.M < Q4_PAIR_ROWS) ? 1 : 2;
    // prompt rows: one workgroup walks every slice of its tiles and leaves their sum in part[0] (the same bits the
    // consumers make of the slices), so no slice is written or read back (at 512 rows the split launches wrote 16-120
    // MB of slices a matrix)
    if (a.M >= Q4_PAIR_ROWS && p.ks > 1 && p.spw == 1 && p.gps % 2 == 0) {
        // Qwen3-4B at 512 rows a step (launches of one sequence's prompt): 2 stripes a wavefront for the wide q|k|v
        // and gate|up (33 and 92 us against 42 and 119 with one; 4 stripes: 42 and 92), one for o and down (54 us
        // against 60 with two); 40.7k -> 43.3k prompt tok/s on one box. The split launches and their slices: 34.7k.
        // o and down (fewer than 384 stripes) in single row tiles: twice their workgroups, 45.0k against 44.1k tok/s
        // with tile pairs (q|k|v in single tiles: 44.5k)
        const int fmt = p.nstripes < 384 ? 1 : 2;
        if (wt == WT_Q4_0 && p.nstripes >= 384) {
            const dim3 grid((p.nstripes + 7) / 8, 1, (a.mtiles + 1) / 2);
            hipLaunchKernelGGL((k_q4_gemm_fk2<WT_Q4_0, 2, 2>), grid, dim3(256), 0, st, GS_ARGS(a));
        } else {
            const dim3 grid(p.sets, 1, (a.mtiles + fmt - 1) / fmt);
            if (wt == WT_Q8_0) launch_gemm<WT_Q8_0, true>(fmt, 1, grid, a, st);
            else launch_gemm<WT_Q4_0, true>(fmt, 1, grid, a, st);
        }
        return 1;
    }
    const dim3 grid(p.sets, p.ks, mt == 1 ? a.mtiles : (a.mtiles + 1) / 2);
    if (wt == WT_Q8_0) launch_gemm<WT_Q8_0>(mt, p.spw, grid, a, st);
    else launch_gemm<WT_Q4_0>(mt, p.spw, grid, a, st);
    return p.ks;
}

// the streaming kernel with a fused epilogue: false when (FE, MT, S, gps) is not instantiated (ring depth 2)
template <int WT, int FE>
static bool launch_gemm_fe(int mt, int spw, int gps, dim3 grid, const GemmArgs& a, hipStream_t st) {
#define GSF(MT_, S_, GM_)                                                                                    \
    if (mt == MT_ && spw == S_ && gps <= GM_) {                                                              \
        hipLaunchKernelGGL((k_q4_gemm_s<WT, MT_, S_, 2, GM_, FE>), grid, dim3(256), 0, st, GS_ARGS(a));               \
        return true;                                                                                         \
    }
    if constexpr (WT == WT_Q4_0) {
        GSF(1, 2, 4) GSF(1, 2, 8) GSF(2, 2, 4) GSF(2, 2, 8)
    } else if constexpr (FE < FE_ROPE) {  // (Q8_0 tiles: one stripe a wavefront; a set is one Q8_0 block of F)
        GSF(1, 1, 4) GSF(1, 1, 8) GSF(2, 1, 4) GSF(2, 1, 8)
    }
#undef GSF
    return false;
}

// the fused launch's shape: stripes a wavefront, row tiles a workgroup, the grid (its sets padded to a multiple of
// nxcd); false when the plan, the weight type or the epilogue's unit does not allow one
static bool fused_shape(int M, int N, int K, int wt, int fe, int nxcd, int cnt_len, GemmPlan& p, int& spw, int& mt,
                        dim3& grid) {
    if (M <= 0 || M >= Q4_PAIR_ROWS || nxcd < 1 || (wt != WT_Q4_0 && wt != WT_Q8_0)) return false;
    p = q4_plan(N, K, wt);
    if (!p.stream || p.gps > 8) return false;
    // a set must hold whole epilogue units: one head (8 stripes: two a wavefront, Q4_0 tiles), or S Q8_0 blocks of
    // SwiGLU columns (64 S interleaved columns)
    if (fe == FE_ROPE) {
        if (wt != WT_Q4_0 || N % 128) return false;
        spw = 2;
    } else if (fe == FE_SWIGLU) {
        spw = wt == WT_Q4_0 ? 2 : 1;  // (the instances: Q8_0 tiles one stripe a wavefront)
        if (N % (64 * spw) || p.ks > 8) return false;  // (more slices: their loads would not fit the registers)
    } else {
        return false;
    }
    const int mtiles = (M + 15) / 16;
    mt = std::min(p.smt, mtiles);
    const int sets = (p.nstripes + 4 * spw - 1) / (4 * spw);
    grid = dim3((sets + nxcd - 1) / nxcd * nxcd, p.ks, (mtiles + mt - 1) / mt);
    return (long) grid.x * grid.z * CNT_STRIDE <= cnt_len;
}

bool q4_gemm_fused_fits(int M, int N, int K, int wt, int fe, int nxcd, int cnt_len) {
    GemmPlan p;
    int spw, mt;
    dim3 grid;
    return fused_shape(M, N, K, wt, fe, nxcd, cnt_len, p, spw, mt, grid);
}

int q4_gemm_fused(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                  hipStream_t st, int wt, int fe, const GemmArgs& ea, int cnt_len) {
    if (M <= 0) return 0;
    if (!ea.cnt || !ea.xerr || (fe == FE_SWIGLU && (!ea.xo || ea.xo == xa))) return -1;
    GemmPlan p;
    int spw, mt;
    dim3 grid;
    if (!fused_shape(M, N, K, wt, fe, ea.nxcd, cnt_len, p, spw, mt, grid)) return 0;
    if (part == nullptr || part_bytes < (size_t) p.ks * M * N * sizeof(float)) return -1;
    GemmArgs a = ea;
    a.w = w; a.xa = xa; a.part = part; a.y = nullptr;
    a.M = M; a.N = N; a.K = K; a.ldy = 0; a.epi = EPI_STORE;
    a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps;
    a.mtiles = (M + 15) / 16;
    a.items = nullptr; a.count = nullptr; a.rmask = nullptr; a.gsrc = nullptr;
    // the epilogue's slice bound: instance FE + fe_slice_index(ks) (KM = fe_slice_bound of it, the least one >= ks)
    const int lk = fe_slice_index(p.ks);
    bool ok = false;
    auto go = [&](auto fe_c) {
        constexpr int F0 = decltype(fe_c)::value;
        auto pick = [&](auto wt_c) {
            constexpr int W = decltype(wt_c)::value;
            switch (lk) {
                case 0: ok = launch_gemm_fe<W, F0 + 0>(mt, spw, p.gps, grid, a, st); break;
                case 1: ok = launch_gemm_fe<W, F0 + 1>(mt, spw, p.gps, grid, a, st); break;
                case 2: ok = launch_gemm_fe<W, F0 + 2>(mt, spw, p.gps, grid, a, st); break;
                case 3: ok = launch_gemm_fe<W, F0 + 3>(mt, spw, p.gps, grid, a, st); break;
                case 4: ok = launch_gemm_fe<W, F0 + 4>(mt, spw, p.gps, grid, a, st); break;
                case 5: ok = launch_gemm_fe<W, F0 + 5>(mt, spw, p.gps, grid, a, st); break;
                case 6: if constexpr (F0 == FE_ROPE) ok = launch_gemm_fe<W, F0 + 6>(mt, spw, p.gps, grid, a, st); break;
                case 7: if constexpr (F0 == FE_ROPE) ok = launch_gemm_fe<W, F0 + 7>(mt, spw, p.gps, grid, a, st); break;
            }
        };
        if (wt == WT_Q8_0) {
            if constexpr (F0 == FE_SWIGLU) pick(std::integral_constant<int, WT_Q8_0>{});  // (SwiGLU: at most 8 slices)
            return;
        }
        pick(std::integral_constant<int, WT_Q4_0>{});
    };
    if (fe == FE_SWIGLU) go(std::integral_constant<int, FE_SWIGLU>{});
    else go(std::integral_constant<int, FE_ROPE>{});
    return ok ? 1 : -1;
}

// One workgroup of the probe records the XCD it runs on
__global__ __launch_bounds__(64) void k_xcd_probe(int32_t* out) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t) (xcc & 15);
}

bool xcd_round_robin(hipStream_t st, int* nxcd) {
    const int n = 8192;
    int32_t* d = nullptr;
    *nxcd = 1;
    if (hipMalloc(&d, n * sizeof(int32_t)) != hipSuccess) return false;
    std::vector<int32_t> h(n, -1);
    hipLaunchKernelGGL(k_xcd_probe, dim3(n), dim3(64), 0, st, d);
    const bool ran = hipStreamSynchronize(st) == hipSuccess &&
                     hipMemcpy(h.data(), d, n * sizeof(int32_t), hipMemcpyDeviceToHost) == hipSuccess;
    hipFree(d);
    if (!ran) return false;
    unsigned seen = 0;
    for (int i = 0; i < n; ++i) {
        if (h[i] < 0 || h[i] > 15) return false;
        seen |= 1u << h[i];
    }
    *nxcd = __builtin_popcount(seen);
    if (*nxcd > 8) return false;  // (the count's XCD fields: 8 of 5 bits)
    for (int i = 0; i < n; ++i)
        if (h[i] != h[i % *nxcd]) return false;
    return true;
}

// An explicit launch plan (for tuning): the streaming kernel with mt row tiles a workgroup (1, 2), spw stripes a
// wavefront (1, 2, 4), ring depth D and gps groups a slice, encoded G = -(100 D + gps); G 0: the default plan. The
// k-slice sums go to part. Returns the slice count, or -1 (a plan not instantiated, or part too small).
int q4_gemm_raw_plan(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                     hipStream_t st, int wt, int mt, int spw, int G) {
    if (mt == 0) {  // the per-column GEMV with the default plan's slices (Q4_0, M <= 4)
        const GemmPlan p = q4_plan(N, K, wt);
        if (wt != WT_Q4_0 || G != 0 || part == nullptr || part_bytes < (size_t) p.ks * M * N * sizeof(float)) return -1;
        GemmArgs a{};
        a.w = w; a.xa = xa; a.part = part;
        a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
        a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps; a.mtiles = (M + 15) / 16;
        return launch_gemv(p, a, st) ? p.ks : -1;
    }
    if (G == 0) return q4_gemm_raw(w, xa, M, N, K, part, part_bytes, st, wt);
    if (G > 0) return -1;
    const int gps = (-G) % 100, D = (-G) / 100;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.part = part;
    a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
    a.nstripes = (N + 15) / 16; a.ngroups = (K / 32 + 3) / 4; a.gps = gps; a.ks = (a.ngroups + gps - 1) / gps;
    a.mtiles = (M + 15) / 16;
    if (gps <= 0 || a.ks > KS_MAX || part == nullptr || part_bytes < (size_t) a.ks * M * N * sizeof(float)) return -1;
    const int sets = (a.nstripes + 4 * spw - 1) / (4 * spw);
    const dim3 grid(sets, a.ks, (a.mtiles + mt - 1) / mt);
    const bool ok = wt == WT_Q8_0 ? launch_gemm_s<WT_Q8_0>(mt, spw, D, gps, grid, a, st)
                                  : launch_gemm_s<WT_Q4_0>(mt, spw, D, gps, grid, a, st);
    return ok ? a.ks : -1;
}

// The grouped matmul through the streaming kernel: one slice (every group of K staged at once, ng <= 16), one row
// tile a workgroup, S stripes a wavefront; false when the combination is not instantiated.
template <int WT>
static bool launch_grouped_s(int S, int ng, dim3 grid, const GemmArgs& a, hipStream_t st) {
#define GSG(S_, GM_)                                                                                         \
    if (S == S_ && ng <= GM_) {                                                                              \
        hipLaunchKernelGGL((k_q4_gemm_s<WT, 1, S_, 2, GM_, FE_NONE, true>), grid, dim3(256), 0, st, GSG_ARGS(a));      \
        return true;                                                                                         \
    }
    if constexpr (WT == WT_Q4_0) {
        GSG(2, 8) GSG(2, 16) GSG(4, 8) GSG(4, 16)
    } else {
        GSG(1, 8) GSG(1, 16)
    }
#undef GSG
    return false;
}

int q4_gemm_grouped(const uint8_t* w, size_t wstride, const int32_t* items, const int32_t* count, int max_items,
                    const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes, hipStream_t st, int wt,
                    const int32_t* rmask, const int32_t* gsrc, int gM) {
    if (M <= 0 || max_items <= 0) return 0;
    if (wt != WT_Q4_0 && wt != WT_Q8_0) return -1;
    if (part == nullptr || part_bytes < (size_t) M * N * sizeof(float)) return -1;
    if (gsrc && gM <= 0) return -1;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.part = part;
    a.items = items; a.count = count; a.wstride = wstride; a.rmask = rmask;
    a.gsrc = gsrc; a.gM = gM;
    a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
    a.nstripes = (N + 15) / 16; a.ngroups = (K / 32 + 3) / 4; a.ks = 1; a.gps = a.ngroups;
    a.mtiles = (M + 15) / 16;
    // the streaming kernel, one slice (K of at most 16 groups). Q4_0: 4 stripes a wavefront past 8 groups, else 2
    // (Qwen3-30B-A3B at 32 rows, µs a launch against the ring kernel's 46.4 / 26.4: gate|up 2048 -> 1536 columns
    // 43.0 with 4 stripes, 45.8 with 2; down 768 -> 2048 24.6 with 2, 25.9 with 4; deeper rings slower)
    if (a.ngroups <= 16) {
        const int gs = wt == WT_Q8_0 ? 1 : a.ngroups > 8 ? 4 : 2;
        const dim3 grid((a.nstripes + 4 * gs - 1) / (4 * gs), 1, max_items);
        if (wt == WT_Q8_0 ? launch_grouped_s<WT_Q8_0>(gs, a.ngroups, grid, a, st)
                          : launch_grouped_s<WT_Q4_0>(gs, a.ngroups, grid, a, st))
            return 1;
    }
    // (K past 16 groups) the ring kernel. Q4_0: 2 stripes a wavefront; Q8_0 tiles take one (twice the weight
    // registers)
    if (wt == WT_Q8_0) {
        hipLaunchKernelGGL((k_q4_gemm<WT_Q8_0, 1, 1, false, true>), dim3((a.nstripes + 3) / 4, 1, max_items), dim3(256), 0,
                           st, GSG_ARGS(a));
    } else {
        hipLaunchKernelGGL((k_q4_gemm<WT_Q4_0, 1, 2, false, true>), dim3((a.nstripes + 7) / 8, 1, max_items), dim3(256), 0,
                           st, GSG_ARGS(a));
    }
    return 1;
}

bool q4_gemm_grouped_swiglu_fits(int N, int K, int wt) {
    return wt == WT_Q4_0 && N > 0 && N % 256 == 0 && K > 0 && (K / 32 + 3) / 4 <= 16;
}
int q4_gemm_grouped_swiglu(const uint8_t* w, size_t wstride, const int32_t* items, const int32_t* count, int max_items,
                           const uint8_t* xa, int M, int N, int K, uint8_t* xo, hipStream_t st, int wt,
                           const int32_t* rmask, const int32_t* gsrc, int gM) {
    if (!q4_gemm_grouped_swiglu_fits(N, K, wt)) return 0;
    if (M <= 0 || max_items <= 0) return 1;  // (nothing to do)
    if (xo == nullptr || xo == xa || (gsrc && gM <= 0)) return -1;
    const int ngroups = (K / 32 + 3) / 4;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.xo = xo;
    a.items = items; a.count = count; a.wstride = wstride; a.rmask = rmask;
    a.gsrc = gsrc; a.gM = gM;
    a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
    a.nstripes = N / 16; a.ngroups = ngroups; a.ks = 1; a.gps = ngroups;
    a.mtiles = (M + 15) / 16;
    const dim3 grid(a.nstripes / 16, 1, max_items);
    if (ngroups <= 8) hipLaunchKernelGGL((k_q4_gemm_s<WT_Q4_0, 1, 4, 2, 8, FE_GSWIGLU>), grid, dim3(256), 0, st, GSG_ARGS(a));
    else hipLaunchKernelGGL((k_q4_gemm_s<WT_Q4_0, 1, 4, 2, 16, FE_GSWIGLU>), grid, dim3(256), 0, st, GSG_ARGS(a));
    return 1;
}

bool q4_gemm_swiglu_fits(int M, int N, int K, int wt) {
    if (wt != WT_Q4_0 || M < Q4_PAIR_ROWS || N % 256 != 0) return false;
    const GemmPlan p = q4_plan(N, K, wt);
    return p.ks > 1 && p.spw == 1 && p.gps % 2 == 0 && p.nstripes >= 384;  // (the FK walk's shapes)
}

int q4_gemm_swiglu(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* h, uint8_t* xo, hipStream_t st,
                   int wt) {
    if (!q4_gemm_swiglu_fits(M, N, K, wt) || xo == xa || h == nullptr || xo == nullptr) return 0;
    const GemmPlan p = q4_plan(N, K, wt);
    GemmArgs a{};
    a.w = w; a.xa = xa; a.h = h; a.xo = xo;
    a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
    a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps;
    a.mtiles = (M + 15) / 16;
    const dim3 grid((p.nstripes + 7) / 8, 1, (a.mtiles + 1) / 2);
    hipLaunchKernelGGL((k_q4_gemm_fk2<WT_Q4_0, 2, 2, true>), grid, dim3(256), 0, st, GS_ARGS(a));
    return 1;
}

void q4_reduce_slices(const float* part, int ks, int M, int N, float* y, hipStream_t st) {
    GemmArgs a{};
    a.part = const_cast<float*>(part); a.y = y;
    a.M = M; a.N = N; a.ldy = N; a.epi = EPI_STORE; a.ks = ks;
    hipLaunchKernelGGL(k_q4_reduce, dim3((M * N + 255) / 256), dim3(256), 0, st, a);
}

int q4_gemm(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* y, int ldy, int epi, float* ws,
            size_t ws_bytes, hipStream_t st, int wt) {
    if (M <= 0) return 0;
    const int ks = q4_gemm_raw(w, xa, M, N, K, ws, ws_bytes, st, wt);
    if (ks < 0) return -1;
    GemmArgs a{};
    a.part = ws; a.y = y;
    a.M = M; a.N = N; a.K = K; a.ldy = ldy; a.epi = epi; a.ks = ks;
    const int tot = M * (epi == EPI_SWIGLU ? N / 2 : N);
    hipLaunchKernelGGL(k_q4_reduce, dim3((tot + 255) / 256), dim3(256), 0, st, a);
    return 0;
}

// ---------------------------------------------------------------------------------------------------------------------
// the matmul without allocation (snk_q4_gemm_noalloc): the k-slice partials in a fixed device array

// Each GPU the library runs on holds its own copy of this array, from the code object's load until the process ends.
// Host code never passes `scratch` itself (in host code the name is a stand-in, not a device address): it looks up the
// current device's copy once with hipGetSymbolAddress and passes that address.
#define Q4_SCRATCH_BYTES (32u << 20)
static __device__ __align__(256) uint8_t scratch[Q4_SCRATCH_BYTES];

// the current device's copy of `scratch`, looked up on the first call on that device (with it current) and kept
static float* q4_scratch(char* err, int err_len) {
    static std::mutex mu;
    static void* addr[64];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        sn_set_err(err, err_len, "snk_q4_gemm_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            sn_set_err(err, err_len, "snk_q4_gemm_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: "
                       "%s", dev, hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = p;
    }
    return (float*) addr[dev];
}

// snk_q4_gemm with the partials in the device's scratch array: the same kernels, the same slices in the same order, so
// the same bits. Nothing in the array has to start at zero: every partial the reduction reads is written first by the
// same call's matmul. Calls that overlap on one GPU (other streams, other threads) share the array and race.
extern "C" int snk_q4_gemm_noalloc(const void* d_stripes, const void* d_xa, int M, int N, int K, float* d_y, int ldy,
                                   int epi, void* stream, char* err, int err_len) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 32 || epi < 0 || epi > 2 ||
        (epi == EPI_SWIGLU ? (N % 32 != 0 || ldy < N / 2) : ldy < N)) {
        sn_set_err(err, err_len, "snk_q4_gemm_noalloc: bad shape (M %d, N %d, K %d, ldy %d, epi %d)", M, N, K, ldy, epi);
        return -1;
    }
    const size_t need = q4_workspace_bytes(M, N, K);
    if (need > Q4_SCRATCH_BYTES) {
        sn_set_err(err, err_len, "snk_q4_gemm_noalloc: %d x %d x %d needs %zu bytes of k-slice partials; the scratch "
                   "array holds %u", M, N, K, need, Q4_SCRATCH_BYTES);
        return -1;
    }
    float* ws = q4_scratch(err, err_len);
    if (!ws) return -1;
    // the error state is read, not cleared: a state HIP held before the call stays the caller's, and only a change of
    // it during the launches is this call's failure
    const hipError_t before = hipPeekAtLastError();
    const int rc = q4_gemm((const uint8_t*) d_stripes, (const uint8_t*) d_xa, M, N, K, d_y, ldy, epi, ws,
                           Q4_SCRATCH_BYTES, (hipStream_t) stream);
    const hipError_t after = hipPeekAtLastError();
    if (rc != 0) {
        sn_set_err(err, err_len, "snk_q4_gemm_noalloc: no launch plan for %d x %d x %d", M, N, K);
        return -1;
    }
    if (after != hipSuccess && after != before) {
        sn_set_err(err, err_len, "snk_q4_gemm_noalloc: launch failed: %s", hipGetErrorString(after));
        return -1;
    }
    return 0;
}

void q4_repack(const uint8_t* src, int N, int K, uint8_t* dst, int sstride, int soff, hipStream_t st, int wt) {
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    if (wt == WT_Q8_0) hipLaunchKernelGGL(k_q8_repack, dim3(tiles), dim3(64), 0, st, src, N, K, dst, sstride, soff);
    else hipLaunchKernelGGL(k_q4_repack, dim3(tiles), dim3(64), 0, st, src, N, K, dst, sstride, soff);
}

template <int IT>
static void launch_resid(int km, int nt, float* x, const float* part, int ks, int M, int K, const float* nw, float eps,
                         uint8_t* xa, int ad, float* xn, hipStream_t st, const WeightPrefetch& pf, int npf) {
#define RQ(KM_)                                                                                                     \
    hipLaunchKernelGGL((k_resid_quant<IT, KM_>), dim3(M + npf), dim3(nt), 0, st, x, part, ks, M, K, nw, eps, xa, ad, xn, \
                       (const int32_t*) nullptr, (const float*) nullptr, pf)
    if (km == 1) RQ(1);
    else if (km == 2) RQ(2);
    else if (km == 4) RQ(4);
    else if (km == 8) RQ(8);
    else if (km == 10) RQ(10);
    else RQ(16);
#undef RQ
}

int resid_quant(float* x, const float* part, int ks, int M, int K, const float* nw, float eps, uint8_t* xa,
                hipStream_t st, bool add, float* xn, const uint8_t* next_w, int next_N, int next_K, int wt) {
    if (M <= 0) return 0;
    // (next_w: the next matmul's first groups into the Infinity Cache by extra workgroups; decode-sized rows only,
    // where that matmul streams its slices)
    WeightPrefetch pf{};
    int npf = 0;
    if (next_w && M < Q4_PAIR_ROWS) {
        const GemmPlan p = q4_plan(next_N, next_K, wt);
        const int tb = wt_tile_bytes(wt);
        if (p.stream) {
            pf.w = next_w, pf.nranges = p.nstripes * p.ks, pf.ks = p.ks, pf.sbytes = p.ngroups * tb;
            // (the groups of each slice a wavefront's ring loads first; each slice's first group alone: the matmuls
            // gained 30 against 61 us a step, the row kernels lost 36 against 45)
            pf.gstep = p.gps * tb, pf.lines = (std::min(p.sd, p.gps) * tb + 127) / 128;
            pf.total = (uint32_t) ((size_t) p.nstripes * pf.sbytes);
            npf = (int) (((long) pf.nranges * pf.lines + 256L * WP_LINES - 1) / (256L * WP_LINES));
        }
    }
    // 4 lanes per block of the padded row, in whole wavefronts, at most 1024 lanes (then IT passes)
    const int lanes = 4 * xa_nbp(K), nt = std::min(1024, (lanes + 63) / 64 * 64), it = (lanes + nt - 1) / nt;
    // (10: the exact count of the deep down projections' plans, no clamped copies of the last slice loaded)
    const int km = ks == 9 || ks == 10 ? 10 : ks_bound(ks);
    if (K % 32 || it > 4 || (xn && !xa) || km == 0) return -1;
    const int ad = add ? 1 : 0;
    if (it == 1) launch_resid<1>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st, pf, npf);
    else if (it == 2) launch_resid<2>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st, pf, npf);
    else launch_resid<4>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st, pf, npf);
    return 0;
}

int moe_resid_quant(float* x, const float* y, const int32_t* prow, const float* w, int k, int M, int K, const float* nw,
                    float eps, uint8_t* xa, hipStream_t st) {
    if (M <= 0) return 0;
    const int lanes = 4 * xa_nbp(K), nt = std::min(1024, (lanes + 63) / 64 * 64), it = (lanes + nt - 1) / nt;
    if (K % 32 || it > 4 || k < 1 || k > MOE_MAX_K) return -1;
#define MQ(IT_) hipLaunchKernelGGL((k_resid_quant<IT_, 1, true>), dim3(M), dim3(nt), 0, st, x, y, k, M, K, nw, eps, xa, 1, \
                                   (float*) nullptr, prow, w)
    if (it == 1) MQ(1);
    else if (it == 2) MQ(2);
    else MQ(4);
#undef MQ
    return 0;
}

#define SWQ_STAGE_ROWS 256  // rows from which k_swiglu_quant stages its sums through LDS
int swiglu_quant(const float* part, int ks, int M, int F, float* h, uint8_t* xa, hipStream_t st, const int32_t* rows) {
    if (M <= 0) return 0;
    const dim3 grid(M, (xa_nbp(F) + 63) / 64);
    const int km = ks_bound(ks);
    if (km == 0 || F % 32) return -1;
    auto go = [&](auto stage) {
        constexpr bool S = decltype(stage)::value;
        if (km == 1) hipLaunchKernelGGL((k_swiglu_quant<1, S>), grid, dim3(256), 0, st, part, ks, M, F, h, xa, rows);
        else if (km == 2) hipLaunchKernelGGL((k_swiglu_quant<2, S>), grid, dim3(256), 0, st, part, ks, M, F, h, xa, rows);
        else if (km == 4) hipLaunchKernelGGL((k_swiglu_quant<4, S>), grid, dim3(256), 0, st, part, ks, M, F, h, xa, rows);
        else if (km == 8) hipLaunchKernelGGL((k_swiglu_quant<8, S>), grid, dim3(256), 0, st, part, ks, M, F, h, xa, rows);
        else hipLaunchKernelGGL((k_swiglu_quant<16, S>), grid, dim3(256), 0, st, part, ks, M, F, h, xa, rows);
    };
    if (M >= SWQ_STAGE_ROWS) go(std::true_type{});
    else go(std::false_type{});
    return 0;
}

void quant_act(const float* x, const int32_t* rows, int M, int K, int ldx, const float* nw, float eps, uint8_t* xa,
               float* xn, int ldn, hipStream_t st) {
    if (M <= 0) return;
    hipLaunchKernelGGL(k_quant_act, dim3(M, (xa_nbp(K) + 63) / 64), dim3(256), 0, st, x, rows, M, K, ldx, nw, eps, xa,
                       xn, ldn);
}

// ---------------------------------------------------------------------------------------------------------------------
// checks: the matmul's own dequantization written out, and one MFMA's lane contents
__global__ void k_q4_dequant(const uint8_t* __restrict__ w, int N, int K, float* __restrict__ out) {
    const int nb = K / 32, ngroups = (nb + 3) / 4;
    const int tile = blockIdx.x, stripe = tile / ngroups, grp = tile % ngroups;
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4, row = stripe * 16 + n;
    const uint8_t* tp = w + (size_t) tile * Q4T_BYTES;
    const u32x4 wq = *(const u32x4*) (tp + 16 * lane);
    const half4v sc = *(const half4v*) (tp + Q4T_SCALE_OFF + 8 * n);
    const float dw[4] = {(float) sc[0], (float) sc[1], (float) sc[2], (float) sc[3]};
    for (int b = 0; b < 4; ++b) {
        const int blk = 4 * grp + b;
        if (row >= N || blk >= nb) continue;
        const half8 q = q4_unpack(wq[b]);  // (1024 + w) for elements 4g.., (1024 + 16 w) for 16 + 4g..
        for (int j = 0; j < 8; ++j) {
            const int e = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
            const float w8 = j < 4 ? (float) q[j] - 1032.0f : ((float) q[j] - 1152.0f) * 0.0625f;  // w - 8, exactly
            out[(size_t) row * K + 32 * blk + e] = w8 * dw[b];
        }
    }
}

__global__ void k_q8_dequant(const uint8_t* __restrict__ w, int N, int K, float* __restrict__ out) {
    const int nb = K / 32, ngroups = (nb + 3) / 4;
    const int tile = blockIdx.x, stripe = tile / ngroups, grp = tile % ngroups;
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4, row = stripe * 16 + n;
    const uint8_t* tp = w + (size_t) tile * Q8T_BYTES;
    const u32x4 w0 = *(const u32x4*) (tp + 32 * lane), w1 = *(const u32x4*) (tp + 32 * lane + 16);
    const half4v sc = *(const half4v*) (tp + Q8T_SCALE_OFF + 8 * n);
    for (int b = 0; b < 4; ++b) {
        const int blk = 4 * grp + b;
        if (row >= N || blk >= nb) continue;
        const u32x4 wv = b < 2 ? w0 : w1;
        const half8 q = q8_unpack(wv[2 * (b % 2)], wv[2 * (b % 2) + 1]);  // 1024 + u, 16 (1024 + u); u = q + 128
        for (int j = 0; j < 8; ++j) {
            const int e = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
            const float qv = j < 4 ? (float) q[j] - 1152.0f : (float) q[j] * 0.0625f - 1152.0f;  // q, exactly
            out[(size_t) row * K + 32 * blk + e] = qv * (float) sc[b];
        }
    }
}

extern "C" int snk_q8_dequant(const void* d_tiles, int N, int K, float* d_w, void* stream) {
    if (N <= 0 || K <= 0 || K % 32) return -1;
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    hipLaunchKernelGGL(k_q8_dequant, dim3(tiles), dim3(64), 0, (hipStream_t) stream, (const uint8_t*) d_tiles, N, K,
                       d_w);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int snk_q4_dequant(const void* d_stripes, int N, int K, float* d_w, void* stream) {
    if (N <= 0 || K <= 0 || K % 32) return -1;
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    hipLaunchKernelGGL(k_q4_dequant, dim3(tiles), dim3(64), 0, (hipStream_t) stream, (const uint8_t*) d_stripes, N, K,
                       d_w);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// A plain streaming read of `n4` 16-byte words: every lane loads RF words 4 KB apart, all issued before any is used,
// one workgroup per 256 x RF words, so every load of the launch is in flight at once (16 KB a workgroup; the sum is kept
// live by a store that only a sum of exactly 1234.5 makes). The time this box takes to read a buffer of that size in
// one launch: the floor against which a matmul of the same weight bytes is measured.
#define RF 4
__global__ __launch_bounds__(256) void k_read_floor(const float4* __restrict__ src, size_t n4, float* __restrict__ sink) {
    float4 v[RF];
    const size_t base = (size_t) blockIdx.x * 256 * RF + threadIdx.x;
    for (int r = 0; r < RF; ++r) v[r] = src[min(base + 256 * r, n4 - 1)];
    float s = 0.0f;
    for (int r = 0; r < RF; ++r) s += (v[r].x + v[r].y) + (v[r].z + v[r].w);
    if (s == 1234.5f) sink[threadIdx.x] = s;
}

void read_floor(const void* buf, size_t bytes, float* sink, hipStream_t st) {
    const size_t n4 = bytes / 16;
    const size_t grid = (n4 + 256 * RF - 1) / (256 * RF);
    hipLaunchKernelGGL(k_read_floor, dim3((unsigned) grid), dim3(256), 0, st, (const float4*) buf, n4, sink);
}

__global__ void k_mfma_probe(const half8* a, const half8* b, floatx4* d) {
    const int l = threadIdx.x;
    const floatx4 z = {0.f, 0.f, 0.f, 0.f};
    d[l] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[l], b[l], z, 0, 0, 0);
}

extern "C" int snk_mfma_probe(const void* d_a, const void* d_b, float* d_d, void* stream) {
    hipLaunchKernelGGL(k_mfma_probe, dim3(1), dim3(64), 0, (hipStream_t) stream, (const half8*) d_a, (const half8*) d_b,
                       (floatx4*) d_d);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
