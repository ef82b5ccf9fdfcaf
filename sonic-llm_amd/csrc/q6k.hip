// Q6_K weights (the LM head of real Qwen3 GGUFs, tied to a Q6_K token table) on gfx950: the tile repack, Q8_K
// activation records, the matmul, and its own dequantization for the bit-exactness check.
//
// The arithmetic is ggml's CPU vec_dot_q6_K_q8_K: activations quantized to Q8_K (256-element blocks, fp32 d, int8 q,
// quantize_row_q8_K_ref), per block the exact integer sum over 16-element groups of scale_g * sum (q6 - 32) * q8, then
// acc += isum * (d6 * d8). Here one v_mfma_f32_16x16x16_f16 per group gives that group's integer dot exactly: the
// weight lane's 4 six-bit quants become fp16 (1024 + q6) by masks and byte permutes, the activation fragment holds q8 as
// fp16, and the MFMA's C input is the group's correction -1056 * sum q8, so the result is sum q8 * (q6 - 32) (every
// term and partial sum an integer below 2^24).
#include "sn_kernels_internal.h"

// ---- tiles: 16 rows x one 256-element block, 3360 bytes (= 16 x 210, the GGUF bytes) --------------------------------
// Lane l = n + 16 g (row n of the tile, g = 0..3) owns elements 16 G + 4 g + j (j = 0..3) of every group G = 0..15 of
// row n's block, 48 bytes at 48 l:
//   dwords 0..7: dword k, byte j: low nibble = the low 4 bits of element j of group 2k, high nibble = of group 2k + 1;
//   dwords 8..11: dword 8 + k, byte j: bits 2i, 2i + 1 = the high 2 bits of element j of group 4k + i (i = 0..3).
// Then the 16 rows' int8 scales (16 a row, at 3072 + 16 n) and fp16 d (at 3328 + 2 n).
// A block_q6_K element e (half h = e / 128, quarter c = (e % 128) / 32, l = e % 32) has its low 4 bits in
// ql[64 h + 32 (c & 1) + l] (the low nibble for c < 2, high for c >= 2) and its high 2 bits at bit 2c of qh[32 h + l].
__device__ __forceinline__ int q6_low4(const uint8_t* blk, int e) {
    const int h = e >> 7, c = (e & 127) >> 5, l = e & 31;
    const uint8_t b = blk[64 * h + 32 * (c & 1) + l];
    return c < 2 ? (b & 15) : (b >> 4);
}
__device__ __forceinline__ int q6_high2(const uint8_t* blk, int e) {
    const int h = e >> 7, c = (e & 127) >> 5, l = e & 31;
    return (blk[128 + 32 * h + l] >> (2 * c)) & 3;
}

// grid (stripes, blocks), 64 threads: lane l writes its 48 bytes; lanes 0..15 also row l's scales and d
__global__ __launch_bounds__(64) void k_q6k_repack(const uint8_t* __restrict__ src, int N, int K,
                                                   uint8_t* __restrict__ dst) {
    const int stripe = blockIdx.x, b = blockIdx.y, nb = K / 256, lane = threadIdx.x;
    const int n = lane & 15, g = lane >> 4, row = stripe * 16 + n;
    uint8_t* tile = dst + ((size_t) stripe * nb + b) * Q6T_BYTES;
    uint32_t w[12] = {0};
    if (row < N) {
        const uint8_t* blk = src + ((size_t) row * nb + b) * 210;
        for (int k = 0; k < 8; ++k)
            for (int j = 0; j < 4; ++j) {
                const int e0 = 16 * (2 * k) + 4 * g + j, e1 = 16 * (2 * k + 1) + 4 * g + j;
                w[k] |= (uint32_t) (q6_low4(blk, e0) | (q6_low4(blk, e1) << 4)) << (8 * j);
            }
        for (int k = 0; k < 4; ++k)
            for (int j = 0; j < 4; ++j) {
                uint32_t v = 0;
                for (int i = 0; i < 4; ++i) v |= (uint32_t) q6_high2(blk, 16 * (4 * k + i) + 4 * g + j) << (2 * i);
                w[8 + k] |= v << (8 * j);
            }
        if (g == 0) {
            for (int i = 0; i < 16; ++i) tile[Q6T_SCALE_OFF + 16 * n + i] = blk[192 + i];
            tile[Q6T_D_OFF + 2 * n] = blk[208];
            tile[Q6T_D_OFF + 2 * n + 1] = blk[209];
        }
    } else if (g == 0) {
        for (int i = 0; i < 16; ++i) tile[Q6T_SCALE_OFF + 16 * n + i] = 0;
        tile[Q6T_D_OFF + 2 * n] = 0;
        tile[Q6T_D_OFF + 2 * n + 1] = 0;
    }
    for (int k = 0; k < 12; ++k) *(uint32_t*) (tile + 48 * lane + 4 * k) = w[k];
}

// The 4 six-bit quants of group G of this lane as fp16 (1024 + q6), from its dwords: lo4 = the low nibbles, hi2 = the
// high 2 bits moved to bits 4..5 of each byte, one OR, then two byte permutes with 0x64 (the high byte of fp16 1024).
__device__ __forceinline__ half4v q6_unpack(const uint32_t (&w)[12], int G) {
    const uint32_t lo = w[G >> 1], hw = w[8 + (G >> 2)];
    const uint32_t lo4 = (G & 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
    const int sh = 2 * (G & 3);  // bits sh, sh + 1 of each byte -> bits 4, 5
    const uint32_t hi2 = sh <= 4 ? (hw << (4 - sh)) & 0x30303030u : (hw >> (sh - 4)) & 0x30303030u;
    const uint32_t q = lo4 | hi2;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, q, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, q, 0x04030402u);
    return __builtin_bit_cast(half4v, (u32x2){p0, p1});
}

// the tiles dequantized back with the matmul's own unpack: (d * scale) * (q6 - 32) in fp32 (dequantize_row_q6_K)
__global__ __launch_bounds__(64) void k_q6k_dequant(const uint8_t* __restrict__ tiles, int N, int K,
                                                    float* __restrict__ out) {
    const int stripe = blockIdx.x, b = blockIdx.y, nb = K / 256, lane = threadIdx.x;
    const int n = lane & 15, g = lane >> 4, row = stripe * 16 + n;
    const uint8_t* tile = tiles + ((size_t) stripe * nb + b) * Q6T_BYTES;
    uint32_t w[12];
    for (int k = 0; k < 12; ++k) w[k] = *(const uint32_t*) (tile + 48 * lane + 4 * k);
    const float d = (float) *(const _Float16*) (tile + Q6T_D_OFF + 2 * n);
    if (row >= N) return;
    for (int G = 0; G < 16; ++G) {
        const half4v h = q6_unpack(w, G);
        const float ds = d * (float) (int8_t) tile[Q6T_SCALE_OFF + 16 * n + G];
        for (int j = 0; j < 4; ++j)
            out[(size_t) row * K + 256 * b + 16 * G + 4 * g + j] = ds * (float) ((int) (float) h[j] - 1056);
    }
}

// ---- Q8_K activation records ----------------------------------------------------------------------------------------
// Row m, block b of an operand of K (K % 256 == 0) from its 256 fp32 values, one per thread of a 256-thread workgroup
// (thread t = element t): ggml quantize_row_q8_K_ref (max = the value of largest |x|, the first on ties; iscale =
// -127 / max; q = min(127, round-half-even(iscale * x)); d = 1 / iscale; an all-zero block: d = 0, q = 0). Writes the
// thread's q into its fragment slot and, per group, the correction -1056 * sum q, and d.
__device__ __forceinline__ void q8k_store(float v, uint8_t* xk, int K, int m, int b, float* red_a, int* red_i,
                                          float* s_max) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    // the block's extreme: |x| max, the lowest element on ties
    float a = fabsf(v);
    int i = t;
    for (int o = 32; o > 0; o >>= 1) {
        const float oa = __shfl_xor(a, o);
        const int oi = __shfl_xor(i, o);
        if (oa > a || (oa == a && oi < i)) {
            a = oa;
            i = oi;
        }
    }
    __syncthreads();  // (the reduction arrays are reused block after block)
    if (lane == 0) {
        red_a[w] = a;
        red_i[w] = i;
    }
    __syncthreads();
    float amax = red_a[0];
    int imax = red_i[0];
    for (int k = 1; k < 4; ++k)
        if (red_a[k] > amax || (red_a[k] == amax && red_i[k] < imax)) {
            amax = red_a[k];
            imax = red_i[k];
        }
    if (t == imax) *s_max = v;
    __syncthreads();
    const float mx = *s_max;
    float q = 0.0f, d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.f / mx;
        q = fminf(127.f, __builtin_rintf(iscale * v));
        d = 1 / iscale;
    }
    // the group's sum (16 consecutive threads)
    float s = q;
    for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o);
    uint8_t* rec = xk + xk_rec_off(K, m, b);
    const int G = t >> 4, e = t & 15, g = e >> 2, j = e & 3;
    *(_Float16*) (rec + G * 512 + 8 * ((m & 15) + 16 * g) + 2 * j) = (_Float16) q;
    if (e == 0) *(float*) (rec + XK_CORR_OFF + G * 64 + 4 * (m & 15)) = -1056.0f * s;
    if (t == 0) *(float*) (rec + XK_D_OFF + 4 * (m & 15)) = d;
}

// grid (rows M), 256 threads: row m (source rows[m] of X when given) RMS-normed by nw when given (scale 1/sqrt(mean
// x^2 + eps), the activation quantizer's) and quantized block by block into Q8_K records.
__global__ __launch_bounds__(256) void k_quant_q8k(const float* __restrict__ X, const int32_t* __restrict__ rows,
                                                   int K, int ldx, const float* __restrict__ nw, float eps,
                                                   uint8_t* __restrict__ xk) {
    __shared__ float red_a[4];
    __shared__ int red_i[4];
    __shared__ float red_s[4];
    __shared__ float s_max;
    const int m = blockIdx.x, t = threadIdx.x;
    const float* x = X + (size_t) (rows ? rows[m] : m) * ldx;
    float scale = 1.0f;
    if (nw) {
        float s = 0.0f;
        for (int i = t; i < K; i += 256) s += x[i] * x[i];
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if ((t & 63) == 0) red_s[t >> 6] = s;
        __syncthreads();
        s = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
        scale = 1.0f / sqrtf(s / (float) K + eps);
    }
    for (int b = 0; b < K / 256; ++b) {
        const int i = 256 * b + t;
        const float v = nw ? (x[i] * scale) * nw[i] : x[i];
        q8k_store(v, xk, K, m, b, red_a, red_i, &s_max);
    }
}

// ---- the matmul -------------------------------------------------------------------------------------------------
// One workgroup (4 wavefronts) owns 4 consecutive 16-row stripes (wavefront w: stripe 4 set + w), MT row tiles and all
// of K; the blocks are walked in order. Block b + 1's weights go into a second register slot and block b + 2's
// activation records into registers while block b is summed; block b + 1's records are stored into an LDS double
// buffer at the top of the iteration. Per (block, group, row tile): one MFMA 16x16x16 f16 with the group's correction
// as C input (the exact integer dot), then isum += scale * dot; per block acc += isum * (d6 * d8). The logits go
// straight to y (no k-split).
#define XK_PER_THREAD ((2 * XK_REC / 16 + 255) / 256)  // 16-byte pieces of two row tiles' records a thread stages
template <int MT>
__global__ __launch_bounds__(256) void k_q6k_gemm(const uint8_t* __restrict__ tiles, const uint8_t* __restrict__ xk,
                                                  int M, int N, int K, int mt_first, float* __restrict__ y, int ldy) {
    __shared__ __attribute__((aligned(16))) uint8_t s_rec[2][MT][XK_REC];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int nb = K / 256, nstripes = (N + 15) / 16;
    const int stripe = blockIdx.x * 4 + wave;
    const int mt0 = mt_first + blockIdx.y * MT;
    const int nvalid = __builtin_amdgcn_readfirstlane(stripe < nstripes ? 1 : 0);
    const __amdgpu_buffer_rsrc_t wr =
        buf_rsrc(tiles + (size_t) min(stripe, nstripes - 1) * nb * Q6T_BYTES, (uint32_t) (nvalid * nb * Q6T_BYTES));
    // this workgroup's records: MT row tiles x nb blocks, row tile mt's block b at (mt * nb + b) * XK_REC
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(xk + (size_t) mt0 * nb * XK_REC, (uint32_t) ((size_t) MT * nb * XK_REC));
    constexpr int PIECES = MT * XK_REC / 16;  // 16-byte pieces of one block's records

    u32x4 wq[2][3];
    u32x4 sc4[2];
    uint32_t dw[2];
    u32x4 rr[XK_PER_THREAD];
    auto load_w = [&](int slot, int b) {
        const int so = min(b, nb - 1) * Q6T_BYTES;
        for (int k = 0; k < 3; ++k) wq[slot][k] = bload16(wr, 48 * lane + 16 * k, so);
        sc4[slot] = bload16(wr, Q6T_SCALE_OFF + 16 * n, so);
        dw[slot] = __builtin_bit_cast(uint32_t, bload4f(wr, Q6T_D_OFF + 4 * (n >> 1), so));
    };
    // block b's records into registers (piece i of row tile i / (XK_REC / 16)), every load issued (index clamped)
    auto load_r = [&](int b) {
        const int bb = min(b, nb - 1);
        for (int k = 0; k < XK_PER_THREAD; ++k) {
            const int i = min((int) threadIdx.x + 256 * k, PIECES - 1), mt = i / (XK_REC / 16), o = i % (XK_REC / 16);
            rr[k] = bload16(xr, 16 * o, (mt * nb + bb) * XK_REC);
        }
    };
    auto store_r = [&](int buf) {
        for (int k = 0; k < XK_PER_THREAD; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < PIECES) *(u32x4*) &s_rec[buf][i / (XK_REC / 16)][16 * (i % (XK_REC / 16))] = rr[k];
        }
    };

    floatx4 acc[MT];
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    load_r(0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_r(0);
    __builtin_amdgcn_sched_barrier(0);
    load_r(1);
    for (int b = 0; b < nb; ++b) {
        const int cur = b & 1;
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // block b's records are in buffer cur; everyone is done reading the other buffer
        store_r(cur ^ 1);  // block b + 1's (unused past the last block)
        __builtin_amdgcn_sched_barrier(0);
        load_r(b + 2);
        __builtin_amdgcn_sched_barrier(0);
        load_w(cur ^ 1, b + 1);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t w[12];
        for (int k = 0; k < 3; ++k)
            for (int i = 0; i < 4; ++i) w[4 * k + i] = wq[cur][k][i];
        floatx4 isum[MT];
        for (int mt = 0; mt < MT; ++mt) isum[mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
        for (int G = 0; G < 16; ++G) {
            const half4v bw = q6_unpack(w, G);
            const float s = (float) (int8_t) (sc4[cur][G >> 2] >> (8 * (G & 3)));
            for (int mt = 0; mt < MT; ++mt) {
                const half4v a = *(const half4v*) &s_rec[cur][mt][G * 512 + 8 * lane];
                const floatx4 cr = *(const floatx4*) &s_rec[cur][mt][XK_CORR_OFF + G * 64 + 16 * g];
                const floatx4 dot = __builtin_amdgcn_mfma_f32_16x16x16f16(a, bw, cr, 0, 0, 0);
                for (int v = 0; v < 4; ++v) isum[mt][v] = __builtin_fmaf(s, dot[v], isum[mt][v]);
            }
        }
        const float d6 = (float) __builtin_bit_cast(_Float16, (uint16_t) (dw[cur] >> (16 * (n & 1))));
        for (int mt = 0; mt < MT; ++mt) {
            const floatx4 d8 = *(const floatx4*) &s_rec[cur][mt][XK_D_OFF + 16 * g];
            for (int v = 0; v < 4; ++v) acc[mt][v] = __builtin_fmaf(isum[mt][v], d6 * d8[v], acc[mt][v]);
        }
    }
    // lane (n, g) holds rows 4g + v of each row tile, column n of the stripe
    const int col = stripe * 16 + n;
    if (stripe >= nstripes || col >= N) return;
    for (int mt = 0; mt < MT; ++mt)
        for (int v = 0; v < 4; ++v) {
            const int row = (mt0 + mt) * 16 + 4 * g + v;
            if (row < M) y[(size_t) row * ldy + col] = acc[mt][v];
        }
}

// ---- host side ----------------------------------------------------------------------------------------------------
void q6k_repack(const uint8_t* src, int N, int K, uint8_t* dst, hipStream_t st) {
    hipLaunchKernelGGL(k_q6k_repack, dim3((N + 15) / 16, K / 256), dim3(64), 0, st, src, N, K, dst);
}
void q6k_dequant(const uint8_t* tiles, int N, int K, float* out, hipStream_t st) {
    hipLaunchKernelGGL(k_q6k_dequant, dim3((N + 15) / 16, K / 256), dim3(64), 0, st, tiles, N, K, out);
}
void quant_q8k(const float* x, const int32_t* rows, int M, int K, int ldx, const float* nw, float eps, uint8_t* xk,
               hipStream_t st) {
    if (M > 0) hipLaunchKernelGGL(k_quant_q8k, dim3(M), dim3(256), 0, st, x, rows, K, ldx, nw, eps, xk);
}
int q6k_gemm(const uint8_t* tiles, const uint8_t* xk, int M, int N, int K, float* y, int ldy, hipStream_t st) {
    if (M <= 0) return 0;
    if (K % 256 || N <= 0) return -1;
    const int mtiles = (M + 15) / 16, sets = ((N + 15) / 16 + 3) / 4;
    // row tiles in pairs (the records are padded to an even count), a last odd tile alone
    const int pairs = mtiles / 2;
    if (pairs > 0) hipLaunchKernelGGL(k_q6k_gemm<2>, dim3(sets, pairs), dim3(256), 0, st, tiles, xk, M, N, K, 0, y, ldy);
    if (mtiles & 1)
        hipLaunchKernelGGL(k_q6k_gemm<1>, dim3(sets, 1), dim3(256), 0, st, tiles, xk, M, N, K, mtiles - 1, y, ldy);
    return 0;
}
