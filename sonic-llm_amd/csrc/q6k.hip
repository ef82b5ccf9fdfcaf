// Q6_K weights (the LM head of real Qwen3 GGUFs, tied to a Q6_K token table) on gfx950: the tile repack, Q8_K
// activation records, the matmul, and its own dequantization for the bit-exactness check.
//
// The arithmetic is ggml's CPU vec_dot_q6_K_q8_K: activations quantized to Q8_K (256-element blocks, fp32 d, int8 q,
// quantize_row_q8_K_ref), per block the exact integer sum over 16-element groups of scale_g * sum (q6 - 32) * q8, then
// acc += isum * (d6 * d8). Here one v_mfma_i32_32x32x16_i8 per group (its K is the group's 16 elements) gives the
// group's dot for 32 activation rows x 32 weight rows as exact int32, the weight lane's 8 six-bit quants turned into
// int8 (q6 - 32) by masks, shifts and one byte-wise subtract; isum += scale * dot stays in int32 (|isum| < 2^31), as
// ggml's aux32 does.
#include "sn_kernels_internal.h"

typedef int int32x16 __attribute__((ext_vector_type(16)));

// ---- tiles: 32 rows x one 256-element block, 6720 bytes (= 32 x 210, the GGUF bytes) --------------------------------
// Lane l = n + 32 h (row n of the tile, h = 0, 1) owns elements 16 G + 8 h + j (j = 0..7) of every group G = 0..15 of
// row n's block: 96 bytes = 24 dwords, dwords 4k..4k+3 at byte 1024 k + 16 l (a wavefront's 16-byte load reads 1 KB
// contiguous):
//   dword G (G = 0..15): byte i = the low 4 bits of element (G, i) | those of (G, i + 4) << 4;
//   dword 16 + p (p = 0..7): byte i = the high 2 bits of elements (2p, i), (2p, i + 4), (2p + 1, i), (2p + 1, i + 4) at
//   bits 0, 2, 4, 6  ((G, j) = element j of group G of this lane).
// Then the 32 rows' int8 scales (16 a row, at 6144 + 16 n) and fp16 d (at 6656 + 2 n).
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

// grid (stripes, blocks), 64 threads: lane l writes its 96 bytes; lanes 0..31 also row l's scales and d
__global__ __launch_bounds__(64) void k_q6k_repack(const uint8_t* __restrict__ src, int N, int K,
                                                   uint8_t* __restrict__ dst) {
    const int stripe = blockIdx.x, b = blockIdx.y, nb = K / 256, lane = threadIdx.x;
    const int n = lane & 31, h = lane >> 5, row = stripe * Q6T_ROWS + n;
    uint8_t* tile = dst + ((size_t) stripe * nb + b) * Q6T_BYTES;
    uint32_t w[24] = {0};
    if (row < N) {
        const uint8_t* blk = src + ((size_t) row * nb + b) * 210;
        auto el = [&](int G, int j) { return 16 * G + 8 * h + j; };
        for (int G = 0; G < 16; ++G)
            for (int i = 0; i < 4; ++i)
                w[G] |= (uint32_t) (q6_low4(blk, el(G, i)) | (q6_low4(blk, el(G, i + 4)) << 4)) << (8 * i);
        for (int p = 0; p < 8; ++p)
            for (int i = 0; i < 4; ++i) {
                const uint32_t v = q6_high2(blk, el(2 * p, i)) | q6_high2(blk, el(2 * p, i + 4)) << 2 |
                                   q6_high2(blk, el(2 * p + 1, i)) << 4 | q6_high2(blk, el(2 * p + 1, i + 4)) << 6;
                w[16 + p] |= v << (8 * i);
            }
        if (h == 0) {
            for (int i = 0; i < 16; ++i) tile[Q6T_SCALE_OFF + 16 * n + i] = blk[192 + i];
            tile[Q6T_D_OFF + 2 * n] = blk[208];
            tile[Q6T_D_OFF + 2 * n + 1] = blk[209];
        }
    } else if (h == 0) {
        for (int i = 0; i < 16; ++i) tile[Q6T_SCALE_OFF + 16 * n + i] = 0;
        tile[Q6T_D_OFF + 2 * n] = 0;
        tile[Q6T_D_OFF + 2 * n + 1] = 0;
    }
    for (int k = 0; k < 6; ++k)
        *(u32x4*) (tile + 1024 * k + 16 * lane) = (u32x4){w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
}

// Group G of this lane as 8 int8 (q6 - 32), element j in byte j: the low nibbles and the high 2 bits (moved to bits
// 4..5) ORed into bytes of 0..63, then v - 32 per byte: (v | 0x80) - 0x20 never borrows across bytes, and flipping
// bit 7 leaves v - 32 in two's complement.
__device__ __forceinline__ long q6_unpack(const uint32_t (&w)[24], int G) {
    const uint32_t lo = w[G], hw = w[16 + (G >> 1)];
    const int s0 = 4 * (G & 1);
    const uint32_t va = (lo & 0x0F0F0F0Fu) | (((hw >> s0) & 0x03030303u) << 4);
    const uint32_t vb = ((lo >> 4) & 0x0F0F0F0Fu) | (((hw >> (s0 + 2)) & 0x03030303u) << 4);
    const uint32_t ra = ((va | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
    const uint32_t rb = ((vb | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
    return (long) (((uint64_t) rb << 32) | ra);
}

// c + a * b on 24-bit signed operands: one v_mad_i32_i24. The empty asm makes the sum opaque, so the compiler keeps
// one multiply-add per product instead of reassociating the group sums into multiplies and three-way adds (the
// multiply-add itself is compiler-generated, so the MFMA result hazards stay the compiler's).
__device__ __forceinline__ int mad_i24(int a, int b, int c) {
    int r = __mul24(a, b) + c;
    asm volatile("" : "+v"(r));
    return r;
}

__device__ __forceinline__ void q6_lane_words(const uint8_t* tile, int lane, uint32_t (&w)[24]) {
    for (int k = 0; k < 6; ++k) {
        const u32x4 p = *(const u32x4*) (tile + 1024 * k + 16 * lane);
        for (int i = 0; i < 4; ++i) w[4 * k + i] = p[i];
    }
}

// the tiles dequantized back with the matmul's own unpack: (d * scale) * (q6 - 32) in fp32 (dequantize_row_q6_K)
__global__ __launch_bounds__(64) void k_q6k_dequant(const uint8_t* __restrict__ tiles, int N, int K,
                                                    float* __restrict__ out) {
    const int stripe = blockIdx.x, b = blockIdx.y, nb = K / 256, lane = threadIdx.x;
    const int n = lane & 31, h = lane >> 5, row = stripe * Q6T_ROWS + n;
    const uint8_t* tile = tiles + ((size_t) stripe * nb + b) * Q6T_BYTES;
    uint32_t w[24];
    q6_lane_words(tile, lane, w);
    const float d = (float) *(const _Float16*) (tile + Q6T_D_OFF + 2 * n);
    if (row >= N) return;
    for (int G = 0; G < 16; ++G) {
        const uint64_t v = (uint64_t) q6_unpack(w, G);
        const float ds = d * (float) (int8_t) tile[Q6T_SCALE_OFF + 16 * n + G];
        for (int j = 0; j < 8; ++j)
            out[(size_t) row * K + 256 * b + 16 * G + 8 * h + j] = ds * (float) (int8_t) (v >> (8 * j));
    }
}

// ---- Q8_K activation records ----------------------------------------------------------------------------------------
// grid (rows M), 256 threads: row m (source rows[m] of X when given) RMS-normed by nw when given (scale 1/sqrt(mean
// x^2 + eps), summed as the activation quantizer does: thread t over elements t, t + 256, ..), then wavefront w
// quantizes blocks w, w + 4, .. with lane l holding elements 4 l .. 4 l + 3: ggml quantize_row_q8_K_ref (max = the
// value of largest |x|, the first on ties; iscale = -127 / max; q = min(127, round-half-even(iscale * x)); d =
// 1 / iscale; an all-zero block: d = 0, q = 0).
__global__ __launch_bounds__(256) void k_quant_q8k(const float* __restrict__ X, const int32_t* __restrict__ rows,
                                                   int K, int ldx, const float* __restrict__ nw, float eps,
                                                   uint8_t* __restrict__ xk) {
    __shared__ float red_s[4];
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const float* x = X + (size_t) (rows ? rows[m] : m) * ldx;
    float scale = 1.0f;
    if (nw) {
        float s = 0.0f;
        for (int i = t; i < K; i += 256) s += x[i] * x[i];
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) red_s[wv] = s;
        __syncthreads();
        s = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
        scale = 1.0f / sqrtf(s / (float) K + eps);
    }
    for (int b = wv; b < K / 256; b += 4) {
        const int e0 = 256 * b + 4 * lane;
        float v[4];
        float a = 0.0f, va = 0.0f;
        int ia = 1 << 30;
        for (int i = 0; i < 4; ++i) {
            v[i] = nw ? (x[e0 + i] * scale) * nw[e0 + i] : x[e0 + i];
            if (fabsf(v[i]) > a) {
                a = fabsf(v[i]);
                ia = 4 * lane + i;
                va = v[i];
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float oa = __shfl_xor(a, o), ov = __shfl_xor(va, o);
            const int oi = __shfl_xor(ia, o);
            if (oa > a || (oa == a && oi < ia)) {
                a = oa;
                ia = oi;
                va = ov;
            }
        }
        uint32_t packed = 0;
        float d = 0.0f;
        if (a != 0.0f) {
            const float iscale = -127.f / va;
            for (int i = 0; i < 4; ++i)
                packed |= ((uint32_t) (int) fminf(127.f, __builtin_rintf(iscale * v[i])) & 0xFFu) << (8 * i);
            d = 1 / iscale;
        }
        // element 4 l + i: group l / 4, half (l / 2) & 1, byte 4 (l & 1) + i of row m's 8 in that half
        uint8_t* rec = xk + xk_rec_off(K, m, b);
        *(uint32_t*) (rec + (lane >> 2) * 512 + 8 * ((m & 31) + 32 * ((lane >> 1) & 1)) + 4 * (lane & 1)) = packed;
        if (lane == 0) *(float*) (rec + XK_D_OFF + 4 * (m & 31)) = d;
    }
}

// ---- the matmul -------------------------------------------------------------------------------------------------
// One workgroup (4 wavefronts) owns 4 consecutive 32-row stripes (wavefront w: stripe 4 set + w), MT row tiles of 32
// and all of K; the blocks are walked in order. Block b + 1's weights go into a second register slot and block b + 2's
// activation records into registers while block b is summed; block b + 1's records are stored into an LDS double
// buffer at the top of the iteration. Per (block, group, row tile): one MFMA 32x32x16 i8 (the exact integer dot),
// then isum += scale * dot in int32; per block acc += isum * (d6 * d8). The logits go straight to y (no k-split).
template <int MT>
__global__ __launch_bounds__(256, MT == 1 ? 4 : 2) void k_q6k_gemm(const uint8_t* __restrict__ tiles, const uint8_t* __restrict__ xk,
                                                  int M, int N, int K, int mt_first, float* __restrict__ y, int ldy) {
    constexpr int QPT = MT * 8192 / 16 / 256;  // 16-byte pieces of one block's record q a thread stages
    __shared__ __attribute__((aligned(16))) uint8_t s_rec[2][MT][XK_REC];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, h = lane >> 5;
    const int nb = K / 256, nstripes = (N + Q6T_ROWS - 1) / Q6T_ROWS;
    const int stripe = blockIdx.x * 4 + wave;
    const int mt0 = mt_first + blockIdx.y * MT;
    // one resource for the whole matrix (a stripe past it reads zeros: the range check covers the scalar offset)
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(tiles, (uint32_t) ((size_t) nstripes * nb * Q6T_BYTES));
    const int sofs = stripe * nb * Q6T_BYTES;
    // this workgroup's records: MT row tiles x nb blocks, row tile mt's block b at (mt * nb + b) * XK_REC
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(xk + (size_t) mt0 * nb * XK_REC, (uint32_t) ((size_t) MT * nb * XK_REC));

    u32x4 wq[2][6];
    u32x4 sc4[2];
    uint32_t dw[2];
    u32x4 rq[QPT];
    uint32_t rd;
    auto load_w = [&](int slot, int b) {
        const int so = sofs + min(b, nb - 1) * Q6T_BYTES;
        for (int k = 0; k < 6; ++k) wq[slot][k] = bload16(wr, 1024 * k + 16 * lane, so);
        sc4[slot] = bload16(wr, Q6T_SCALE_OFF + 16 * n, so);
        dw[slot] = __builtin_bit_cast(uint32_t, bload4f(wr, Q6T_D_OFF + 4 * (n >> 1), so));
    };
    // block b's records into registers: 16-byte piece i of the q (row tile i / 512), and dword t of the d (row tile
    // t / 32) for threads t < 32 MT; every load issued (index clamped)
    auto load_r = [&](int b) {
        const int bb = min(b, nb - 1);
        for (int k = 0; k < QPT; ++k) {
            const int i = threadIdx.x + 256 * k;
            rq[k] = bload16(xr, 16 * (i & 511), ((i >> 9) * nb + bb) * XK_REC);
        }
        const int t = min((int) threadIdx.x, 32 * MT - 1);
        rd = __builtin_bit_cast(uint32_t, bload4f(xr, XK_D_OFF + 4 * (t & 31), ((t >> 5) * nb + bb) * XK_REC));
    };
    auto store_r = [&](int buf) {
        for (int k = 0; k < QPT; ++k) {
            const int i = threadIdx.x + 256 * k;
            *(u32x4*) &s_rec[buf][i >> 9][16 * (i & 511)] = rq[k];
        }
        const int t = threadIdx.x;
        if (t < 32 * MT) *(uint32_t*) &s_rec[buf][t >> 5][XK_D_OFF + 4 * (t & 31)] = rd;
    };

    float acc[MT][16];
    for (int mt = 0; mt < MT; ++mt)
        for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
    const int32x16 zero = {0};
    load_r(0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_r(0);
    __builtin_amdgcn_sched_barrier(0);
    load_r(1);
    // block b from buffer / register slot cur (a constant in each of the two calls below, so the slots stay registers)
    auto block = [&](int b, const int cur) {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // block b's records are in buffer cur; everyone is done reading the other buffer
        store_r(cur ^ 1);  // block b + 1's (unused past the last block)
        __builtin_amdgcn_sched_barrier(0);
        load_r(b + 2);
        __builtin_amdgcn_sched_barrier(0);
        load_w(cur ^ 1, b + 1);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t w[24];
        for (int k = 0; k < 6; ++k)
            for (int i = 0; i < 4; ++i) w[4 * k + i] = wq[cur][k][i];
        int32x16 isum[MT];
        for (int mt = 0; mt < MT; ++mt) isum[mt] = zero;
#pragma unroll
        for (int G = 0; G < 16; ++G) {
            const long bw = q6_unpack(w, G);
            const int s = (int) (int8_t) (sc4[cur][G >> 2] >> (8 * (G & 3)));
            for (int mt = 0; mt < MT; ++mt) {
                const long a = *(const long*) &s_rec[cur][mt][G * 512 + 8 * lane];
                const int32x16 dot = __builtin_amdgcn_mfma_i32_32x32x16_i8(a, bw, zero, 0, 0, 0);
                for (int r = 0; r < 16; ++r) isum[mt][r] = mad_i24(dot[r], s, isum[mt][r]);
            }
        }
        const float d6 = (float) __builtin_bit_cast(_Float16, (uint16_t) (dw[cur] >> (16 * (n & 1))));
        // lane (n, h) holds rows 8 q + 4 h + t (register 4 q + t) of each row tile, column n of the stripe
        for (int mt = 0; mt < MT; ++mt)
            for (int q = 0; q < 4; ++q) {
                const floatx4 d8 = *(const floatx4*) &s_rec[cur][mt][XK_D_OFF + 4 * (8 * q + 4 * h)];
                for (int t = 0; t < 4; ++t)
                    acc[mt][4 * q + t] = __builtin_fmaf((float) isum[mt][4 * q + t], d6 * d8[t], acc[mt][4 * q + t]);
            }
    };
    for (int b = 0; b < nb; b += 2) {
        block(b, 0);
        if (b + 1 < nb) block(b + 1, 1);
    }
    const int col = stripe * Q6T_ROWS + n;
    if (stripe >= nstripes || col >= N) return;
    for (int mt = 0; mt < MT; ++mt)
        for (int r = 0; r < 16; ++r) {
            const int row = (mt0 + mt) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row < M) y[(size_t) row * ldy + col] = acc[mt][r];
        }
}

// ---- host side ----------------------------------------------------------------------------------------------------
void q6k_repack(const uint8_t* src, int N, int K, uint8_t* dst, hipStream_t st) {
    hipLaunchKernelGGL(k_q6k_repack, dim3((N + Q6T_ROWS - 1) / Q6T_ROWS, K / 256), dim3(64), 0, st, src, N, K, dst);
}
void q6k_dequant(const uint8_t* tiles, int N, int K, float* out, hipStream_t st) {
    hipLaunchKernelGGL(k_q6k_dequant, dim3((N + Q6T_ROWS - 1) / Q6T_ROWS, K / 256), dim3(64), 0, st, tiles, N, K, out);
}
void quant_q8k(const float* x, const int32_t* rows, int M, int K, int ldx, const float* nw, float eps, uint8_t* xk,
               hipStream_t st) {
    if (M > 0) hipLaunchKernelGGL(k_quant_q8k, dim3(M), dim3(256), 0, st, x, rows, K, ldx, nw, eps, xk);
}
int q6k_gemm(const uint8_t* tiles, const uint8_t* xk, int M, int N, int K, float* y, int ldy, hipStream_t st) {
    if (M <= 0) return 0;
    if (K % 256 || N <= 0) return -1;
    const int mtiles = (M + 31) / 32, sets = ((N + Q6T_ROWS - 1) / Q6T_ROWS + 3) / 4;
    // row tiles in pairs (the records are padded to an even count), a last odd tile alone
    const int pairs = mtiles / 2;
    if (pairs > 0) hipLaunchKernelGGL(k_q6k_gemm<2>, dim3(sets, pairs), dim3(256), 0, st, tiles, xk, M, N, K, 0, y, ldy);
    if (mtiles & 1)
        hipLaunchKernelGGL(k_q6k_gemm<1>, dim3(sets, 1), dim3(256), 0, st, tiles, xk, M, N, K, mtiles - 1, y, ldy);
    return 0;
}
