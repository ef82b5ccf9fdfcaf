// Q4_0 x Q8_0 matmul for gfx950: Y[m][n] (+)= sum_k X[m][k] W[n][k].
//
// Replaces the reference's Q4_0 mat-vec / few-row / block matmuls (kernels.metal:1324-1411 mv_q4_0_*, :1413-1490
// mvm_q4_0_*, :746-1007 qmm_ks/qmmh_ks_q4_0_*, dispatched by mm() in core_mm.inc.h:307-325), with ggml's CPU numerics
// (Q8_0-quantized activations, integer block sums scaled by dw*dx) instead of the reference's fp16 weights.
//
// How a block's sum is formed: the weights' (q4 - 8) and the activations' q8 are exact in fp16, and
// v_mfma_f32_16x16x32_f16 multiplies exactly and accumulates in fp32, where every partial sum of a block (|sum| <=
// 32512) is an exact integer: the MFMA gives ggml's integer block sum isum. One fma per output then adds
// isum * (dw * dx) (the product of two fp16 values is exact in fp32) to the fp32 accumulator. The order of the sums
// of an output is fixed by (N, K) alone, never by the number of rows, so a row's result is the same in any step
// (sn.h:1-3).
#include <algorithm>

#include "sn_kernels_internal.h"

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
        for (int j = 0; j < 4; ++j) q[4 * b + j] = ok ? s[2 + 4 * g + j] : 0;
        d[b] = ok ? (uint16_t) (s[0] | (s[1] << 8)) : 0;
    }
    for (int j = 0; j < 16; ++j) t[16 * l + j] = q[j];
    if (g == 0)
        for (int b = 0; b < 4; ++b) {
            t[Q4T_SCALE_OFF + 8 * n + 2 * b] = (uint8_t) d[b];
            t[Q4T_SCALE_OFF + 8 * n + 2 * b + 1] = (uint8_t) (d[b] >> 8);
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

__device__ __forceinline__ void q8_store(const float* v, int g, uint8_t* frag, _Float16* dsl);

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
    if (src < 0) {  // a zero row (padding of an expert's tile)
        const int b = blockIdx.y * 64 + (t >> 2), g = t & 3;
        if (b >= xa_nbp(K)) return;
        *(half8*) (xa + xa_frag_off(K, m >> 4, b) + 16 * ((m & 15) + 16 * g)) = (half8){};
        if (g == 0) *((_Float16*) (xa + xa_scale_off(M, K, m >> 4, b)) + (m & 15)) = (_Float16) 0.0f;
        return;
    }
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
    uint8_t* frag = xa + xa_frag_off(K, m >> 4, b) + 16 * ((m & 15) + 16 * g);
    _Float16* dsl = (_Float16*) (xa + xa_scale_off(M, K, m >> 4, b)) + (m & 15);
    if (b >= nb) {  // a padding block of the last 4-block group: zero
        *(half8*) frag = (half8){};
        if (g == 0) *dsl = (_Float16) 0.0f;
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
    q8_store(v, g, frag, dsl);
}

// Row m, block b of a Q8_0 operand from its 32 fp32 values (this lane's 8: elements 4g..4g+3, 16+4g..16+4g+3):
// ggml x86 quantize_row_q8_0, d = amax / 127 (stored fp16), q = round-half-even(x * 127 / amax). The 4 lanes of a
// block are adjacent (the shuffles stay within them).
__device__ __forceinline__ void q8_store(const float* v, int g, uint8_t* frag, _Float16* dsl) {
    float amax = 0.0f;
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float d = amax / 127.f;
    const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    half8 q;
    for (int j = 0; j < 8; ++j) q[j] = (_Float16) __builtin_rintf(v[j] * id);
    *(half8*) frag = q;
    if (g == 0) *dsl = (_Float16) d;
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

// Residual rows: x[m] += the k-slice sums of a matmul (part[ks][M][K], slices added in order; add 0: x[m] = the
// sums), written back; then, when xa is given, the RMSNorm (weight nw) and Q8_0 operand of the new row. One workgroup
// per row (the norm needs the whole row before any value is quantized), 4 lanes per 32-block: lane t covers blocks
// t / 4 + (blockDim / 4) i, i < IT. Every load (residual, slices, norm weight) is issued before the row's reduction.
template <int IT, int KM>
__global__ __launch_bounds__(1024) void k_resid_quant(float* __restrict__ X, const float* __restrict__ part, int ks,
                                                      int M, int K, const float* __restrict__ nw, float eps,
                                                      uint8_t* __restrict__ xa, int add, float* __restrict__ xn) {
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
        const float4 slo = slices_sum4<KM>(part + (size_t) m * K + e0, (size_t) M * K, ks);
        const float4 shi = slices_sum4<KM>(part + (size_t) m * K + e1, (size_t) M * K, ks);
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
        uint8_t* frag = xa + xa_frag_off(K, m >> 4, b) + 16 * ((m & 15) + 16 * g);
        _Float16* dsl = (_Float16*) (xa + xa_scale_off(M, K, m >> 4, b)) + (m & 15);
        if (b >= nb) {  // a padding block of the last 4-block group: zero
            *(half8*) frag = (half8){};
            if (g == 0) *dsl = (_Float16) 0.0f;
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
        q8_store(y, g, frag, dsl);
    }
}

// SwiGLU of a stripe-interleaved gate/up matmul's k-slice sums (part[ks][M][2F]: output column 16p + n is
// silu(column 32p + n) * column 32p + 16 + n), written as fp32 rows h (when given) and as the Q8_0 operand of the next
// matmul. Workgroup (row m, 64 blocks), 4 lanes per block as in k_quant_act.
template <int KM>
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ part, int ks, int M, int F,
                                                      float* __restrict__ h, uint8_t* __restrict__ xa) {
    const int m = blockIdx.x, t = threadIdx.x;
    const int nb = F / 32, nbp = xa_nbp(F);
    const int b = blockIdx.y * 64 + (t >> 2), g = t & 3;
    if (b >= nbp) return;
    uint8_t* frag = xa + xa_frag_off(F, m >> 4, b) + 16 * ((m & 15) + 16 * g);
    _Float16* dsl = (_Float16*) (xa + xa_scale_off(M, F, m >> 4, b)) + (m & 15);
    if (b >= nb) {
        *(half8*) frag = (half8){};
        if (g == 0) *dsl = (_Float16) 0.0f;
        return;
    }
    // elements 32b + 4g + j (pair 2b) and 32b + 16 + 4g + j (pair 2b + 1): gate at 64b + 4g (+32), up 16 further
    const size_t N = 2 * (size_t) F;
    auto sum4 = [&](int c) { return slices_sum4<KM>(part + (size_t) m * N + c, (size_t) M * N, ks); };
    const float4 g0 = sum4(64 * b + 4 * g), u0 = sum4(64 * b + 16 + 4 * g);
    const float4 g1 = sum4(64 * b + 32 + 4 * g), u1 = sum4(64 * b + 48 + 4 * g);
    float v[8] = {silu(g0.x) * u0.x, silu(g0.y) * u0.y, silu(g0.z) * u0.z, silu(g0.w) * u0.w,
                  silu(g1.x) * u1.x, silu(g1.y) * u1.y, silu(g1.z) * u1.z, silu(g1.w) * u1.w};
    if (h) {
        float* o = h + (size_t) m * F + 32 * b;
        *(float4*) (o + 4 * g) = (float4){v[0], v[1], v[2], v[3]};
        *(float4*) (o + 16 + 4 * g) = (float4){v[4], v[5], v[6], v[7]};
    }
    q8_store(v, g, frag, dsl);
}

// ---------------------------------------------------------------------------------------------------------------------
// the matmul
__device__ __forceinline__ half8 q4_unpack(uint32_t w) {
    // (q - 8) of the 8 nibbles of w as fp16: low nibbles are elements 4g..4g+3, high nibbles 16+4g..16+4g+3.
    // 0x6400 | q is fp16(1024 + q); subtracting 1032 is exact.
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
    const half2v off = {(_Float16) 1032.0f, (_Float16) 1032.0f};
    const half2v h0 = __builtin_bit_cast(half2v, p0) - off;
    const half2v h1 = __builtin_bit_cast(half2v, p1) - off;
    const half2v h2 = __builtin_bit_cast(half2v, p2) - off;
    const half2v h3 = __builtin_bit_cast(half2v, p3) - off;
    half8 r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// One workgroup (4 wavefronts) owns a set of 4 consecutive 16-row stripes (wavefront w: stripe 4 set + w) and a
// k-slice of consecutive 4-block groups; the four wavefronts walk the slice's groups together, so a group's activation
// operand (MT row tiles x 4 blocks: 1 KB fragments and fp16 scales) is loaded from global memory once per workgroup:
// each wavefront loads MT fragments of it (wavefront 0 also the scales) into a register ring D groups ahead and stages
// them into an LDS double buffer one group ahead (scales as fp32). The weight tiles go straight from global memory into
// a ring of D groups of registers, so each wavefront keeps D tiles of its stripe in flight. Loads are issued in group
// order (activations before weights), the order they are used in: vmcnt counts in issue order, so waiting for the
// oldest group leaves the newer ones in flight. Every load is unconditional: stripes past the matrix are clamped to its
// last stripe (their sums are never stored) and groups past the slice repeat its last group (cache hits), so no load
// sits behind a branch.
//
// The kernel writes each slice's raw fp32 sums, part[slice][M][N]; whoever consumes them adds the slices in slice
// order (k_q4_reduce here; the row kernels of the step), so the order of every sum is fixed by (N, K) alone.
template <int MT, int D>
__global__ __launch_bounds__(256) void k_q4_gemm(GemmArgs a) {
    static_assert(D >= 2, "ring of at least two groups");
    constexpr int U = D % 2 ? 2 * D : D;  // unroll: a multiple of the ring and of the LDS double buffer
    __shared__ __attribute__((aligned(16))) uint8_t s_act[2][MT * 4][1024];
    __shared__ __attribute__((aligned(16))) float s_sc[2][MT * 64];  // tile mt: [block][row] as fp32
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n_in = lane & 15, g = lane >> 4;
    const int set = blockIdx.x, slice = blockIdx.y;
    int mt0 = blockIdx.z * MT;
    const uint8_t* wbase = a.w;
    if (a.items) {  // grouped: this workgroup's (expert, row tile)
        if ((int) blockIdx.z >= *a.count) return;
        wbase = a.w + (size_t) a.items[2 * blockIdx.z] * a.wstride;
        mt0 = a.items[2 * blockIdx.z + 1];
    }
    const int stripe = set * 4 + wave;
    const int c0 = slice * a.gps, ng = min(a.gps, a.ngroups - c0);  // groups c0 .. c0 + ng - 1 (ng >= 1)

    const uint8_t* wp = wbase + (size_t) min(stripe, a.nstripes - 1) * a.ngroups * Q4T_BYTES;
    // activation fragment f = wave * MT + j of a group: row tile mt0 + f / 4, block f % 4
    const uint8_t* af[MT];
    for (int j = 0; j < MT; ++j) {
        const int f = wave * MT + j;
        af[j] = a.xa + xa_frag_off(a.K, mt0 + f / 4, f % 4) + 16 * lane;
    }
    // scales: lane l < 32 MT loads dword l % 32 of row tile mt0 + l / 32 (its 4 blocks' 128 B are contiguous)
    const int sl = lane < 32 * MT ? lane : 0;
    const uint8_t* asp = a.xa + xa_scale_off(a.M, a.K, mt0 + sl / 32, 0) + 4 * (sl % 32);

    u32x4 wq[D];
    half4v ws[D];
    u32x4 ra[D][MT];
    uint32_t rs[D];
    floatx4 acc[MT];
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    auto load = [&](int slot, int i) {
        const int c = c0 + min(i, ng - 1);
        for (int j = 0; j < MT; ++j) ra[slot][j] = *(const u32x4*) (af[j] + (size_t) c * 4 * XA_FRAG_BYTES);
        rs[slot] = *(const uint32_t*) (asp + (size_t) c * 128);
        const size_t off = (size_t) c * Q4T_BYTES;
        wq[slot] = *(const u32x4*) (wp + off + 16 * lane);
        ws[slot] = *(const half4v*) (wp + off + Q4T_SCALE_OFF + 8 * n_in);
    };
    auto stage = [&](int buf, int slot) {
        for (int j = 0; j < MT; ++j) *(u32x4*) (&s_act[buf][wave * MT + j][16 * lane]) = ra[slot][j];
        if (wave == 0 && lane < 32 * MT) {
            // dword l % 32 of tile l / 32 holds fp16 [block][row] entries 2 (l % 32) and 2 (l % 32) + 1
            const half2v h = __builtin_bit_cast(half2v, rs[slot]);
            *(float2*) &s_sc[buf][(lane / 32) * 64 + 2 * (lane % 32)] = (float2){(float) h[0], (float) h[1]};
        }
    };
    auto compute = [&](int slot, int buf) {
        for (int b = 0; b < 4; ++b) {
            const half8 bw = q4_unpack(wq[slot][b]);
            const float dw = (float) ws[slot][b];
            for (int mt = 0; mt < MT; ++mt) {
                const half8 A = *(const half8*) (&s_act[buf][mt * 4 + b][16 * lane]);
                const floatx4 dx = *(const floatx4*) &s_sc[buf][mt * 64 + b * 16 + 4 * g];
                const floatx4 isum = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bw, zero, 0, 0, 0);
                for (int v = 0; v < 4; ++v) acc[mt][v] = __builtin_fmaf(isum[v], dw * dx[v], acc[mt][v]);
            }
        }
    };

    for (int j = 0; j < D; ++j) load(j, j);
    stage(0, 0);
    for (int i0 = 0; i0 < ng; i0 += U) {
        for (int j = 0; j < U; ++j) {
            const int i = i0 + j;
            if (i >= ng) break;
            __syncthreads();  // group i is staged; everyone is done reading the buffer group i + 1 goes to
            stage((j + 1) % 2, (j + 1) % D);
            compute(j % D, j % 2);
            load(j % D, i + D);
        }
    }

    // lane (n, g) holds rows 4g + v of each row tile, column n of the stripe
    const int col = stripe * 16 + n_in;
    if (stripe >= a.nstripes || col >= a.N) return;
    for (int mt = 0; mt < MT; ++mt)
        for (int v = 0; v < 4; ++v) {
            const int row = (mt0 + mt) * 16 + 4 * g + v;
            if (row < a.M) a.part[((size_t) slice * a.M + row) * a.N + col] = acc[mt][v];
        }
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

// The launch shape depends on (N, K) only, never on the rows (row invariance): 4 stripes per workgroup, and k-slices
// across workgroups while there are fewer than 512 workgroups, at most KS_MAX slices. 512 is two workgroups per CU:
// a launch of 256-511 workgroups leaves CUs holding one next to CUs holding two (gate/up at 304 sets: 19.6 us at
// one slice, 15.5 us at two, M = 32 on MI355X), while more slices mean more partial sums for the consumer to add.
GemmPlan q4_plan(int N, int K) {
    GemmPlan p;
    p.nstripes = (N + 15) / 16;
    p.ngroups = (K / 32 + 3) / 4;
    p.sets = (p.nstripes + 3) / 4;
    int ks = 1;
    while (p.sets * ks < 512 && ks < p.ngroups && ks < KS_MAX) ++ks;
    p.gps = (p.ngroups + ks - 1) / ks;
    p.ks = (p.ngroups + p.gps - 1) / p.gps;
    return p;
}

size_t q4_workspace_bytes(int M, int N, int K) { return (size_t) q4_plan(N, K).ks * M * N * sizeof(float); }

int q4_gemm_raw(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes,
                hipStream_t st) {
    if (M <= 0) return 0;
    const GemmPlan p = q4_plan(N, K);
    if (part == nullptr || part_bytes < (size_t) p.ks * M * N * sizeof(float)) return -1;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.part = part; a.y = nullptr;
    a.M = M; a.N = N; a.K = K; a.ldy = 0; a.epi = EPI_STORE;
    a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps;
    a.mtiles = (M + 15) / 16;
    if (a.mtiles == 1) hipLaunchKernelGGL((k_q4_gemm<1, 4>), dim3(p.sets, p.ks, 1), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_q4_gemm<2, 4>), dim3(p.sets, p.ks, (a.mtiles + 1) / 2), dim3(256), 0, st, a);
    return p.ks;
}

int q4_gemm_grouped(const uint8_t* w, size_t wstride, const int32_t* items, const int32_t* count, int max_items,
                    const uint8_t* xa, int M, int N, int K, float* part, size_t part_bytes, hipStream_t st) {
    if (M <= 0 || max_items <= 0) return 0;
    if (part == nullptr || part_bytes < (size_t) M * N * sizeof(float)) return -1;
    GemmArgs a{};
    a.w = w; a.xa = xa; a.part = part;
    a.items = items; a.count = count; a.wstride = wstride;
    a.M = M; a.N = N; a.K = K; a.epi = EPI_STORE;
    a.nstripes = (N + 15) / 16; a.ngroups = (K / 32 + 3) / 4; a.ks = 1; a.gps = a.ngroups;
    a.mtiles = (M + 15) / 16;
    hipLaunchKernelGGL((k_q4_gemm<1, 4>), dim3((a.nstripes + 3) / 4, 1, max_items), dim3(256), 0, st, a);
    return 1;
}

int q4_gemm(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* y, int ldy, int epi, float* ws,
            size_t ws_bytes, hipStream_t st) {
    if (M <= 0) return 0;
    const int ks = q4_gemm_raw(w, xa, M, N, K, ws, ws_bytes, st);
    if (ks < 0) return -1;
    GemmArgs a{};
    a.part = ws; a.y = y;
    a.M = M; a.N = N; a.K = K; a.ldy = ldy; a.epi = epi; a.ks = ks;
    const int tot = M * (epi == EPI_SWIGLU ? N / 2 : N);
    hipLaunchKernelGGL(k_q4_reduce, dim3((tot + 255) / 256), dim3(256), 0, st, a);
    return 0;
}

void q4_repack(const uint8_t* src, int N, int K, uint8_t* dst, int sstride, int soff, hipStream_t st) {
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    hipLaunchKernelGGL(k_q4_repack, dim3(tiles), dim3(64), 0, st, src, N, K, dst, sstride, soff);
}

template <int IT>
static void launch_resid(int km, int nt, float* x, const float* part, int ks, int M, int K, const float* nw, float eps,
                         uint8_t* xa, int ad, float* xn, hipStream_t st) {
#define RQ(KM_) hipLaunchKernelGGL((k_resid_quant<IT, KM_>), dim3(M), dim3(nt), 0, st, x, part, ks, M, K, nw, eps, xa, ad, xn)
    if (km == 1) RQ(1);
    else if (km == 2) RQ(2);
    else if (km == 4) RQ(4);
    else RQ(8);
#undef RQ
}

int resid_quant(float* x, const float* part, int ks, int M, int K, const float* nw, float eps, uint8_t* xa,
                hipStream_t st, bool add, float* xn) {
    if (M <= 0) return 0;
    // 4 lanes per block of the padded row, in whole wavefronts, at most 1024 lanes (then IT passes)
    const int lanes = 4 * xa_nbp(K), nt = std::min(1024, (lanes + 63) / 64 * 64), it = (lanes + nt - 1) / nt;
    const int km = ks_bound(ks);
    if (K % 32 || it > 4 || (xn && !xa) || km == 0) return -1;
    const int ad = add ? 1 : 0;
    if (it == 1) launch_resid<1>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st);
    else if (it == 2) launch_resid<2>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st);
    else launch_resid<4>(km, nt, x, part, ks, M, K, nw, eps, xa, ad, xn, st);
    return 0;
}

void swiglu_quant(const float* part, int ks, int M, int F, float* h, uint8_t* xa, hipStream_t st) {
    if (M <= 0) return;
    const dim3 grid(M, (xa_nbp(F) + 63) / 64);
    const int km = ks_bound(ks);
    if (km == 0) return;
    if (km == 1) hipLaunchKernelGGL((k_swiglu_quant<1>), grid, dim3(256), 0, st, part, ks, M, F, h, xa);
    else if (km == 2) hipLaunchKernelGGL((k_swiglu_quant<2>), grid, dim3(256), 0, st, part, ks, M, F, h, xa);
    else if (km == 4) hipLaunchKernelGGL((k_swiglu_quant<4>), grid, dim3(256), 0, st, part, ks, M, F, h, xa);
    else hipLaunchKernelGGL((k_swiglu_quant<8>), grid, dim3(256), 0, st, part, ks, M, F, h, xa);
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
        const half8 q = q4_unpack(wq[b]);
        for (int j = 0; j < 8; ++j) {
            const int e = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
            out[(size_t) row * K + 32 * blk + e] = (float) q[j] * dw[b];
        }
    }
}

extern "C" int snk_q4_dequant(const void* d_stripes, int N, int K, float* d_w, void* stream) {
    if (N <= 0 || K <= 0 || K % 32) return -1;
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    hipLaunchKernelGGL(k_q4_dequant, dim3(tiles), dim3(64), 0, (hipStream_t) stream, (const uint8_t*) d_stripes, N, K,
                       d_w);
    return hipGetLastError() == hipSuccess ? 0 : -1;
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
