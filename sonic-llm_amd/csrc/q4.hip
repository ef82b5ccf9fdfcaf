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
__device__ __forceinline__ float block_reduce_sum256(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Four lanes per 32-block: lane part g holds the block's elements {4g..4g+3, 16+4g..16+4g+3}, which is exactly its
// 8-value fragment of the MFMA operand, so each lane writes one 16-byte hi and one 16-byte lo fragment. The block's
// amax is a max over the 4 lanes. Workgroup (row m, block group y): 64 blocks; with a norm weight every workgroup of
// the row first sums the row's squares (the row is read from L2 once per workgroup).
__global__ __launch_bounds__(256) void k_quant_act(const float* __restrict__ X, const int32_t* __restrict__ rows,
                                                   int M, int K, int ldx, const float* __restrict__ nw, float eps,
                                                   uint8_t* __restrict__ xa, float* __restrict__ xn, int ldn) {
    __shared__ float red[4];
    const int m = blockIdx.x, nb = K / 32, t = threadIdx.x;
    const float* x = X + (size_t) (rows ? rows[m] : m) * ldx;
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
    // ggml x86 quantize_row_q8_0: d = amax / 127 (stored fp16), q = round-half-even(x * 127 / amax)
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

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// One workgroup (4 wavefronts) owns NT consecutive 16-row stripes (16 NT output columns) of a k-slice; the 4
// wavefronts split the slice's 4-block groups between them (wavefront w takes groups w, w + 4, ...) and their fp32
// sums are added in LDS in wavefront order. A wavefront streams its groups with a ring of D groups of weight tiles;
// the activation fragments and scales of a group are loaded one group ahead, before the weight refill of the group
// being computed, so that waiting for them (vmcnt counts in issue order) leaves the newer weight loads in flight.
// Every load is unconditional: stripes past the matrix are clamped to its last stripe (their sums are never stored),
// groups past a wavefront's last repeat it, and the xa operand is padded (sn_common.h), so no load waits on a branch.
template <int MT, int NT, int D>
__global__ __launch_bounds__(256) void k_q4_gemm(GemmArgs a) {
    constexpr int U = D % 2 ? 2 * D : D;  // unroll: a multiple of both ring sizes
    __shared__ floatx4 red[4][NT][MT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n_in = lane & 15, g = lane >> 4;
    const int s0 = blockIdx.x * NT, slice = blockIdx.y, mt0 = blockIdx.z * MT;
    const int c0 = slice * a.gps, c1 = min(c0 + a.gps, a.ngroups);
    const int ng = c1 - c0 > wave ? (c1 - c0 - wave + 3) / 4 : 0;  // this wavefront's groups: c0 + wave + 4 i
    const uint8_t* wp[NT];
    for (int t = 0; t < NT; ++t) wp[t] = a.w + (size_t) min(s0 + t, a.nstripes - 1) * a.ngroups * Q4T_BYTES;
    const uint8_t* xf = a.xa + xa_frag_off(a.K, mt0, 0) + 16 * lane;
    const uint8_t* xs = a.xa + xa_scale_off(a.M, a.K, mt0, 0) + 8 * g;
    const int nbp = a.ngroups * 4;

    floatx4 acc[NT][MT];
    for (int t = 0; t < NT; ++t)
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    u32x4 wq[D][NT];
    half4v ws[D][NT];
    half8 aq[2][4][MT];
    half4v ad[2][4][MT];
    auto grp = [&](int i) { return c0 + wave + 4 * min(i, max(ng - 1, 0)); };
    auto load_w = [&](int slot, int i) {
        const size_t off = (size_t) grp(i) * Q4T_BYTES;
        for (int t = 0; t < NT; ++t) {
            wq[slot][t] = *(const u32x4*) (wp[t] + off + 16 * lane);
            ws[slot][t] = *(const half4v*) (wp[t] + off + Q4T_SCALE_OFF + 8 * n_in);
        }
    };
    auto load_a = [&](int buf, int i) {
        const int c = grp(i);
        for (int b = 0; b < 4; ++b)
            for (int mt = 0; mt < MT; ++mt) {
                const size_t blk = (size_t) mt * nbp + 4 * c + b;
                aq[buf][b][mt] = *(const half8*) (xf + blk * XA_FRAG_BYTES);
                ad[buf][b][mt] = *(const half4v*) (xs + blk * 32);
            }
    };
    auto compute = [&](int slot, int buf) {
        for (int t = 0; t < NT; ++t) {
            const u32x4 w4 = wq[slot][t];
            const half4v sc = ws[slot][t];
            for (int b = 0; b < 4; ++b) {
                const half8 bw = q4_unpack(w4[b]);
                const float dw = (float) sc[b];
                for (int mt = 0; mt < MT; ++mt) {
                    const floatx4 isum = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[buf][b][mt], bw, zero, 0, 0, 0);
                    const half4v dx = ad[buf][b][mt];
                    for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(isum[v], dw * (float) dx[v], acc[t][mt][v]);
                }
            }
        }
    };
    if (ng > 0) {
        load_w(0, 0);
        load_a(0, 0);
        for (int j = 1; j < D; ++j) load_w(j, j);
        for (int i0 = 0; i0 < ng; i0 += U) {
            for (int j = 0; j < U; ++j) {
                const int i = i0 + j;
                if (i >= ng) break;
                load_a((j + 1) % 2, i + 1);
                compute(j % D, j % 2);
                load_w(j % D, i + D);
            }
        }
    }

    // the 4 wavefronts' sums, added in wavefront order; wavefront w then finishes stripe(s) of its own
    for (int t = 0; t < NT; ++t)
        for (int mt = 0; mt < MT; ++mt) red[wave][t][mt][lane] = acc[t][mt];
    __syncthreads();
    for (int t = wave; t < NT; t += 4)
        for (int mt = 0; mt < MT; ++mt) {
            floatx4 v4 = red[0][t][mt][lane];
            for (int w = 1; w < 4; ++w) {
                const floatx4 o = red[w][t][mt][lane];
                for (int v = 0; v < 4; ++v) v4[v] += o[v];
            }
            red[0][t][mt][lane] = v4;
        }
    __syncthreads();

    // lane (n, g) holds rows 4g+v of each row tile, column n of each stripe
    if (a.ks > 1 || a.epi != EPI_SWIGLU) {
        for (int t = wave; t < NT; t += 4) {
            const int s = s0 + t;
            const int col = s * 16 + n_in;
            if (s >= a.nstripes || col >= a.N) continue;
            for (int mt = 0; mt < MT; ++mt)
                for (int v = 0; v < 4; ++v) {
                    const int row = (mt0 + mt) * 16 + 4 * g + v;
                    if (row >= a.M) continue;
                    const float val = red[0][t][mt][lane][v];
                    if (a.ks > 1) a.part[((size_t) slice * a.M + row) * a.N + col] = val;
                    else if (a.epi == EPI_STORE) a.y[(size_t) row * a.ldy + col] = val;
                    else a.y[(size_t) row * a.ldy + col] += val;
                }
        }
    } else {
        // stripes 2p (gate) and 2p + 1 (up) of a pair are both in this workgroup (NT even, s0 even)
        for (int t = 2 * wave; t + 1 < NT; t += 8) {
            const int s = s0 + t;
            if (s + 1 >= a.nstripes) continue;
            const int col = (s / 2) * 16 + n_in;
            for (int mt = 0; mt < MT; ++mt)
                for (int v = 0; v < 4; ++v) {
                    const int row = (mt0 + mt) * 16 + 4 * g + v;
                    if (row >= a.M || col >= a.N / 2) continue;
                    a.y[(size_t) row * a.ldy + col] = silu(red[0][t][mt][lane][v]) * red[0][t + 1][mt][lane][v];
                }
        }
    }
}

// k-slice partials added in slice order, then the epilogue
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
        // output column col = 16 p + n is gate column 32 p + n and up column 32 p + 16 + n
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

// The launch shape of a matrix depends on (N, K) only, never on the rows (row invariance): NT = 4 stripes per
// workgroup, and k-slices across workgroups only while there are fewer than 1024 wavefronts and each slice keeps at
// least 16 groups (2048 values), so the slices' partial sums stay a small fraction of the weight bytes.
GemmPlan q4_plan(int N, int K) {
    GemmPlan p;
    p.nstripes = (N + 15) / 16;
    p.ngroups = (K / 32 + 3) / 4;
    p.nt = 4;
    const int wgs = (p.nstripes + p.nt - 1) / p.nt;
    int ks = 1;
    while (wgs * ks * 4 < 1024 && p.ngroups / (ks + 1) >= 16) ++ks;
    p.gps = (p.ngroups + ks - 1) / ks;
    p.ks = (p.ngroups + p.gps - 1) / p.gps;
    return p;
}

size_t q4_workspace_bytes(int M, int N, int K) {
    const GemmPlan p = q4_plan(N, K);
    return p.ks > 1 ? (size_t) p.ks * M * N * sizeof(float) : 0;
}

template <int MT>
static void launch_mt(const GemmArgs& a, int mblocks, hipStream_t st) {
    dim3 grid((a.nstripes + 3) / 4, a.ks, mblocks);
    hipLaunchKernelGGL((k_q4_gemm<MT, 4, 2>), grid, dim3(256), 0, st, a);
}

int q4_gemm(const uint8_t* w, const uint8_t* xa, int M, int N, int K, float* y, int ldy, int epi, float* part,
            size_t part_bytes, hipStream_t st) {
    if (M <= 0) return 0;
    const GemmPlan p = q4_plan(N, K);
    GemmArgs a;
    a.w = w; a.xa = xa; a.y = y; a.part = part;
    a.M = M; a.N = N; a.K = K; a.ldy = ldy; a.epi = epi;
    a.nstripes = p.nstripes; a.ngroups = p.ngroups; a.ks = p.ks; a.gps = p.gps;
    a.mtiles = (M + 15) / 16;
    if (p.ks > 1 && (part == nullptr || part_bytes < (size_t) p.ks * M * N * sizeof(float))) return -1;
    if (a.mtiles == 1) launch_mt<1>(a, 1, st);
    else launch_mt<2>(a, (a.mtiles + 1) / 2, st);
    if (p.ks > 1) {
        const int outN = epi == EPI_SWIGLU ? N / 2 : N;
        const int tot = M * outN;
        hipLaunchKernelGGL(k_q4_reduce, dim3((tot + 255) / 256), dim3(256), 0, st, a);
    }
    return 0;
}

void q4_repack(const uint8_t* src, int N, int K, uint8_t* dst, int sstride, int soff, hipStream_t st) {
    const int tiles = ((N + 15) / 16) * ((K / 32 + 3) / 4);
    hipLaunchKernelGGL(k_q4_repack, dim3(tiles), dim3(64), 0, st, src, N, K, dst, sstride, soff);
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
