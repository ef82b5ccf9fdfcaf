// Device functions shared by the row kernels (ops.hip) and the matmul epilogues (q4.hip): the per-head QK-norm + NEOX
// RoPE + K/V cache write of one row (qk_rope, kernels.metal:149-197), so that both give a row the same bits.
#pragma once
#include "sn_common.h"

// The rotation's cos / sin of theta_i = p * s^i for lane i (i successive fp32 multiplies from p, ggml_rope_cache_init's
// loop; s = base^(-2/128) computed on the host)
__device__ __forceinline__ void rope_cs(int p, int lane, float theta_scale, float& c, float& s) {
#pragma clang fp contract(off)
    float theta = (float) p;
    for (int i = 0; i < lane; ++i) theta *= theta_scale;
    c = cosf(theta);
    s = sinf(theta);
}
// head h (q heads, k heads, v heads in that order) of the row at x, cell off of page; (w0, w1) the lane's norm weights
__device__ __forceinline__ void qk_head(float* __restrict__ x, int lane, int h, int H, int KVH, bool raw_kv, float a0,
                                        float a1, float c, float s, float w0, float w1, float eps,
                                        uint16_t* __restrict__ kpool, uint16_t* __restrict__ vpool, int page,
                                        int page_cells, int off) {
#pragma clang fp contract(off)
    const bool isq = h < H, isv = h >= H + KVH;
    if (raw_kv && !isq) {  // k and v as the matmul made them (q is overwritten below)
        x[lane] = a0;
        x[lane + 64] = a1;
    }
    if (isv) {
        uint16_t* vc = vpool + (((size_t) page * KVH + (h - H - KVH)) * page_cells + off) * 128;
        vc[lane] = __builtin_bit_cast(uint16_t, (_Float16) a0);
        vc[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16) a1);
        return;
    }
    float ss = a0 * a0 + a1 * a1;
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float sc = 1.0f / sqrtf(ss / 128.f + eps);
    a0 = (a0 * sc) * w0;
    a1 = (a1 * sc) * w1;
    const float y0 = a0 * c - a1 * s, y1 = a0 * s + a1 * c;
    if (isq) {
        x[lane] = y0;
        x[lane + 64] = y1;
    } else {
        uint16_t* kc = kpool + ((size_t) page * KVH + (h - H)) * page_cells * 128;
        kc[kcell_at(page_cells, off, lane)] = __builtin_bit_cast(uint16_t, (_Float16) y0);
        kc[kcell_at(page_cells, off, lane + 64)] = __builtin_bit_cast(uint16_t, (_Float16) y1);
    }
}

