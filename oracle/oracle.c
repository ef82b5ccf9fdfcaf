// CPU oracle (test infrastructure only; see oracle.h for what each function restates and where it is cited).
// Built with -ffp-contract=off so every float expression rounds exactly as written.
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

static int nthr(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void) n;
    return 1;
#endif
}

// ---- fp16: F16C round-to-nearest-even conversion (ggml's GGML_FP32_TO_FP16 on x86) ----
uint16_t or_f32_to_f16(float f) { return (uint16_t) _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
float or_f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

static float h2f(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_f16_to_f32(h);
}
static void f2h_store(uint8_t* p, float f) {
    const uint16_t h = or_f32_to_f16(f);
    memcpy(p, &h, 2);
}

// ---- Q4_0: ggml quantize_row_q4_0_ref. The element of largest |x| (the first on ties) maps to q = 0:
// d = max / -8, id = 1/d, q = min(15, (int8)(x*id + 8.5)) (truncation toward zero), d stored fp16.
void or_quantize_row_q4_0(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        const float* xb = x + i * QK;
        uint8_t* yb = y + i * 18;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK; j++) {
            const float v = xb[j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        f2h_store(yb, d);
        for (int j = 0; j < QK / 2; ++j) {
            const float x0 = xb[j] * id;
            const float x1 = xb[QK / 2 + j] * id;
            int8_t t0 = (int8_t) (x0 + 8.5f), t1 = (int8_t) (x1 + 8.5f);
            const uint8_t xi0 = (uint8_t) (t0 < 15 ? t0 : 15);
            const uint8_t xi1 = (uint8_t) (t1 < 15 ? t1 : 15);
            yb[2 + j] = (uint8_t) (xi0 | (xi1 << 4));
        }
    }
}

// ggml dequantize_row_q4_0: y[j] = (qs[j] & 15 - 8) * d, y[j + 16] = (qs[j] >> 4 - 8) * d
// (patch 0001:543-565 restates the same loop; kernels.metal:21-28 is the GPU form)
void or_dequantize_row_q4_0(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* b = x + i * 18;
        const float d = h2f(b);
        for (int j = 0; j < QK / 2; ++j) {
            const int x0 = (b[2 + j] & 0x0F) - 8;
            const int x1 = (b[2 + j] >> 4) - 8;
            y[i * QK + j] = x0 * d;
            y[i * QK + j + QK / 2] = x1 * d;
        }
    }
}

// ggml x86 quantize_row_q8_0 (the activations of every Q4_0 mul_mat on the CPU backend): per 32-block,
// amax = max |x|, d = amax / 127 (stored fp16), id = 127 / amax (0 when amax is 0), q = round-half-even(x * id).
void or_quantize_row_q8_0(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        const float* xb = x + i * QK;
        uint8_t* yb = y + i * 34;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        f2h_store(yb, d);
        for (int j = 0; j < QK; ++j) {
            const float v = xb[j] * id;
            yb[2 + j] = (uint8_t) (int8_t) (int) nearbyintf(v);
        }
    }
}

void or_dequantize_row_q8_0(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* b = x + i * 34;
        const float d = h2f(b);
        for (int j = 0; j < QK; ++j) y[i * QK + j] = (int8_t) b[2 + j] * d;
    }
}

// ggml quantize_row_q8_0_ref (the quantizer of Q8_0 weights in a model file): d = amax / 127 stored fp16, id = 1/d (0
// when d is 0), q = roundf(x * id) (halves away from zero). The activations of a mul_mat use or_quantize_row_q8_0.
void or_quantize_row_q8_0_ref(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        const float* xb = x + i * QK;
        uint8_t* yb = y + i * 34;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        f2h_store(yb, d);
        for (int j = 0; j < QK; ++j) yb[2 + j] = (uint8_t) (int8_t) (int) roundf(xb[j] * id);
    }
}

// ggml_vec_dot_q8_0_q8_0 (generic form): per block the integer sum of qw * qx, then sumf += sumi * (dw * dx)
// Test hook (or_set_sum_order): the Q4_0 / Q8_0 dots add their blocks' fp32 terms last block first. The same
// arithmetic in another summation order: how far two correct implementations drift apart over a model's layers.
static int g_sum_reverse = 0;
void or_set_sum_order(int reverse) { g_sum_reverse = reverse != 0; }

float or_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq) {
    const int64_t nb = k / QK;
    float sumf = 0.0f;
    for (int64_t jb = 0; jb < nb; ++jb) {
        const int64_t ib = g_sum_reverse ? nb - 1 - jb : jb;
        const uint8_t* bw = w + ib * 34;
        const uint8_t* bx = xq + ib * 34;
        int sumi = 0;
        for (int j = 0; j < QK; ++j) sumi += (int8_t) bw[2 + j] * (int8_t) bx[2 + j];
        sumf += (float) sumi * (h2f(bw) * h2f(bx));
    }
    return sumf;
}

// ggml CPU mul_mat of Q8_0 weights: the activation rows quantized to Q8_0 (x86 quantize_row_q8_0), then
// ---- Q6_K / Q8_K ----
// dequantize_row_q6_K: per 128-element half, l = 0..31 gives elements l, l+32, l+64, l+96 from ql[l], ql[l+32], qh[l]
void or_dequantize_row_q6_K(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* b = x + i * 210;
        const float d = h2f(b + 208);
        const uint8_t* ql = b;
        const uint8_t* qh = b + 128;
        const int8_t* sc = (const int8_t*) (b + 192);
        for (int n = 0; n < 256; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int) ((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int) ((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

// ggml's nearest_int: round half to even through the fp32 magic constant 1.5 * 2^23
static int nearest_int(float fval) {
    const float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof i);
    return (i & 0x007fffff) - 0x00400000;
}

void or_quantize_row_q8_K(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i) {
        uint8_t* b = y + i * 292;
        int8_t* qs = (int8_t*) (b + 4);
        int16_t bs[16];
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (!amax) {
            const float z = 0.0f;
            memcpy(b, &z, 4);
            memset(qs, 0, 256);
            memset(b + 260, 0, 32);
            x += 256;
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < 256; ++j) {
            const int v = nearest_int(iscale * x[j]);
            qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += qs[j * 16 + ii];
            bs[j] = (int16_t) sum;
        }
        memcpy(b + 260, bs, 32);
        const float d = 1 / iscale;
        memcpy(b, &d, 4);
        x += 256;
    }
}

float or_vec_dot_q6_K_q8_K(int64_t k, const uint8_t* w, const uint8_t* xq) {
    const int64_t nb = k / 256;
    int8_t aux8[256];
    int16_t aux16[8];
    int32_t aux32[8];
    float sums[8] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* bw = w + i * 210;
        const uint8_t* bx = xq + i * 292;
        const uint8_t* q4 = bw;
        const uint8_t* qh = bw + 128;
        const int8_t* sc = (const int8_t*) (bw + 192);
        const int8_t* q8 = (const int8_t*) (bx + 4);
        memset(aux32, 0, sizeof aux32);
        int8_t* a = aux8;
        for (int j = 0; j < 256; j += 128) {
            for (int l = 0; l < 32; ++l) {
                a[l + 0] = (int8_t) ((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                a[l + 32] = (int8_t) ((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                a[l + 64] = (int8_t) ((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                a[l + 96] = (int8_t) ((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            }
            a += 128;
            q4 += 64;
            qh += 32;
        }
        a = aux8;
        for (int j = 0; j < 16; ++j) {
            const int scale = sc[j];
            for (int l = 0; l < 8; ++l) aux16[l] = (int16_t) (q8[l] * a[l]);
            for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
            q8 += 8;
            a += 8;
            for (int l = 0; l < 8; ++l) aux16[l] = (int16_t) (q8[l] * a[l]);
            for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
            q8 += 8;
            a += 8;
        }
        float d8;
        memcpy(&d8, bx, 4);
        const float d = h2f(bw + 208) * d8;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    float sumf = 0.0f;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

void or_mul_mat_q6_K(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads) {
    const int64_t nb = K / 256;
    uint8_t* xq = (uint8_t*) malloc((size_t) M * nb * 292);
    for (int64_t m = 0; m < M; ++m) or_quantize_row_q8_K(X + m * K, xq + m * nb * 292, K);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) Y[m * N + n] = or_vec_dot_q6_K_q8_K(K, W + n * nb * 210, xq + m * nb * 292);
    free(xq);
}

// vec_dot_q8_0_q8_0 per (row, output)
void or_mul_mat_q8_0(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads) {
    const int64_t nb = K / QK;
    uint8_t* xq = (uint8_t*) malloc((size_t) M * nb * 34);
    for (int64_t m = 0; m < M; ++m) or_quantize_row_q8_0(X + m * K, xq + m * nb * 34, K);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) Y[m * N + n] = or_vec_dot_q8_0_q8_0(K, W + n * nb * 34, xq + m * nb * 34);
    free(xq);
}

// ggml_vec_dot_q4_0_q8_0 (generic form): per block the integer sum of (q4 - 8) * q8, then sumf += sumi * dw * dx
float or_vec_dot_q4_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq) {
    const int64_t nb = k / QK;
    float sumf = 0.0f;
    for (int64_t jb = 0; jb < nb; ++jb) {
        const int64_t ib = g_sum_reverse ? nb - 1 - jb : jb;
        const uint8_t* bw = w + ib * 18;
        const uint8_t* bx = xq + ib * 34;
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < QK / 2; ++j) {
            const int v0 = (bw[2 + j] & 0x0F) - 8;
            const int v1 = (bw[2 + j] >> 4) - 8;
            sumi0 += v0 * (int8_t) bx[2 + j];
            sumi1 += v1 * (int8_t) bx[2 + j + QK / 2];
        }
        const int sumi = sumi0 + sumi1;
        sumf += sumi * h2f(bw) * h2f(bx);
    }
    return sumf;
}

void or_mul_mat_q4_0(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nthreads) {
    const int64_t nb = K / QK;
    uint8_t* xq = (uint8_t*) malloc((size_t) (M * nb * 34));
    for (int64_t m = 0; m < M; ++m) or_quantize_row_q8_0(X + m * K, xq + m * nb * 34, K);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) Y[m * N + n] = or_vec_dot_q4_0_q8_0(K, W + n * nb * 18, xq + m * nb * 34);
    free(xq);
}

void or_mul_mat_q4_0_f64(const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, double* Y, int nthreads) {
    const int64_t nb = K / QK;
#pragma omp parallel num_threads(nthr(nthreads))
    {
        float* row = (float*) malloc((size_t) K * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            or_dequantize_row_q4_0(W + n * nb * 18, row, K);
            for (int64_t m = 0; m < M; ++m) {
                double s = 0.0;
                for (int64_t k = 0; k < K; ++k) s += (double) row[k] * (double) X[m * K + k];
                Y[m * N + n] = s;
            }
        }
        free(row);
    }
}

// ---- elementwise ----
// ggml rms_norm (squares summed in double) followed by the weight multiply: y = (x * scale) * w
void or_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double) (x[i] * x[i]);
    const float mean = (float) (sum / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] * scale) * (w ? w[i] : 1.0f);
}

float or_silu(float x) { return x / (1.0f + expf(-x)); }

int32_t or_argmax(const float* x, int64_t n, const int32_t* ban, int nban) {
    float best = -INFINITY;
    int32_t idx = -1;
    for (int64_t i = 0; i < n; i++) {
        int banned = 0;
        for (int b = 0; b < nban; ++b) banned |= ban[b] == i;
        if (!banned && (idx < 0 || x[i] > best)) {  // strictly greater: an equal score keeps the lower id
            best = x[i];
            idx = (int32_t) i;
        }
    }
    return idx;
}

void or_top2(const float* x, int64_t n, int32_t* i1, float* v1, int32_t* i2, float* v2, float* lse) {
    float m1 = -INFINITY, m2 = -INFINITY;
    int32_t a = 0x7fffffff, b = 0x7fffffff;
    for (int64_t i = 0; i < n; i++) {
        if (x[i] > m1) {
            m2 = m1;
            b = a;
            m1 = x[i];
            a = (int32_t) i;
        } else if (x[i] > m2) {
            m2 = x[i];
            b = (int32_t) i;
        }
    }
    double s = 0.0;
    if (m1 > -INFINITY)
        for (int64_t i = 0; i < n; i++) s += exp((double) x[i] - (double) m1);
    *i1 = a;
    *v1 = m1;
    *i2 = b;
    *v2 = m2;
    *lse = m1 > -INFINITY ? (float) ((double) m1 + log(s)) : -INFINITY;  // no finite score: -inf (kernels.metal:436)
}

// ggml_rope_cache_init with ext_factor 0, freq_scale 1, mscale 1: theta starts at p and is multiplied by theta_scale
// after each pair, in fp32
void or_rope_cache(int32_t pos, float theta_scale, int D, float* cs) {
    float theta = (float) pos;
    for (int i = 0; i < D / 2; ++i) {
        cs[2 * i] = cosf(theta);
        cs[2 * i + 1] = sinf(theta);
        theta *= theta_scale;
    }
}

void or_qk_norm_rope(float* x, const float* w, int D, float eps, const float* cs, int do_norm) {
    if (do_norm) or_rmsnorm(x, w, D, eps, x);
    for (int i = 0; i < D / 2; ++i) {
        const float c = cs[2 * i], s = cs[2 * i + 1];
        const float x0 = x[i], x1 = x[i + D / 2];
        x[i] = x0 * c - x1 * s;
        x[i + D / 2] = x0 * s + x1 * c;
    }
}

// ---- attention over a list of cells (cell c's K head vector at kp[c], V at vp[c]) ----
static void attn_cells(const float* q, int D, int n, const uint16_t* const* kp, const uint16_t* const* vp, float scale,
                       float* out, int f64) {
    if (n <= 0) {
        for (int d = 0; d < D; ++d) out[d] = 0.0f;
        return;
    }
    if (f64) {
        double* s = (double*) malloc((size_t) n * sizeof(double));
        double m = -INFINITY;
        for (int c = 0; c < n; ++c) {
            double t = 0.0;
            for (int d = 0; d < D; ++d) t += (double) q[d] * (double) or_f16_to_f32(kp[c][d]);
            s[c] = t * (double) scale;
            if (s[c] > m) m = s[c];
        }
        double l = 0.0;
        for (int c = 0; c < n; ++c) {
            s[c] = exp(s[c] - m);
            l += s[c];
        }
        for (int d = 0; d < D; ++d) {
            double o = 0.0;
            for (int c = 0; c < n; ++c) o += s[c] * (double) or_f16_to_f32(vp[c][d]);
            out[d] = (float) (o / l);
        }
        free(s);
        return;
    }
    float* s = (float*) malloc((size_t) n * sizeof(float));
    float m = -INFINITY;
    for (int c = 0; c < n; ++c) {
        float t = 0.0f;
        for (int d = 0; d < D; ++d) t += q[d] * or_f16_to_f32(kp[c][d]);
        s[c] = t * scale;
        if (s[c] > m) m = s[c];
    }
    double l = 0.0;
    for (int c = 0; c < n; ++c) {
        s[c] = expf(s[c] - m);
        l += (double) s[c];
    }
    const float il = (float) (1.0 / l);
    for (int c = 0; c < n; ++c) s[c] *= il;
    for (int d = 0; d < D; ++d) {
        float o = 0.0f;
        for (int c = 0; c < n; ++c) o += s[c] * or_f16_to_f32(vp[c][d]);
        out[d] = o;
    }
    free(s);
}

static const uint16_t* pool_cell(const uint16_t* pool, const int32_t* pt, int max_pages, int page_cells, int KVH, int D,
                                 int s, int h, int c) {
    const int p = pt[(size_t) s * max_pages + c / page_cells];
    return pool + (((size_t) p * KVH + h) * page_cells + c % page_cells) * D;
}

void or_paged_attn(const float* q, int nq, const int32_t* qseq, const int32_t* qpos, int H, int KVH, int D,
                   const uint16_t* kpool, const uint16_t* vpool, int page_cells, const int32_t* pt, int max_pages,
                   float scale, float* out, int f64, int nthreads) {
    const int G = H / KVH;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(dynamic, 1)
    for (int rh = 0; rh < nq * H; ++rh) {
        const int r = rh / H, h = rh % H, kh = h / G, n = qpos[r] + 1;
        const uint16_t** kp = (const uint16_t**) malloc((size_t) n * sizeof(void*));
        const uint16_t** vp = (const uint16_t**) malloc((size_t) n * sizeof(void*));
        for (int c = 0; c < n; ++c) {
            kp[c] = pool_cell(kpool, pt, max_pages, page_cells, KVH, D, qseq[r], kh, c);
            vp[c] = pool_cell(vpool, pt, max_pages, page_cells, KVH, D, qseq[r], kh, c);
        }
        attn_cells(q + ((size_t) r * H + h) * D, D, n, kp, vp, scale, out + ((size_t) r * H + h) * D, f64);
        free(kp);
        free(vp);
    }
}

void or_paged_attn_chunked(const float* q, int nq, const int32_t* qseq, const int32_t* qpos, int H, int KVH, int D,
                           const uint16_t* kpool, const uint16_t* vpool, int page_cells, const int32_t* pt,
                           int max_pages, float scale, int chunk, float* out) {
    const int G = H / KVH;
    float* acc = (float*) malloc((size_t) D * sizeof(float));
    float* pa = (float*) malloc((size_t) D * sizeof(float));
    for (int r = 0; r < nq; ++r)
        for (int h = 0; h < H; ++h) {
            const int kh = h / G, n = qpos[r] + 1;
            const float* qh = q + ((size_t) r * H + h) * D;
            float M = -INFINITY, L = 0.0f;
            for (int d = 0; d < D; ++d) acc[d] = 0.0f;
            for (int c0 = 0; c0 < n; c0 += chunk) {
                const int c1 = c0 + chunk < n ? c0 + chunk : n;
                // the chunk's partial: its own max, sum and unnormalised accumulator
                float m = -INFINITY, l = 0.0f;
                for (int d = 0; d < D; ++d) pa[d] = 0.0f;
                float* s = (float*) malloc((size_t) (c1 - c0) * sizeof(float));
                for (int c = c0; c < c1; ++c) {
                    const uint16_t* kc = pool_cell(kpool, pt, max_pages, page_cells, KVH, D, qseq[r], kh, c);
                    float t = 0.0f;
                    for (int d = 0; d < D; ++d) t += qh[d] * or_f16_to_f32(kc[d]);
                    s[c - c0] = t * scale;
                    if (s[c - c0] > m) m = s[c - c0];
                }
                for (int c = c0; c < c1; ++c) {
                    const uint16_t* vc = pool_cell(vpool, pt, max_pages, page_cells, KVH, D, qseq[r], kh, c);
                    const float p = expf(s[c - c0] - m);
                    l += p;
                    for (int d = 0; d < D; ++d) pa[d] += p * or_f16_to_f32(vc[d]);
                }
                free(s);
                // merged in chunk order (attn_merge)
                const float mn = M > m ? M : m;
                const float e0 = expf(M - mn), e1 = expf(m - mn);
                for (int d = 0; d < D; ++d) acc[d] = acc[d] * e0 + pa[d] * e1;
                L = L * e0 + l * e1;
                M = mn;
            }
            for (int d = 0; d < D; ++d) out[((size_t) r * H + h) * D + d] = n > 0 ? acc[d] / L : 0.0f;
        }
    free(acc);
    free(pa);
}

// ---- MoE routing (moe_topk, mode 0) ----
void or_moe_route(const float* logits, int n_expert, int k, int32_t* ids, float* w) {
    float m = -INFINITY;
    for (int i = 0; i < n_expert; ++i) m = fmaxf(m, logits[i]);
    float* p = (float*) malloc((size_t) n_expert * sizeof(float));
    float tot = 0.0f;
    for (int i = 0; i < n_expert; ++i) {
        p[i] = expf(logits[i] - m);
        tot += p[i];
    }
    float sel = 0.0f;
    for (int j = 0; j < k; ++j) {
        int bi = -1;
        for (int i = 0; i < n_expert; ++i)
            if (bi < 0 || p[i] > p[bi]) bi = i;
        ids[j] = bi;
        w[j] = p[bi] / tot;
        sel += w[j];
        p[bi] = -INFINITY;
    }
    sel = fmaxf(sel, 6.103515625e-5f);
    for (int j = 0; j < k; ++j) w[j] = w[j] / sel;
    free(p);
}

// Test hook (or_moe_trace): each routing's margin, the smallest router logit chosen minus the largest one not chosen
// (a near tie there is where two implementations may pick different experts), in call order: layer by layer, row by row.
static float* g_moe_margin = NULL;
static int g_moe_cap = 0, g_moe_n = 0;
void or_moe_trace(float* margins, int cap) {
    g_moe_margin = margins;
    g_moe_cap = margins ? cap : 0;
    g_moe_n = 0;
}
int or_moe_trace_count(void) { return g_moe_n; }
static void moe_note_margin(const float* lg, int n_expert, const int32_t* ids, int k) {
    if (!g_moe_margin || g_moe_n >= g_moe_cap) return;
    float lo = INFINITY, hi = -INFINITY;
    for (int j = 0; j < k; ++j) lo = fminf(lo, lg[ids[j]]);
    for (int i = 0; i < n_expert; ++i) {
        int chosen = 0;
        for (int j = 0; j < k; ++j) chosen |= ids[j] == i;
        if (!chosen) hi = fmaxf(hi, lg[i]);
    }
    g_moe_margin[g_moe_n++] = lo - hi;
}

int or_accept(const int32_t* draft, const int32_t* target, int k) {
    int a = 0;
    while (a < k && draft[a] == target[a]) ++a;
    return a;
}

// ---- the Qwen3 step ----
static void mm(const or_qwen3* m, const uint8_t* W, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nt) {
    if (m->wtype == 8) or_mul_mat_q8_0(W, N, K, X, M, Y, nt);
    else or_mul_mat_q4_0(W, N, K, X, M, Y, nt);
}
// the LM head (its own block type: Q6_K when tied to a Q6_K token table)
static void mm_head(const or_qwen3* m, int64_t N, int64_t K, const float* X, int64_t M, float* Y, int nt) {
    const int t = m->head_type ? m->head_type : m->wtype;
    if (t == 14) or_mul_mat_q6_K(m->output, N, K, X, M, Y, nt);
    else if (t == 8) or_mul_mat_q8_0(m->output, N, K, X, M, Y, nt);
    else or_mul_mat_q4_0(m->output, N, K, X, M, Y, nt);
}
// bytes of one block of the model's matrices
static size_t wblock(const or_qwen3* m) { return m->wtype == 8 ? 34 : 18; }

// One Qwen3 block over R rows, in place on the residual rows x [R][E] (the rows' rope tables in cs [R][D]). The block's
// K/V cells go to layer `kl` of the cache. kv_only: stop after writing them (the guess head's cache fill).
static void block(const or_qwen3* m, const or_layer* L, or_kv* kv, int kl, int R, const int32_t* seq,
                  const int32_t* pos, float* x, const float* cs, int kv_only, int nthreads) {
    const int E = m->n_embd, H = m->n_head, KVH = m->n_head_kv, D = m->head_dim, F = m->n_ff;
    const int QD = H * D, KD = KVH * D, G = H / KVH;
    const float scale = 1.0f / sqrtf((float) D);
    const int FF = F > m->n_ff_exp ? F : m->n_ff_exp;
    float* h = (float*) calloc((size_t) R * E, 4);
    float* q = (float*) malloc((size_t) R * QD * 4);
    float* k = (float*) malloc((size_t) R * KD * 4);
    float* v = (float*) malloc((size_t) R * KD * 4);
    float* ao = (float*) malloc((size_t) R * QD * 4);
    float* y = (float*) malloc((size_t) R * (E > QD ? E : QD) * 4);
    float* g = (float*) malloc((size_t) R * FF * 4);
    float* u = (float*) malloc((size_t) R * FF * 4);
    const size_t lstride = (size_t) kv->ctx * KD;  // one layer of one sequence
    for (int r = 0; r < R; ++r) or_rmsnorm(x + (size_t) r * E, L->attn_norm, E, m->eps, h + (size_t) r * E);
    if (!kv_only) mm(m, L->wq, QD, E, h, R, q, nthreads);
    mm(m, L->wk, KD, E, h, R, k, nthreads);
    mm(m, L->wv, KD, E, h, R, v, nthreads);
    for (int r = 0; r < R; ++r) {
        if (!kv_only)
            for (int hh = 0; hh < H; ++hh)
                or_qk_norm_rope(q + (size_t) r * QD + hh * D, L->q_norm, D, m->eps, cs + (size_t) r * D, 1);
        for (int hh = 0; hh < KVH; ++hh)
            or_qk_norm_rope(k + (size_t) r * KD + hh * D, L->k_norm, D, m->eps, cs + (size_t) r * D, 1);
        // the row's cell: K and V in fp16
        const size_t base = ((size_t) seq[r] * kv->n_layer + kl) * lstride + (size_t) pos[r] * KD;
        for (int i = 0; i < KD; ++i) {
            kv->k[base + i] = or_f32_to_f16(k[(size_t) r * KD + i]);
            kv->v[base + i] = or_f32_to_f16(v[(size_t) r * KD + i]);
        }
    }
    if (kv_only) goto done;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(dynamic, 1)
    for (int rh = 0; rh < R * H; ++rh) {
        const int r = rh / H, hh = rh % H, kh = hh / G, n = pos[r] + 1;
        const size_t base = ((size_t) seq[r] * kv->n_layer + kl) * lstride;
        const uint16_t** kp = (const uint16_t**) malloc((size_t) n * sizeof(void*));
        const uint16_t** vp = (const uint16_t**) malloc((size_t) n * sizeof(void*));
        for (int c = 0; c < n; ++c) {
            kp[c] = kv->k + base + (size_t) c * KD + (size_t) kh * D;
            vp[c] = kv->v + base + (size_t) c * KD + (size_t) kh * D;
        }
        attn_cells(q + (size_t) r * QD + hh * D, D, n, kp, vp, scale, ao + (size_t) r * QD + hh * D, 0);
        free(kp);
        free(vp);
    }
    mm(m, L->wo, E, QD, ao, R, y, nthreads);
    for (size_t i = 0; i < (size_t) R * E; ++i) x[i] += y[i];
    for (int r = 0; r < R; ++r) or_rmsnorm(x + (size_t) r * E, L->ffn_norm, E, m->eps, h + (size_t) r * E);
    if (m->n_expert > 0) {
        const int NE = m->n_expert, K = m->n_expert_used, FE = m->n_ff_exp;
        const size_t gsz = (size_t) FE * (E / QK) * wblock(m), dsz = (size_t) E * (FE / QK) * wblock(m);
        for (int r = 0; r < R; ++r) {
            float* lg = (float*) malloc((size_t) NE * 4);
            int32_t ids[64];
            float w[64];
            for (int e = 0; e < NE; ++e) {
                float s = 0.0f;
                for (int ii = 0; ii < E; ++ii) {
                    const int i = g_sum_reverse ? E - 1 - ii : ii;
                    s += L->router[(size_t) e * E + i] * h[(size_t) r * E + i];
                }
                lg[e] = s;
            }
            or_moe_route(lg, NE, K, ids, w);
            moe_note_margin(lg, NE, ids, K);
            float* acc = (float*) calloc((size_t) E, 4);
            for (int j = 0; j < K; ++j) {
                mm(m, L->eg + ids[j] * gsz, FE, E, h + (size_t) r * E, 1, g, nthreads);
                mm(m, L->eu + ids[j] * gsz, FE, E, h + (size_t) r * E, 1, u, nthreads);
                for (int i = 0; i < FE; ++i) g[i] = or_silu(g[i]) * u[i];
                mm(m, L->ed + ids[j] * dsz, E, FE, g, 1, y, nthreads);
                for (int i = 0; i < E; ++i) acc[i] += w[j] * y[i];
            }
            for (int i = 0; i < E; ++i) x[(size_t) r * E + i] += acc[i];
            free(acc);
            free(lg);
        }
    } else {
        mm(m, L->wg, F, E, h, R, g, nthreads);
        mm(m, L->wu, F, E, h, R, u, nthreads);
        for (size_t i = 0; i < (size_t) R * F; ++i) g[i] = or_silu(g[i]) * u[i];
        mm(m, L->wd, E, F, g, R, y, nthreads);
        for (size_t i = 0; i < (size_t) R * E; ++i) x[i] += y[i];
    }
done:
    free(h); free(q); free(k); free(v); free(ao); free(y); free(g); free(u);
}

void or_qwen3_step(const or_qwen3* m, or_kv* kv, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos,
                   int n_out, const int32_t* out_rows, float* logits, float* hidden, int32_t* out_tok, float* hn_all,
                   int nthreads) {
    const int E = m->n_embd, D = m->head_dim, V = m->n_vocab;
    const float theta_scale = powf(m->rope_base, -2.0f / D);
    float* x = (float*) malloc((size_t) R * E * 4);
    float* cs = (float*) malloc((size_t) R * D * 4);
    for (int r = 0; r < R; ++r) {
        memcpy(x + (size_t) r * E, m->tok_embd + (size_t) tok[r] * E, (size_t) E * 4);
        or_rope_cache(pos[r], theta_scale, D, cs + (size_t) r * D);
    }
    for (int il = 0; il < m->n_layer; ++il) block(m, &m->layers[il], kv, il, R, seq, pos, x, cs, 0, nthreads);
    if (hn_all)
        for (int r = 0; r < R; ++r) or_rmsnorm(x + (size_t) r * E, m->output_norm, E, m->eps, hn_all + (size_t) r * E);
    float* ho = (float*) malloc((size_t) (n_out > 0 ? n_out : 1) * E * 4);
    for (int j = 0; j < n_out; ++j) or_rmsnorm(x + (size_t) out_rows[j] * E, m->output_norm, E, m->eps, ho + (size_t) j * E);
    if (hidden) memcpy(hidden, ho, (size_t) n_out * E * 4);
    if (n_out > 0) mm_head(m, V, E, ho, n_out, logits, nthreads);
    for (int j = 0; j < n_out; ++j) out_tok[j] = or_argmax(logits + (size_t) j * V, V, NULL, 0);
    free(ho);
    free(x);
    free(cs);
}

// the guess head's input rows: eh_proj([enorm(embed(tok)); hnorm(hprev)]) (sn_cache.inc.h:357-363, sn_state.inc.h:294-305)
static void mtp_in(const or_qwen3* m, int R, const int32_t* tok, const float* hprev, float* x, int nthreads) {
    const int E = m->n_embd;
    float* cat = (float*) malloc((size_t) R * 2 * E * 4);
    for (int r = 0; r < R; ++r) {
        or_rmsnorm(m->tok_embd + (size_t) tok[r] * E, m->mtp_enorm, E, m->eps, cat + (size_t) r * 2 * E);
        or_rmsnorm(hprev + (size_t) r * E, m->mtp_hnorm, E, m->eps, cat + (size_t) r * 2 * E + E);
    }
    mm(m, m->mtp_eh, E, 2 * E, cat, R, x, nthreads);
    free(cat);
}

void or_mtp_fill(const or_qwen3* m, or_kv* kv, int R, const int32_t* tok, const int32_t* seq, const int32_t* pos,
                 const float* hprev, int nthreads) {
    const int E = m->n_embd, D = m->head_dim;
    const float theta_scale = powf(m->rope_base, -2.0f / D);
    float* x = (float*) malloc((size_t) R * E * 4);
    float* cs = (float*) malloc((size_t) R * D * 4);
    for (int r = 0; r < R; ++r) or_rope_cache(pos[r], theta_scale, D, cs + (size_t) r * D);
    mtp_in(m, R, tok, hprev, x, nthreads);
    block(m, m->mtp, kv, m->n_layer, R, seq, pos, x, cs, 1, nthreads);
    free(x);
    free(cs);
}

void or_mtp_guess(const or_qwen3* m, or_kv* kv, int seq, int32_t tok, int pos, int k, const float* hprev,
                  int32_t* out_tok, float* logits, int nthreads) {
    const int E = m->n_embd, D = m->head_dim, V = m->n_vocab;
    const float theta_scale = powf(m->rope_base, -2.0f / D);
    float* h = (float*) malloc((size_t) E * 4);
    float* x = (float*) malloc((size_t) E * 4);
    float* cs = (float*) malloc((size_t) D * 4);
    float* lg = (float*) malloc((size_t) V * 4);
    memcpy(h, hprev, (size_t) E * 4);
    int32_t t = tok;
    for (int j = 0; j < k; ++j) {
        const int32_t p = pos + j;
        or_rope_cache(p, theta_scale, D, cs);
        mtp_in(m, 1, &t, h, x, nthreads);
        block(m, m->mtp, kv, m->n_layer, 1, &seq, &p, x, cs, 0, nthreads);
        or_rmsnorm(x, m->mtp_head_norm, E, m->eps, h);  // the head's output state: the next row's hprev
        mm_head(m, V, E, h, 1, lg, nthreads);
        t = or_argmax(lg, V, NULL, 0);
        out_tok[j] = t;
        if (logits) memcpy(logits + (size_t) j * V, lg, (size_t) V * 4);
    }
    free(h); free(x); free(cs); free(lg);
}
