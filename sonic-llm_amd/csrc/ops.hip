// Row kernels of the step: token embedding, per-head QK-norm + NEOX RoPE + the fp16 K/V cache write, and greedy
// argmax (with the top-2 / log-sum-exp record of sn_want_probs).
#include <algorithm>

#include "sn_kernels_internal.h"
#include "sn_rows.h"

// ---- embedding: the token's fp32 table row (embed_rows / embed_into, sn_state.inc.h:250-272; the table is fp32 here)
// Token ids come from the host (checked there) or from an argmax on the GPU (a queued step's tokens, the guess head's
// drafts), which gives -1 for a row without a finite score (all NaN): an id outside [0, V) makes a zero row, read from
// nowhere, so such a row is garbage but never an access out of the table.
__global__ void k_embed(const float* __restrict__ table, int V, int E, const int32_t* __restrict__ tok,
                        float* __restrict__ x) {
    const int r = blockIdx.x, id = tok[r];
    const bool ok = id >= 0 && id < V;
    const float* src = table + (size_t) (ok ? id : 0) * E;
    for (int i = threadIdx.x; i < E; i += blockDim.x) x[(size_t) r * E + i] = ok ? src[i] : 0.0f;
}

void embed_rows(const float* table, int V, int E, const int32_t* tok, int R, float* x, hipStream_t st) {
    if (R > 0) hipLaunchKernelGGL(k_embed, dim3(R), dim3(256), 0, st, table, V, E, tok, x);
}

// ---- QK-norm + RoPE + K/V into the cache (qk_rope, kernels.metal:149-197) -------------------------------------------
// Lane i of a wavefront takes the dims (i, i + 64) of a head, which are a rotation pair for q and k. The rotation's
// cos / sin of theta_i = p * s^i (i successive fp32 multiplies from p, ggml_rope_cache_init's loop; s = base^(-2/128)
// computed on the host) are the same for every head of a row. Per q/k head: RMSNorm over 128 dims with weight w, then
// y_i = x_i cos - x_{i+64} sin, y_{i+64} = x_i sin + x_{i+64} cos. q stays in place (fp32); k and v go to the row's
// cell in fp16 (with part given, k and v as the matmul made them are also written into the row). Two launch shapes do
// the same operations in the same order with contraction off, so a row gets the same bits from either: k_qk_rope, a
// wavefront a head (the most wavefronts, for decode-sized steps), and k_qk_rope_rows (through rope_cs, qk_load and
// qk_head of sn_rows.h), a workgroup a row with the angles formed once and shared through LDS (for prompt-sized steps).
// The q|k|v matmul's fused epilogue (q4.hip) goes through rope_cs and qk_head too.
// a head's two dims: the q|k|v matmul's k-slice sums (added in slice order) or the row's values
template <int KM>
__device__ __forceinline__ void qk_load(const float* __restrict__ qkv, int ldqkv, const float* __restrict__ part, int ks,
                                        int R, int N, int r, int h, int lane, float& a0, float& a1) {
    if (part) {
        a0 = slices_sum1<KM>(part + (size_t) r * N + h * 128 + lane, (size_t) R * N, ks);
        a1 = slices_sum1<KM>(part + (size_t) r * N + h * 128 + lane + 64, (size_t) R * N, ks);
    } else {
        const float* x = qkv + (size_t) r * ldqkv + (size_t) h * 128;
        a0 = x[lane];
        a1 = x[lane + 64];
    }
}
// Workgroup (row, y): wavefront w takes head 4 y + w
template <int KM>
__global__ __launch_bounds__(256) void k_qk_rope(float* __restrict__ qkv, int ldqkv, const float* __restrict__ part,
                                                 int ks, int R, int H, int KVH, const float* __restrict__ qw,
                                                 const float* __restrict__ kw, float eps, float theta_scale,
                                                 const int32_t* __restrict__ seq, const int32_t* __restrict__ pos,
                                                 const int32_t* __restrict__ pt, int max_pages, int page_cells,
                                                 uint16_t* __restrict__ kpool, uint16_t* __restrict__ vpool,
                                                 const float2* __restrict__ cs) {
#pragma clang fp contract(off)
    const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = 4 * blockIdx.y + wave;
    if (h >= H + 2 * KVH) return;
    const bool isq = h < H, isv = h >= H + KVH;
    const int N = (H + 2 * KVH) * 128;
    float* x = qkv + (size_t) r * ldqkv + (size_t) h * 128;  // q heads, k heads, v heads: contiguous
    const float* w = isq ? qw : kw;
    const float w0 = isv ? 0.0f : w[lane], w1 = isv ? 0.0f : w[lane + 64];
    const int p = pos[r];
    const int page = pt[(size_t) seq[r] * max_pages + p / page_cells];
    const int off = p % page_cells;
    float x0, x1;
    if (part) {  // the q|k|v matmul's k-slice sums, added in slice order
        x0 = slices_sum1<KM>(part + (size_t) r * N + h * 128 + lane, (size_t) R * N, ks);
        x1 = slices_sum1<KM>(part + (size_t) r * N + h * 128 + lane + 64, (size_t) R * N, ks);
        if (!isq) {  // k and v as the matmul made them (q is overwritten below)
            x[lane] = x0;
            x[lane + 64] = x1;
        }
    } else {
        x0 = x[lane];
        x1 = x[lane + 64];
    }
    if (isv) {
        uint16_t* vc = vpool + (((size_t) page * KVH + (h - H - KVH)) * page_cells + off) * 128;
        vc[lane] = __builtin_bit_cast(uint16_t, (_Float16) x0);
        vc[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16) x1);
        return;
    }
    float c, s;
    if (cs) {  // the step's table (rope_table: the same function of (p, lane))
        const float2 t = cs[(size_t) r * 64 + lane];
        c = t.x, s = t.y;
    } else {
        rope_cs(p, lane, theta_scale, c, s);
    }
    float ss = x0 * x0 + x1 * x1;
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float sc = 1.0f / sqrtf(ss / 128.f + eps);
    x0 = (x0 * sc) * w0;
    x1 = (x1 * sc) * w1;
    const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
    if (isq) {
        x[lane] = y0;
        x[lane + 64] = y1;
    } else {
        uint16_t* kc = kpool + ((size_t) page * KVH + (h - H)) * page_cells * 128;
        kc[kcell_at(page_cells, off, lane)] = __builtin_bit_cast(uint16_t, (_Float16) y0);
        kc[kcell_at(page_cells, off, lane + 64)] = __builtin_bit_cast(uint16_t, (_Float16) y1);
    }
}

// Workgroup = one row of QKR_WAVES wavefronts: wavefront w takes heads w, w + QKR_WAVES, ... in rounds of
// QKR_WAVES x QKR_HPW heads, each round's loads issued before anything waits on them; wavefront 0 forms the angles
#define QKR_WAVES 16
#define QKR_HPW 4
#define QKR_ROWS_MIN 128  // steps of at least this many rows take k_qk_rope_rows
template <int KM>
__global__ __launch_bounds__(64 * QKR_WAVES) void k_qk_rope_rows(
    float* __restrict__ qkv, int ldqkv, const float* __restrict__ part, int ks, int R, int H, int KVH,
    const float* __restrict__ qw, const float* __restrict__ kw, float eps, float theta_scale,
    const int32_t* __restrict__ seq, const int32_t* __restrict__ pos, const int32_t* __restrict__ pt, int max_pages,
    int page_cells, uint16_t* __restrict__ kpool, uint16_t* __restrict__ vpool) {
    __shared__ float s_cs[2][64];
    const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NH = H + 2 * KVH;
    const float qw0 = qw[lane], qw1 = qw[lane + 64], kw0 = kw[lane], kw1 = kw[lane + 64];
    const int p = pos[r];
    const int page = pt[(size_t) seq[r] * max_pages + p / page_cells];
    float c = 0.0f, s = 0.0f;
    for (int h0 = 0; h0 < NH; h0 += QKR_WAVES * QKR_HPW) {  // the same trips in every wavefront
        float a0[QKR_HPW], a1[QKR_HPW];
        for (int j = 0; j < QKR_HPW; ++j)  // (past the last head: a re-read of it, unused)
            qk_load<KM>(qkv, ldqkv, part, ks, R, NH * 128, r, min(h0 + wave + QKR_WAVES * j, NH - 1), lane, a0[j],
                        a1[j]);
        if (h0 == 0) {
            if (wave == 0) rope_cs(p, lane, theta_scale, s_cs[0][lane], s_cs[1][lane]);
            __syncthreads();
            c = s_cs[0][lane];
            s = s_cs[1][lane];
        }
        for (int j = 0; j < QKR_HPW; ++j) {
            const int h = h0 + wave + QKR_WAVES * j;
            if (h >= NH) break;
            const bool isq = h < H;
            qk_head(qkv + (size_t) r * ldqkv + (size_t) h * 128, lane, h, H, KVH, part != nullptr, a0[j], a1[j], c,
                    s, isq ? qw0 : kw0, isq ? qw1 : kw1, eps, kpool, vpool, page, page_cells, p % page_cells);
        }
    }
}

// the rotation's (cos, sin) of rows 0 .. R - 1 at positions pos, lanes 0 .. 63 (rope_cs), into cs [R][64]
__global__ __launch_bounds__(64) void k_rope_table(const int32_t* __restrict__ pos, float theta_scale,
                                                   float2* __restrict__ cs) {
    float c, s;
    rope_cs(pos[blockIdx.x], threadIdx.x, theta_scale, c, s);
    cs[(size_t) blockIdx.x * 64 + threadIdx.x] = make_float2(c, s);
}

void rope_table(const int32_t* pos, int R, float theta_scale, float2* cs, hipStream_t st) {
    if (R > 0) hipLaunchKernelGGL(k_rope_table, dim3(R), dim3(64), 0, st, pos, theta_scale, cs);
}

int qk_norm_rope_kv(float* qkv, int ldqkv, const float* part, int ks, int R, int H, int KVH, const float* qw,
                    const float* kw, float eps, float theta_scale, const int32_t* seq, const int32_t* pos,
                    const int32_t* pt, int max_pages, int page_cells, uint16_t* kpool, uint16_t* vpool,
                    hipStream_t st, const float2* cs) {
    if (R <= 0) return 0;
    const int km = part ? ks_bound(ks) : 1;
    if (km == 0) return -1;  // more k-slices than the kernels add (q4_plan keeps every plan within KS_MAX)
    const bool rows = R >= QKR_ROWS_MIN;
    const dim3 grid = rows ? dim3(R) : dim3(R, (H + 2 * KVH + 3) / 4);
#define QKR(KM_)                                                                                                   \
    do {                                                                                                           \
        if (rows)                                                                                                  \
            hipLaunchKernelGGL((k_qk_rope_rows<KM_>), grid, dim3(64 * QKR_WAVES), 0, st, qkv, ldqkv, part, ks, R, \
                               H, KVH, qw, kw, eps, theta_scale, seq, pos, pt, max_pages, page_cells, kpool, vpool); \
        else                                                                                                       \
            hipLaunchKernelGGL((k_qk_rope<KM_>), grid, dim3(256), 0, st, qkv, ldqkv, part, ks, R, H, KVH, qw, kw, \
                               eps, theta_scale, seq, pos, pt, max_pages, page_cells, kpool, vpool, cs);         \
    } while (0)
    if (km == 1) QKR(1);
    else if (km == 2) QKR(2);
    else if (km == 4) QKR(4);
    else if (km == 8) QKR(8);
    else QKR(16);
#undef QKR
    return 0;
}

// ---- greedy argmax (argmax / argmax_p, kernels.metal:327-442) -------------------------------------------------------
// The first index of the largest score; rows with skip[r] never take the ids in ban (a row whose every id is banned
// gets -1). rec (optional): per row 8 words: chosen id, chosen score, best id, best score, second id, second score,
// log-sum-exp, 0 (ids ascending among ties; the best/second pair over all ids, banned or not). NaN scores never win.
// Two launches: every (row, chunk of AMX_CHUNK ids) workgroup reduces its chunk to a partial record, then one
// wavefront per row merges the row's partials, so a batch of rows spreads over the whole chip.
struct Top2 {
    float m1;
    int i1;
    float m2;
    int i2;
};
__device__ __forceinline__ bool better(float v, int i, float w, int j) { return v > w || (v == w && i < j); }
__device__ __forceinline__ Top2 top2_merge(Top2 a, Top2 b) {
    Top2 w = a, l = b;
    if (better(b.m1, b.i1, a.m1, a.i1)) {
        w = b;
        l = a;
    }
    Top2 o = w;
    if (better(l.m1, l.i1, w.m2, w.i2)) {
        o.m2 = l.m1;
        o.i2 = l.i1;
    }
    return o;
}
// the partial of a chunk: chosen (best, idx), the pair (tp), and the chunk's sum of exp(x - tp.m1) (z)
struct AmxPart {
    float best;
    int idx;
    Top2 tp;
    float z;
    float pad;
};
// merge of two partials; z of the one with the smaller max is rescaled (an empty side, max -inf, adds nothing)
__device__ __forceinline__ AmxPart amx_merge(AmxPart a, AmxPart b, bool lse) {
    AmxPart o;
    const bool bb = better(b.best, b.idx, a.best, a.idx);
    o.best = bb ? b.best : a.best;
    o.idx = bb ? b.idx : a.idx;
    o.tp = top2_merge(a.tp, b.tp);
    o.z = 0.0f;
    if (lse) {
        const float m = o.tp.m1;
        if (m > -INFINITY) {
            if (a.tp.m1 > -INFINITY) o.z += a.z * expf(a.tp.m1 - m);
            if (b.tp.m1 > -INFINITY) o.z += b.z * expf(b.tp.m1 - m);
        }
    }
    o.pad = 0.0f;
    return o;
}
__device__ __forceinline__ AmxPart amx_shfl(AmxPart p, int o) {
    AmxPart q;
    q.best = __shfl_xor(p.best, o);
    q.idx = __shfl_xor(p.idx, o);
    q.tp.m1 = __shfl_xor(p.tp.m1, o);
    q.tp.i1 = __shfl_xor(p.tp.i1, o);
    q.tp.m2 = __shfl_xor(p.tp.m2, o);
    q.tp.i2 = __shfl_xor(p.tp.i2, o);
    q.z = __shfl_xor(p.z, o);
    q.pad = 0.0f;
    return q;
}
__device__ __forceinline__ AmxPart amx_wave(AmxPart p, bool lse) {
    for (int o = 32; o > 0; o >>= 1) p = amx_merge(p, amx_shfl(p, o), lse);
    return p;
}

#define AMX_PER_THREAD (AMX_CHUNK / 256)
template <bool LSE>
__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ logits, int V, int nch,
                                                     const int32_t* __restrict__ ban, int nban,
                                                     const uint8_t* __restrict__ skip, AmxPart* __restrict__ part) {
    __shared__ AmxPart sp[4];
    const int c = blockIdx.x, r = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float* x = logits + (size_t) r * V;
    const int nb = (skip && skip[r]) ? nban : 0;
    int bn[8];
    for (int k = 0; k < 8; ++k) bn[k] = k < nb ? ban[k] : -1;
    const int i0 = c * AMX_CHUNK + t;
    float v[AMX_PER_THREAD];
    for (int k = 0; k < AMX_PER_THREAD; ++k) {
        const int i = i0 + 256 * k;
        v[k] = i < V ? x[i] : -INFINITY;
    }
    AmxPart p = {-INFINITY, 0x7fffffff, {-INFINITY, 0x7fffffff, -INFINITY, 0x7fffffff}, 0.0f, 0.0f};
    for (int k = 0; k < AMX_PER_THREAD; ++k) {  // ids ascending: strict > keeps the lower id of a tie
        const int i = i0 + 256 * k;
        if (i >= V) break;
        bool b = false;
        for (int j = 0; j < 8; ++j) b = b || i == bn[j];
        if (!b && (p.idx == 0x7fffffff || v[k] > p.best)) {
            p.best = v[k];
            p.idx = i;
        }
        if (v[k] > p.tp.m1) {
            p.tp.m2 = p.tp.m1;
            p.tp.i2 = p.tp.i1;
            p.tp.m1 = v[k];
            p.tp.i1 = i;
        } else if (v[k] > p.tp.m2) {
            p.tp.m2 = v[k];
            p.tp.i2 = i;
        }
    }
    if (LSE && p.tp.m1 > -INFINITY)
        for (int k = 0; k < AMX_PER_THREAD; ++k)
            if (i0 + 256 * k < V) p.z += expf(v[k] - p.tp.m1);
    p = amx_wave(p, LSE);
    if (lane == 0) sp[w] = p;
    __syncthreads();
    if (t == 0) {
        for (int k = 1; k < 4; ++k) p = amx_merge(p, sp[k], LSE);
        part[(size_t) r * nch + c] = p;
    }
}

template <bool LSE>
__global__ __launch_bounds__(64) void k_argmax_fin(const AmxPart* __restrict__ part, int nch, int32_t* __restrict__ out,
                                                   float* __restrict__ rec) {
    const int r = blockIdx.x, lane = threadIdx.x;
    AmxPart p = {-INFINITY, 0x7fffffff, {-INFINITY, 0x7fffffff, -INFINITY, 0x7fffffff}, 0.0f, 0.0f};
    for (int c = lane; c < nch; c += 64) p = amx_merge(p, part[(size_t) r * nch + c], LSE);
    p = amx_wave(p, LSE);
    if (lane != 0) return;
    const int idx = p.idx == 0x7fffffff ? -1 : p.idx;
    out[r] = idx;
    if (!LSE) return;
    float* q = rec + (size_t) r * 8;
    q[0] = __builtin_bit_cast(float, idx);
    q[1] = p.best;
    q[2] = __builtin_bit_cast(float, p.tp.i1);
    q[3] = p.tp.m1;
    q[4] = __builtin_bit_cast(float, p.tp.i2);
    q[5] = p.tp.m2;
    q[6] = p.tp.m1 > -INFINITY ? p.tp.m1 + logf(p.z) : -INFINITY;
    q[7] = 0.0f;
}

size_t argmax_workspace_bytes(int n, int V) { return (size_t) n * argmax_chunks(V) * sizeof(AmxPart); }

int argmax_rows(const float* logits, int V, int n, const int32_t* ban, int nban, const uint8_t* skip, int32_t* out,
                float* rec, void* ws, size_t ws_bytes, hipStream_t st) {
    if (n <= 0) return 0;
    if (V <= 0 || nban < 0 || nban > 8 || argmax_workspace_bytes(n, V) > ws_bytes) return -1;
    const int nch = argmax_chunks(V);
    AmxPart* part = (AmxPart*) ws;
    if (rec) {
        hipLaunchKernelGGL(k_argmax_part<true>, dim3(nch, n), dim3(256), 0, st, logits, V, nch, ban, nban, skip, part);
        hipLaunchKernelGGL(k_argmax_fin<true>, dim3(n), dim3(64), 0, st, part, nch, out, rec);
    } else {
        hipLaunchKernelGGL(k_argmax_part<false>, dim3(nch, n), dim3(256), 0, st, logits, V, nch, ban, nban, skip, part);
        hipLaunchKernelGGL(k_argmax_fin<false>, dim3(n), dim3(64), 0, st, part, nch, out, rec);
    }
    return 0;
}

// ---- page operations of the cache (sn_copy / sn_clear / freed pages; sn_seq.inc.h:5-145) ----------------------------
__global__ void k_kv_page_op(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int KVH, int page_cells, int src,
                             int dst, int a, int b) {
    const int l = blockIdx.x, t = blockIdx.y, h = blockIdx.z;  // (cells a .. b - 1 of the page)
    uint16_t* pool = (t == 0 ? kbase : vbase) + (size_t) l * layer_halves;
    uint16_t* d = pool + ((size_t) dst * KVH + h) * page_cells * 128;
    const uint16_t* s = src >= 0 ? pool + ((size_t) src * KVH + h) * page_cells * 128 : nullptr;
    const int n = (b - a) * 128;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const size_t at = t == 0 ? kcell_at(page_cells, a + i / 128, i % 128) : (size_t) a * 128 + i;
        d[at] = s ? s[at] : (uint16_t) 0;
    }
}

void kv_page_op(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells, int src, int dst,
                int a, int b, hipStream_t st) {
    if (b > a)
        hipLaunchKernelGGL(k_kv_page_op, dim3(L, 2, KVH), dim3(256), 0, st, kbase, vbase, layer_halves, KVH, page_cells,
                           src, dst, a, b);
}

__global__ void k_kv_stage(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int KVH, int page_cells,
                           const int32_t* pages, int n, uint16_t* staging, int save) {
    const int l = blockIdx.y, t = blockIdx.z;
    const int c = blockIdx.x;  // cell
    if (c >= n) return;
    uint16_t* pool = (t == 0 ? kbase : vbase) + (size_t) l * layer_halves;
    const int p = pages[c / page_cells];
    uint16_t* stg = staging + (((size_t) l * 2 + t) * n + c) * (size_t) KVH * 128;
    for (int i = threadIdx.x; i < KVH * 128; i += blockDim.x) {
        const int h = i / 128, d = i % 128;
        const size_t in = t == 0 ? kcell_at(page_cells, c % page_cells, d) : (size_t) (c % page_cells) * 128 + d;
        uint16_t* cell = pool + ((size_t) p * KVH + h) * page_cells * 128 + in;
        if (save) stg[i] = *cell;
        else *cell = stg[i];
    }
}

void kv_stage(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells,
              const int32_t* pages, int n, uint16_t* staging, int save, hipStream_t st) {
    if (n > 0)
        hipLaunchKernelGGL(k_kv_stage, dim3(n, L, 2), dim3(256), 0, st, kbase, vbase, layer_halves, KVH, page_cells,
                           pages, n, staging, save);
}

// ---- synthetic context: seeded N(0, 1) fp16 cells (snx_fill_kv) ------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void k_kv_fill(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int KVH, int page_cells,
                          const int32_t* pages, int n, uint64_t seed) {
    const int c = blockIdx.x, l = blockIdx.y, t = blockIdx.z;  // cell, layer, K or V
    if (c >= n) return;
    uint16_t* pool = (t == 0 ? kbase : vbase) + (size_t) l * layer_halves;
    const int p = pages[c / page_cells];
    for (int i = threadIdx.x; i < KVH * 128; i += blockDim.x) {
        const int h = i / 128, d = i % 128;
        const uint64_t key = seed ^ mix64(((uint64_t) l * 2 + t) * 0x100000000ull + (uint64_t) c * 4096 + i);
        const uint64_t a = mix64(key), b = mix64(key ^ 0x9E3779B97F4A7C15ull);
        const float u1 = ((a >> 40) + 1) * 0x1.0p-24f, u2 = (b >> 40) * 0x1.0p-24f;
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
        const size_t in = t == 0 ? kcell_at(page_cells, c % page_cells, d) : (size_t) (c % page_cells) * 128 + d;
        pool[((size_t) p * KVH + h) * page_cells * 128 + in] = __builtin_bit_cast(uint16_t, (_Float16) z);
    }
}

void kv_fill_normal(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int L, int KVH, int page_cells,
                    const int32_t* pages, int n, uint64_t seed, hipStream_t st) {
    if (n > 0)
        hipLaunchKernelGGL(k_kv_fill, dim3(n, L, 2), dim3(256), 0, st, kbase, vbase, layer_halves, KVH, page_cells, pages,
                           n, seed);
}

// ---- the guess head (MTP) and the fused draft-verify step ----------------------------------------------------------

__device__ __forceinline__ float row_sumsq256(const float* x, int n, float* red) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s += x[i] * x[i];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// The head's input rows [enorm(embed(tok)); hnorm(h)] (sn_cache.inc.h:357-363, sn_state.inc.h:294-305), h the row's
// hidden state before it: src NULL: hrows row r when hrows is given, else the slot's kept state pend[seq]; with src:
// src[r] >= 0 row src[r] of hrows, -1 pend[seq[r]], -2 none (zeros: a sequence's first cell). Both rows (E <=
// 256 MTP_CAT_J) are loaded before either sum of squares is reduced: one latency period, not two; each sum keeps the
// per-thread order and reduction of row_sumsq256.
#define MTP_CAT_J 16
__global__ __launch_bounds__(256) void k_mtp_cat(const float* __restrict__ table, int V, int E,
                                                 const int32_t* __restrict__ tok,
                                                 const float* __restrict__ hrows, const float* __restrict__ pend,
                                                 const int32_t* __restrict__ src, const int32_t* __restrict__ seq,
                                                 const float* __restrict__ enorm, const float* __restrict__ hnorm,
                                                 float eps, float* __restrict__ cat) {
    __shared__ float red[2][4];
    const int r = blockIdx.x, t = threadIdx.x;
    const int id = tok[r];
    const bool tok_ok = id >= 0 && id < V;  // (an id outside [0, V): a zero embedding, as in k_embed)
    const float* em = table + (size_t) (tok_ok ? id : 0) * E;
    const int s = src ? src[r] : (hrows ? r : -1);
    const float* h = s >= 0 ? hrows + (size_t) s * E : s == -1 ? pend + (size_t) seq[r] * E : nullptr;
    float* y = cat + (size_t) r * 2 * E;
    float ve[MTP_CAT_J], vh[MTP_CAT_J];
    for (int j = 0; j < MTP_CAT_J; ++j) {
        const int i = t + 256 * j;
        ve[j] = tok_ok && i < E ? em[i] : 0.0f;
        vh[j] = h && i < E ? h[i] : 0.0f;
    }
    float se = 0.0f, sh = 0.0f;
    for (int j = 0; j < MTP_CAT_J; ++j)
        if (t + 256 * j < E) {
            se += ve[j] * ve[j];
            sh += vh[j] * vh[j];
        }
    for (int o = 32; o > 0; o >>= 1) {
        se += __shfl_xor(se, o);
        sh += __shfl_xor(sh, o);
    }
    if ((t & 63) == 0) {
        red[0][t >> 6] = se;
        red[1][t >> 6] = sh;
    }
    __syncthreads();
    const float ie = 1.0f / sqrtf(((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / (float) E + eps);
    const float ih = 1.0f / sqrtf(((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float) E + eps);
    for (int j = 0; j < MTP_CAT_J; ++j) {
        const int i = t + 256 * j;
        if (i >= E) break;
        y[i] = (ve[j] * ie) * enorm[i];
        y[E + i] = h ? (vh[j] * ih) * hnorm[i] : 0.0f;
    }
}

void mtp_cat(const float* table, int V, int E, const int32_t* tok, const float* hrows, const float* pend,
             const int32_t* src, const int32_t* seq, const float* enorm, const float* hnorm, float eps, float* cat,
             int R, hipStream_t st) {
    if (R > 0 && E <= 256 * MTP_CAT_J)
        hipLaunchKernelGGL(k_mtp_cat, dim3(R), dim3(256), 0, st, table, V, E, tok, hrows, pend, src, seq, enorm, hnorm,
                           eps, cat);
}

// keep[j] = (slot, row): dst row `slot` = src row `row` (mtp_keep: a slot's last hidden state of the step)
__global__ void k_rows_keep(const float* __restrict__ src, const int32_t* __restrict__ keep, int E,
                            float* __restrict__ dst) {
    const int slot = keep[2 * blockIdx.x], row = keep[2 * blockIdx.x + 1];
    if (slot < 0) return;
    for (int i = threadIdx.x; i < E; i += 256) dst[(size_t) slot * E + i] = src[(size_t) row * E + i];
}

void rows_keep(const float* src, const int32_t* keep, int n, int E, float* dst, hipStream_t st) {
    if (n > 0) hipLaunchKernelGGL(k_rows_keep, dim3(n), dim3(256), 0, st, src, keep, E, dst);
}

// Verify rows (sequence s, row i = 0 .. k at position pos_s + i) from the drafts gtok[j][s] (round j's guess of s):
// row i > 0 takes draft i - 1; ftok[row] = the draft the row's argmax is checked against (row i < k: draft i).
__global__ void k_spec_rows(int n, int k, int slots, const int32_t* __restrict__ gtok, int32_t* __restrict__ vtok,
                            int32_t* __restrict__ ftok) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * (k + 1)) return;
    const int s = t / (k + 1), i = t % (k + 1);
    if (i > 0) vtok[t] = gtok[(i - 1) * slots + s];
    ftok[t] = i < k ? gtok[i * slots + s] : 0;
}

// rows with force[r]: the draft ftok[r] becomes the row's greedy token (a seeded acceptance rate for benchmarks)
__global__ void k_force(float* __restrict__ logits, int V, int R, const uint8_t* __restrict__ force,
                        const int32_t* __restrict__ ftok) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < R && force[r] && ftok[r] >= 0 && ftok[r] < V) logits[(size_t) r * V + ftok[r]] = 3.0e38f;
}

// Greedy acceptance (next_engine/take.rs:339-357) per sequence: a = the leading drafts equal to their row's argmax;
// the sequence takes drafts 1 .. a and then row a's argmax. out_n[s] = a + 1, out_tok[s][0 .. a]; keep[s] = (slot,
// row of the last kept cell) for the guess head's state; acc[s] = a.
__global__ void k_accept(int n, int k, int slots, const int32_t* __restrict__ gtok, const int32_t* __restrict__ otok,
                         const int32_t* __restrict__ seq, int32_t* __restrict__ out_n, int32_t* __restrict__ out_tok,
                         int32_t* __restrict__ keep, int32_t* __restrict__ acc) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const int r0 = s * (k + 1);
    int a = 0;
    while (a < k && gtok[a * slots + s] == otok[r0 + a]) ++a;
    for (int i = 0; i < a; ++i) out_tok[s * (k + 1) + i] = gtok[i * slots + s];
    out_tok[s * (k + 1) + a] = otok[r0 + a];
    for (int i = a + 1; i <= k; ++i) out_tok[s * (k + 1) + i] = -1;
    out_n[s] = a + 1;
    keep[2 * s] = seq[r0];
    keep[2 * s + 1] = r0 + a;
    acc[s] = a;
}

// the cells of the refused rows (positions pos_s + acc_s + 1 .. pos_s + k) zeroed in every cache layer
__global__ void k_cut_cells(uint16_t* __restrict__ kbase, uint16_t* __restrict__ vbase, size_t layer_halves, int KVH,
                            int page_cells, const int32_t* __restrict__ pt, int max_pages, int k,
                            const int32_t* __restrict__ seq, const int32_t* __restrict__ pos,
                            const int32_t* __restrict__ acc) {
    const int s = blockIdx.x, i = blockIdx.y + 1, layer = blockIdx.z;
    if (i <= acc[s]) return;
    const int r0 = s * (k + 1), c = pos[r0] + i;
    const int page = pt[(size_t) seq[r0] * max_pages + c / page_cells];
    if (page < 0) return;
    const size_t base = (size_t) layer * layer_halves;
    for (int t = threadIdx.x; t < KVH * 128; t += 256) {
        const int h = t / 128, d = t % 128;
        const size_t reg = base + ((size_t) page * KVH + h) * page_cells * 128;
        kbase[reg + kcell_at(page_cells, c % page_cells, d)] = 0;
        vbase[reg + (size_t) (c % page_cells) * 128 + d] = 0;
    }
}

void spec_rows(int n, int k, int slots, const int32_t* gtok, int32_t* vtok, int32_t* ftok, hipStream_t st) {
    const int R = n * (k + 1);
    hipLaunchKernelGGL(k_spec_rows, dim3((R + 255) / 256), dim3(256), 0, st, n, k, slots, gtok, vtok, ftok);
}
void force_rows(float* logits, int V, int R, const uint8_t* force, const int32_t* ftok, hipStream_t st) {
    hipLaunchKernelGGL(k_force, dim3((R + 255) / 256), dim3(256), 0, st, logits, V, R, force, ftok);
}
void accept_rows(int n, int k, int slots, const int32_t* gtok, const int32_t* otok, const int32_t* seq, int32_t* out_n,
                 int32_t* out_tok, int32_t* keep, int32_t* acc, hipStream_t st) {
    hipLaunchKernelGGL(k_accept, dim3((n + 63) / 64), dim3(64), 0, st, n, k, slots, gtok, otok, seq, out_n, out_tok, keep,
                       acc);
}
void cut_cells(uint16_t* kbase, uint16_t* vbase, size_t layer_halves, int CL, int KVH, int page_cells, const int32_t* pt,
               int max_pages, int n, int k, const int32_t* seq, const int32_t* pos, const int32_t* acc, hipStream_t st) {
    if (k > 0)
        hipLaunchKernelGGL(k_cut_cells, dim3(n, k, CL), dim3(256), 0, st, kbase, vbase, layer_halves, KVH, page_cells, pt,
                           max_pages, k, seq, pos, acc);
}

// ---- mixture of experts (moe_ffn, sn_layers.inc.h:129-144) -----------------------------------------------------------

// Wavefront reductions by DPP, to lane 63 (then read from it): pairs, quads, half rows, rows, then row 0 into row 1 and
// row 2 into row 3, then rows 0-1 into rows 2-3. A fixed order: the sum of 64 values depends on their lanes alone.
// (a lane of a row that ROWMASK leaves out keeps `old`)
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ float dppf(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xF, false));
}
__device__ __forceinline__ float lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dppf<0xB1>(0.0f, v);        // quad_perm [1,0,3,2]
    v += dppf<0x4E>(0.0f, v);        // quad_perm [2,3,0,1]
    v += dppf<0x141>(0.0f, v);       // row_half_mirror
    v += dppf<0x140>(0.0f, v);       // row_mirror
    v += dppf<0x142, 0xA>(0.0f, v);  // row_bcast15 into rows 1, 3
    v += dppf<0x143, 0xC>(0.0f, v);  // row_bcast31 into rows 2, 3
    return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dppf<0xB1>(v, v));
    v = fmaxf(v, dppf<0x4E>(v, v));
    v = fmaxf(v, dppf<0x141>(v, v));
    v = fmaxf(v, dppf<0x140>(v, v));
    v = fmaxf(v, dppf<0x142, 0xA>(v, v));
    v = fmaxf(v, dppf<0x143, 0xC>(v, v));
    return lane63(v);
}

// Router logits [R][NE] = hn [R][E] (the normed rows) x router [NE][E] (fp32). Workgroup of 4 wavefronts: 4 experts x
// RT_ROWS rows, wavefront q a quarter of E for all 16 (expert, row) pairs. Lane l's part of a pair is, for its quarter,
// the elements 4l + 256j .. 4l + 256j + 3 (j of the quarter ascending, each 256-element step a 1 KB load of the
// wavefront); the four quarters' parts are added in order through LDS, then the 64 lanes by wave_sum. The order of a
// row's sum depends on E alone, not on the other rows. Every load of a wavefront (JM / 4 float4 of each of 4 rows and 4
// experts a lane, E <= 256 JM) is issued before any is used.
#define RT_ROWS 4
// the quarters' parts (s_part [quarter][pair][lane], written by every wavefront) added, then the lanes: wavefront q
// finishes expert x0 + q's rows
__device__ __forceinline__ void router_finish(int R, int NE, float* __restrict__ out, int x0, int r0,
                                              float (*s_part)[4 * RT_ROWS][64]) {
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
    __syncthreads();
    float v[RT_ROWS];
    for (int i = 0; i < RT_ROWS; ++i) {
        const int p = q * RT_ROWS + i;
        v[i] = ((s_part[0][p][lane] + s_part[1][p][lane]) + s_part[2][p][lane]) + s_part[3][p][lane];
    }
    for (int i = 0; i < RT_ROWS; ++i) v[i] = wave_sum(v[i]);
    if (lane == 0 && x0 + q < NE)
        for (int i = 0; i < RT_ROWS; ++i)
            if (r0 + i < R) out[(size_t) (r0 + i) * NE + x0 + q] = v[i];
}
template <int JM>
__device__ __forceinline__ void router_dot(const float* __restrict__ hn, const float* __restrict__ router, int R, int E,
                                           int NE, float* __restrict__ out, int x0, int r0,
                                           float (*s_part)[4 * RT_ROWS][64]) {
    constexpr int JQ = JM / 4;
    const int t = threadIdx.x, lane = t & 63, q = t >> 6;
    float4 wv[4][JQ], hv[RT_ROWS][JQ];
    for (int jj = 0; jj < JQ; ++jj) {
        const int e0 = min(4 * lane + 256 * (q * JQ + jj), E - 4);
        for (int u = 0; u < 4; ++u) wv[u][jj] = *(const float4*) (router + (size_t) min(x0 + u, NE - 1) * E + e0);
        for (int i = 0; i < RT_ROWS; ++i) hv[i][jj] = *(const float4*) (hn + (size_t) min(r0 + i, R - 1) * E + e0);
    }
    for (int u = 0; u < 4; ++u)
        for (int i = 0; i < RT_ROWS; ++i) {
            float s = 0.0f;
            for (int jj = 0; jj < JQ; ++jj)
                if (4 * lane + 256 * (q * JQ + jj) < E) {
                    const float4 h = hv[i][jj], w = wv[u][jj];
                    s += h.x * w.x + h.y * w.y + h.z * w.z + h.w * w.w;
                }
            s_part[q][u * RT_ROWS + i][lane] = s;
        }
    router_finish(R, NE, out, x0, r0, s_part);
}
// the rows' logits for experts 4 blockIdx.x .. + 3, rows RT_ROWS blockIdx.y ..
template <int JM>
__global__ __launch_bounds__(256) void k_router(const float* __restrict__ hn, const float* __restrict__ router, int R,
                                                int E, int NE, float* __restrict__ out) {
    __shared__ float s_part[4][4 * RT_ROWS][64];
    router_dot<JM>(hn, router, R, E, NE, out, blockIdx.x * 4, blockIdx.y * RT_ROWS, s_part);
}
// E > MOE_ROUTE_EMAX: quarters of ceil(E / 1024) steps, each step's loads in turn
__global__ __launch_bounds__(256) void k_router_any(const float* __restrict__ hn, const float* __restrict__ router,
                                                    int R, int E, int NE, float* __restrict__ out) {
    __shared__ float s_part[4][4 * RT_ROWS][64];
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6, x0 = blockIdx.x * 4, r0 = blockIdx.y * RT_ROWS;
    const int JQ = (E + 1023) / 1024;
    float s[4][RT_ROWS];
    for (int u = 0; u < 4; ++u)
        for (int i = 0; i < RT_ROWS; ++i) s[u][i] = 0.0f;
    for (int jj = 0; jj < JQ; ++jj) {
        const int e0 = 4 * lane + 256 * (q * JQ + jj);
        if (e0 >= E) break;
        for (int u = 0; u < 4; ++u) {
            const float4 w = *(const float4*) (router + (size_t) min(x0 + u, NE - 1) * E + e0);
            for (int i = 0; i < RT_ROWS; ++i) {
                const float4 h = *(const float4*) (hn + (size_t) min(r0 + i, R - 1) * E + e0);
                s[u][i] += h.x * w.x + h.y * w.y + h.z * w.z + h.w * w.w;
            }
        }
    }
    for (int u = 0; u < 4; ++u)
        for (int i = 0; i < RT_ROWS; ++i) s_part[q][u * RT_ROWS + i][lane] = s[u][i];
    router_finish(R, NE, out, x0, r0, s_part);
}
// the register width of the routing kernels' instances for E (0: E > MOE_ROUTE_EMAX)
static inline int router_jm(int E) { return E <= 1024 ? 4 : E <= 2048 ? 8 : E <= MOE_ROUTE_EMAX ? 16 : 0; }

// Routing of a row (moe_topk1, kernels.metal:3419-3467): softmax of its NE <= 256 logits, the k <= 8 largest (ties: the
// lower id), weights p / sum(p) renormalised by their own sum floored at 6.103515625e-5. One wavefront a row, lane l
// holding experts l + 64 s (s = 0..3): the max and the sum by wave_max / wave_sum (lane l's four added first, in slot
// order), then k rounds of: the largest remaining probability (wave_max), the lowest id holding it (ballots over the
// slots, in id order), that slot marked taken. A NaN probability counts as -1, below every number, so the ids are
// always k distinct experts of [0, NE). l4: this lane's logits (-inf past NE); ids, w: the row's k outputs.
template <bool SYS = false>  // SYS: the ids stored system-coherently (read on another XCD in the same launch)
__device__ __forceinline__ void moe_topk_wave(const float l4[4], int NE, int k, int32_t* __restrict__ ids,
                                              float* __restrict__ w) {
    const int lane = threadIdx.x & 63;
    const float m = wave_max(fmaxf(fmaxf(l4[0], l4[1]), fmaxf(l4[2], l4[3])));
    float p[4], e[4];
    for (int s = 0; s < 4; ++s) {
        e[s] = lane + 64 * s < NE ? expf(l4[s] - m) : 0.0f;
        p[s] = lane + 64 * s < NE ? (e[s] == e[s] ? e[s] : -1.0f) : -4.0f;  // (-4: no expert; -3: taken)
    }
    const float tot = wave_sum((e[0] + e[1]) + (e[2] + e[3]));
    int my_id = 0;
    float my_p = 0.0f, sel = 0.0f;
    for (int j = 0; j < MOE_MAX_K; ++j) {
        if (j >= k) break;
        const float M = wave_max(fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])));
        int id = -1;
        for (int s = 0; s < 4; ++s) {
            const uint64_t b = __ballot(p[s] == M);
            if (id < 0 && b) id = 64 * s + __ffsll((unsigned long long) b) - 1;
        }
        for (int s = 0; s < 4; ++s)
            if (id == lane + 64 * s) p[s] = -3.0f;
        if (lane == j) {
            my_id = id;
            my_p = M;
        }
        sel += M / tot;
    }
    sel = fmaxf(sel, 6.103515625e-5f);
    if (lane < k) {
        if (SYS)
            __hip_atomic_store(ids + lane, my_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        else
            ids[lane] = my_id;
        w[lane] = (my_p / tot) / sel;
    }
}
// rows 4 blockIdx.x + wave
__global__ __launch_bounds__(256) void k_moe_topk(const float* __restrict__ lg, int R, int NE, int k,
                                                  int32_t* __restrict__ ids, float* __restrict__ w) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= R) return;
    float l4[4];
    for (int s = 0; s < 4; ++s) l4[s] = lane + 64 * s < NE ? lg[(size_t) r * NE + lane + 64 * s] : -INFINITY;
    moe_topk_wave(l4, NE, k, ids + (size_t) r * k, w + (size_t) r * k);
}

// The (row, slot) pairs in expert-major tiles of 16 rows (moe_lists, kernels.metal:3468-3497), deterministically: expert
// x's pairs take tiles toff[x] .. in (row, slot) order. prow[r][j] = the pair's row in that layout; rsrc[p] = the row
// whose operand tile row p carries (-1: padding); items = (expert, tile) of every tile, count = their number. One
// workgroup of NW wavefronts: wavefront w owns the w-th of NW chunks of the pairs and counts its experts (LDS atomics:
// counts, not order); an expert's chunk counts become its chunks' starting places (a prefix over chunks) and its total
// gives the tile offsets (a wavefront prefix over experts); then each wavefront walks its chunk 64 pairs at a time, a
// pair's place = its chunk's place for the expert + the earlier pairs of the 64 with that expert (the lanes holding
// the same expert found by ballots over the id's bits). The result does not depend on NW.
#define MOE_MAX_PAIRS 4096
template <int NW>
struct GroupShared {
    int sid[MOE_MAX_PAIRS];
    int hist[NW][256];  // [chunk][expert]: counts, then the chunk's next place for the expert
    int cnt[256], toff[257];
};
// SYS: the ids were written on other XCDs in this launch (system-coherent loads)
template <bool SYS, int NW>
__device__ __forceinline__ void moe_group(GroupShared<NW>& sh, const int32_t* __restrict__ ids, int RK, int NE, int P,
                                          int k, int32_t* __restrict__ prow, int32_t* __restrict__ rsrc,
                                          int32_t* __restrict__ items, int32_t* __restrict__ count) {
    constexpr int NT = 64 * NW;
    int* sid = sh.sid;
    int (*hist)[256] = sh.hist;
    int* cnt = sh.cnt;
    int* toff = sh.toff;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int i = t; i < NW * 256; i += NT) (&hist[0][0])[i] = 0;
    for (int p = t; p < P; p += NT) rsrc[p] = -1;
    for (int q = t; q < RK; q += NT)
        sid[q] = SYS ? __hip_atomic_load(ids + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : ids[q];
    __syncthreads();
    const int C = (RK + NW - 1) / NW, q0 = wave * C, q1 = min(RK, q0 + C);
    for (int q = q0 + lane; q < q1; q += 64) atomicAdd(&hist[wave][sid[q]], 1);
    __syncthreads();
    for (int x = t; x < NE; x += NT) {
        int s = 0;
        for (int c = 0; c < NW; ++c) {
            const int h = hist[c][x];
            hist[c][x] = s;
            s += h;
        }
        cnt[x] = s;
    }
    __syncthreads();
    if (wave == 0) {  // toff[x] = tiles of the experts before x (lane l: experts 4l .. 4l + 3)
        int c[4], loc = 0;
        for (int j = 0; j < 4; ++j) {
            const int x = 4 * lane + j;
            c[j] = x < NE ? (cnt[x] + 15) / 16 : 0;
            loc += c[j];
        }
        int inc = loc;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(inc, o);
            if (lane >= o) inc += v;
        }
        int o = inc - loc;
        for (int j = 0; j < 4; ++j) {
            const int x = 4 * lane + j;
            if (x < NE) toff[x] = o;
            o += c[j];
        }
        if (lane == 63) {
            toff[NE] = inc;
            *count = inc;
        }
    }
    __syncthreads();
    for (int g0 = q0; g0 < q1; g0 += 64) {  // (wavefront-uniform trips; LDS ops of a wavefront complete in order)
        const int q = g0 + lane;
        const bool in = q < q1;
        const int x = in ? sid[q] : 0x1FF;  // (no expert id: bit 8 set)
        uint64_t same = __ballot(in);
        for (int b = 0; b < 9; ++b) {
            const bool bit = (x >> b) & 1;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const int before = __popcll(same & ((1ull << lane) - 1)), after = __popcll(same & ~((2ull << lane) - 1));
        if (in) {
            const int p = toff[x] * 16 + hist[wave][x] + before;
            prow[q] = p;
            rsrc[p] = q / k;
            if (after == 0) hist[wave][x] += before + 1;  // the group's last pair of x moves the place on
        }
    }
    for (int x = t; x < NE; x += NT)
        for (int i = toff[x]; i < toff[x + 1]; ++i) {
            items[2 * i] = x;
            items[2 * i + 1] = i;
        }
}
__global__ __launch_bounds__(1024) void k_moe_group(const int32_t* __restrict__ ids, int RK, int NE, int P, int k,
                                                    int32_t* __restrict__ prow, int32_t* __restrict__ rsrc,
                                                    int32_t* __restrict__ items, int32_t* __restrict__ count) {
    __shared__ GroupShared<16> sh;
    moe_group<false, 16>(sh, ids, RK, NE, P, k, prow, rsrc, items, count);
}

// The whole routing in one launch (router, top-k and grouping; the same arithmetic as k_router, k_moe_topk and
// k_moe_group): workgroup (row block b of RT_ROWS rows, expert block of 4 experts), 4 wavefronts (router_dot). The row
// block's workgroups are dealt to one XCD (grid x: the row blocks, padded to a multiple of the XCD count), so the last
// of them to count itself in the block's counter (XCD-local, in the L2 that holds the block's logits) routes the
// block's rows, a wavefront each (moe_topk_wave). It stores the rows' expert ids system-coherently and counts itself
// in a system-scope counter; the last row block to do so reads every id the same way and groups the pairs
// (moe_group). Counters return to zero. Counter layout: bits 0-7 the arrivals, 7 bits an XCD from bit 8 (the check
// that a block's workgroups shared one XCD).
template <int JM>
__global__ __launch_bounds__(256) void k_moe_route(const float* __restrict__ hn, const float* __restrict__ router, int R,
                                                   int E, int NE, int k, int P, float* __restrict__ lg,
                                                   int32_t* __restrict__ ids, float* __restrict__ w,
                                                   int32_t* __restrict__ prow, int32_t* __restrict__ rsrc,
                                                   int32_t* __restrict__ items, int32_t* __restrict__ count,
                                                   uint64_t* __restrict__ cnt, int32_t* __restrict__ gcnt,
                                                   int32_t* __restrict__ xerr) {
    __shared__ union {
        float part[4][4 * RT_ROWS][64];  // the router's quarter sums
        GroupShared<4> g;                // the grouping (the last row block, after its own rows are done)
    } u;
    __shared__ int s_last;
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nrb = (R + RT_ROWS - 1) / RT_ROWS, nxb = (int) gridDim.y;
    if (b >= nrb) return;  // a padding row block
    const int r0 = b * RT_ROWS;
    router_dot<JM>(hn, router, R, E, NE, lg, blockIdx.y * 4, r0, u.part);
    __builtin_amdgcn_s_waitcnt(0);  // the logits have reached the L2
    __syncthreads();
    uint64_t done = 0;  // (the completer's thread 0: the count, taken back with the ids' stores)
    if (t == 0) {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        const int f = 8 + 7 * (int) (xcc & 7);
        const uint64_t add = 1ull + (1ull << f);
        const uint64_t n = __hip_atomic_fetch_add(cnt + b * CNT_STRIDE, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
        s_last = (int) (n & 255) == nxb;
        if (s_last) {
            if ((int) ((n >> f) & 127) != nxb) __hip_atomic_fetch_or(xerr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            done = n;
        }
    }
    __syncthreads();
    if (!s_last) return;
    l1_drop();
    // row r0 + wave, its logits through the XCD's L2 (L1 lines dropped), its ids stored system-coherently (the last
    // row block reads them from another XCD)
    if (r0 + wave < R) {
        const int r = r0 + wave;
        const __amdgpu_buffer_rsrc_t rl = buf_rsrc(lg, (uint32_t) ((size_t) R * NE * 4));
        float l4[4];
        for (int s = 0; s < 4; ++s)
            l4[s] = lane + 64 * s < NE ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                    rl, (r * NE + lane + 64 * s) * 4, 0, 1))
                                       : -INFINITY;
        moe_topk_wave<true>(l4, NE, k, ids + (size_t) r * k, w + (size_t) r * k);
    }
    // the block's counter back to zero by an atomic of the same kind, where the counts were (every count of the
    // block has been made); it lands with the ids' stores
    if (t == 0) __hip_atomic_fetch_add(cnt + b * CNT_STRIDE, (uint64_t) 0 - done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        const int n = __hip_atomic_fetch_add(gcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        s_last = n == nrb - 1;
    }
    __syncthreads();
    if (!s_last) return;
    moe_group<true, 4>(u.g, ids, R * k, NE, P, k, prow, rsrc, items, count);
    if (t == 0) __hip_atomic_store(gcnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);  // (no barrier waits for it)
}

void moe_router(const float* hn, const float* router, int R, int E, int NE, float* lg, hipStream_t st) {
    if (R <= 0) return;
    const dim3 g((NE + 3) / 4, (R + RT_ROWS - 1) / RT_ROWS);
    switch (router_jm(E)) {
        case 4: hipLaunchKernelGGL(k_router<4>, g, dim3(256), 0, st, hn, router, R, E, NE, lg); break;
        case 8: hipLaunchKernelGGL(k_router<8>, g, dim3(256), 0, st, hn, router, R, E, NE, lg); break;
        case 16: hipLaunchKernelGGL(k_router<16>, g, dim3(256), 0, st, hn, router, R, E, NE, lg); break;
        default: hipLaunchKernelGGL(k_router_any, g, dim3(256), 0, st, hn, router, R, E, NE, lg);
    }
}
int moe_route(const float* hn, const float* router, int R, int E, int NE, int k, int P, float* lg, int32_t* ids,
              float* w, int32_t* prow, int32_t* rsrc, int32_t* items, int32_t* count, uint64_t* cnt, int cnt_len,
              int32_t* gcnt, int32_t* xerr, int nxcd, hipStream_t st) {
    if (R <= 0) return 0;
    if (NE < 1 || NE > 256 || k < 1 || k > MOE_MAX_K || k > NE || R * k > MOE_MAX_PAIRS || E % 4 || nxcd < 1 ||
        !router_jm(E))
        return -1;
    if (P < 16 * (std::min(NE, R * k) + (R * k + 15) / 16)) return -1;
    const int nrb = (R + RT_ROWS - 1) / RT_ROWS, gx = (nrb + nxcd - 1) / nxcd * nxcd;
    if ((long) gx * CNT_STRIDE > cnt_len || (NE + 3) / 4 > 127) return -1;
    const dim3 g(gx, (NE + 3) / 4);
#define ROUTE(JM)                                                                                                     \
    hipLaunchKernelGGL(k_moe_route<JM>, g, dim3(256), 0, st, hn, router, R, E, NE, k, P, lg, ids, w, prow, rsrc,    \
                       items, count, cnt, gcnt, xerr)
    switch (router_jm(E)) {
        case 4: ROUTE(4); break;
        case 8: ROUTE(8); break;
        default: ROUTE(16); break;
    }
#undef ROUTE
    return 0;
}

int moe_select(const float* lg, int R, int NE, int k, int P, int32_t* ids, float* w, int32_t* prow, int32_t* rsrc,
               int32_t* items, int32_t* count, hipStream_t st) {
    if (R <= 0) return 0;
    if (NE < 1 || NE > 256 || k < 1 || k > MOE_MAX_K || k > NE || R * k > MOE_MAX_PAIRS) return -1;
    if (P < 16 * (std::min(NE, R * k) + (R * k + 15) / 16)) return -1;  // the tiles of any grouping
    hipLaunchKernelGGL(k_moe_topk, dim3((R + 3) / 4), dim3(256), 0, st, lg, R, NE, k, ids, w);
    hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), 0, st, ids, R * k, NE, P, k, prow, rsrc, items, count);
    return 0;
}
