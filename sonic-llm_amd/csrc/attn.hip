// Paged-KV GQA decode/verify attention for gfx950 (head_dim 128).
//
// Replaces the reference's attn_part + attn_merge (kernels.metal:1122-1192, dispatched by qwen_attn_write,
// sn_attn.inc.h:176-192) and the verify rows' fa2/fa2r (kernels.metal:2674-2770): softmax(q.K^T * scale).V over each
// row's cells 0..pos, in fixed chunks of cells whose (acc, m, l) partials are merged in chunk order.
//
// A workgroup (4 wavefronts) takes one (query group, KV head, 256-cell chunk); wavefront w takes 64 of the cells.
// The G query heads of the KV head for each of the group's rows make up to 16 MFMA columns, so the K and V of a cell
// are read once for all of them:
//   S^T = K . Q^T : v_mfma_f32_16x16x32_f16, A = 16 cells x 32 dims of fp16 K, B = the queries in fp16 hi + lo
//                   (q*scale = hi + lo to 2^-22), so the scores are fp32-accurate;
//   O   = P . V   : A = 16 queries x 32 cells of p in fp16 hi + lo, B = 32 cells x 16 dims of fp16 V.
// Scores of cells past a row's position are -inf and their p exactly 0, so a row's result does not depend on the
// other rows of its group, and a verify row equals the same row run alone.
#include <algorithm>
#include <map>
#include <type_traits>

#include "sn_kernels_internal.h"

#define ATT_D 128

// x = hi + lo in fp16 (to 2^-22 relative): slot j of the two fragments
__device__ __forceinline__ void split_hl(float x, half8& hi, half8& lo, int j) {
    const _Float16 h = (_Float16) x;
    hi[j] = h;
    lo[j] = (_Float16) (x - (float) h);
}

__device__ __forceinline__ uint32_t pick_half(uint32_t w_lo_cell, uint32_t w_hi_cell, int odd) {
    // the fp16 at half `odd` of two words (cells j, j+1) packed as (cell j, cell j+1)
    return __builtin_amdgcn_perm(w_hi_cell, w_lo_cell, odd ? 0x07060302u : 0x05040100u);
}

// ---- the steps of one wavefront's 64 cells (shared by both kernels, so a chunk's arithmetic is the same in each)

// Q^T fragments of step row `row` (an unused column passes a valid row and qvalid false)
__device__ __forceinline__ void attn_qfrag_row(const AttnArgs& a, int row, int qhead, bool qvalid, int g,
                                               half8 (&qh)[4], half8 (&ql)[4]) {
    const float* qp = a.q + (size_t) row * a.ldq + (size_t) qhead * ATT_D;
    for (int t = 0; t < 4; ++t) {
        const float4 x0 = *(const float4*) (qp + 32 * t + 8 * g), x1 = *(const float4*) (qp + 32 * t + 8 * g + 4);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        for (int j = 0; j < 8; ++j) split_hl(qvalid ? xs[j] * a.scale : 0.0f, qh[t], ql[t], j);
    }
}

// Q^T fragments: MFMA t covers dims 32t .. 32t+31; lane (n, g) holds dims 32t + 8g .. +7 of query n. Loaded as
// 16-byte pieces from a valid row (an unused column reads the group's first row) and zeroed by a select, so no load
// sits behind a branch.
__device__ __forceinline__ void attn_qfrag(const AttnArgs& a, const AttnGroup& gr, int qrow, int qhead, bool qvalid,
                                           int g, half8 (&qh)[4], half8 (&ql)[4]) {
    attn_qfrag_row(a, gr.row0 + (qvalid ? qrow : 0), qhead, qvalid, g, qh, ql);
}

// The page ids of a wavefront's 64 cells from cbase: one page (64-cell pages) or two (32-cell pages). Cells past the
// group's last position read the first page (memory that exists; the cells are zeroed later).
__device__ __forceinline__ void attn_pages(const AttnArgs& a, const int32_t* ptrow, int cbase, int pos_last, int& p_lo,
                                           int& p_hi) {
    // (both entries are read unconditionally, from an index clamped to the last cell's page: no branch)
    const int sh = a.page_cells == 64 ? 6 : 5;  // page_cells is 32 or 64
    const int last = max(pos_last, 0) >> sh;
    const int e_lo = ptrow[min(cbase >> sh, last)], e_hi = ptrow[min((cbase + 32) >> sh, last)];
    p_lo = cbase <= pos_last ? e_lo : 0;
    p_hi = cbase + 32 <= pos_last ? e_hi : p_lo;
}

// Every K and V load of the wavefront's 64 cells (32 KB), issued together as buffer loads: kf[jg][t] = cell cbase + 16 jg
// + n, dims 32t + 8g .. +7 (the A operand of S^T); vf[st][4 jj + v] = cell cbase + 32 st + 16 jj + 4 g + v, dims 8n ..
// 8n + 7. A cell past the group's last position gets an offset past its page's bytes, so it reads as zeros without a
// memory access (a masked cell's p is exactly 0, and 0 * V must not meet a NaN); with live false every load does.
#define ATT_OOB 0x40000000
struct AttnRsrc {
    __amdgpu_buffer_rsrc_t k0, k1, v0, v1;
};
__device__ __forceinline__ AttnRsrc attn_rsrc(const AttnArgs& a, int kvh, int p_lo, int p_hi, bool live) {
    const size_t head_stride = (size_t) a.page_cells * ATT_D;
    const uint32_t hb = live ? (uint32_t) head_stride * 2 : 0u;  // bytes of one (page, KV head) region
    AttnRsrc r;
    r.k0 = buf_rsrc(a.kpool + ((size_t) p_lo * a.KVH + kvh) * head_stride, hb);
    r.k1 = buf_rsrc(a.kpool + ((size_t) p_hi * a.KVH + kvh) * head_stride, hb);
    r.v0 = buf_rsrc(a.vpool + ((size_t) p_lo * a.KVH + kvh) * head_stride, hb);
    r.v1 = buf_rsrc(a.vpool + ((size_t) p_hi * a.KVH + kvh) * head_stride, hb);
    return r;
}
template <int CPOL = 2>  // the loads' cache policy: nt (cells read once a step), 0 for run items (cells read again)
__device__ __forceinline__ void attn_issue_k(const AttnArgs& a, const AttnRsrc& r, int cbase, int pos_last, int n,
                                             int g, u32x4 (&kf)[4][4]) {
    // (dims 32 t + 8 g .. +7 are chunk 4 t + g of the cell: 16 g pc bytes into the region for the lane, 64 t pc for
    // the instruction)
    const int pc = a.page_cells;  // 32 or 64
    for (int jg = 0; jg < 4; ++jg) {
        const int c = cbase + 16 * jg + n;
        const int off = c <= pos_last ? (c & (pc - 1)) * 16 + 16 * pc * g : ATT_OOB;
        for (int t = 0; t < 4; ++t) kf[jg][t] = bload16nt<CPOL>(jg < 2 ? r.k0 : r.k1, off, 64 * pc * t);
    }
}
template <int CPOL = 2>
__device__ __forceinline__ void attn_issue_v(const AttnArgs& a, const AttnRsrc& r, int cbase, int pos_last, int n,
                                             int g, u32x4 (&vf)[2][8]) {
    const int pc = a.page_cells;
    for (int st = 0; st < 2; ++st)
        for (int jj = 0; jj < 2; ++jj)
            for (int v = 0; v < 4; ++v) {
                const int c = cbase + 32 * st + 16 * jj + 4 * g + v;
                const int off = c <= pos_last ? (c & (pc - 1)) * (ATT_D * 2) + 16 * n : ATT_OOB;
                vf[st][4 * jj + v] = bload16nt<CPOL>(st == 0 ? r.v0 : r.v1, off, 0);
            }
}
__device__ __forceinline__ void attn_issue(const AttnArgs& a, int kvh, int cbase, int pos_last, int p_lo, int p_hi,
                                           bool live, int n, int g, u32x4 (&kf)[4][4], u32x4 (&vf)[2][8]) {
    const AttnRsrc r = attn_rsrc(a, kvh, p_lo, p_hi, live);
    attn_issue_k(a, r, cbase, pos_last, n, g, kf);
    attn_issue_v(a, r, cbase, pos_last, n, g, vf);
}

// The wavefront's softmax partial over its 64 cells (the cells past the group's last position read as zeros): scores
// S^T = K . Q^T; per query the max m and sum l of exp(s - m) (lanes n, n+16, n+32, n+48 share query n); O = P . V, MFMA
// t covering output dims {8 c + t : c = 0..15}. full (wavefront-uniform): every one of the 64 cells lies at or below
// every valid query's position, so no score is masked and the masking is skipped (the same values; a column without
// a query then holds finite garbage that no one reads).
__device__ __forceinline__ void attn_scores(const u32x4 (&kf)[4][4], const half8 (&qh)[4], const half8 (&ql)[4],
                                            int cbase, bool qvalid, int qpos, int g, float& m, float& l,
                                            floatx4 (&s)[4], bool full) {
    for (int jg = 0; jg < 4; ++jg) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int t = 0; t < 4; ++t) {
            const half8 kh = __builtin_bit_cast(half8, kf[jg][t]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[t], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[t], acc, 0, 0, 0);
        }
        s[jg] = acc;  // lane (n, g): cells cbase + 16 jg + 4 g + v, query n
    }
    m = -INFINITY;
    if (full) {
        for (int jg = 0; jg < 4; ++jg)
            for (int v = 0; v < 4; ++v) m = fmaxf(m, s[jg][v]);
    } else {
        for (int jg = 0; jg < 4; ++jg)
            for (int v = 0; v < 4; ++v) {
                const int c = cbase + 16 * jg + 4 * g + v;
                const bool ok = qvalid && c <= qpos;
                s[jg][v] = ok ? s[jg][v] : -INFINITY;
                m = fmaxf(m, s[jg][v]);
            }
    }
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    l = 0.0f;
    if (full) {  // (m is finite)
        for (int jg = 0; jg < 4; ++jg)
            for (int v = 0; v < 4; ++v) {
                const float p = __expf(s[jg][v] - m);
                s[jg][v] = p;
                l += p;
            }
    } else {
        for (int jg = 0; jg < 4; ++jg)
            for (int v = 0; v < 4; ++v) {
                const float p = m == -INFINITY ? 0.0f : __expf(s[jg][v] - m);
                s[jg][v] = p;
                l += p;
            }
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
}
__device__ __forceinline__ void attn_pv(const u32x4 (&vf)[2][8], const floatx4 (&s)[4], floatx4 (&o)[8]) {
    for (int t = 0; t < 8; ++t) o[t] = (floatx4){0.f, 0.f, 0.f, 0.f};
    for (int st = 0; st < 2; ++st) {
        // P fragment: k slot 4 jj + v <-> cell cbase + 32 st + 16 jj + 4 g + v
        half8 ph, pl;
        for (int jj = 0; jj < 2; ++jj)
            for (int v = 0; v < 4; ++v) split_hl(s[2 * st + jj][v], ph, pl, 4 * jj + v);
        for (int t = 0; t < 8; ++t) {
            u32x4 bw;
            for (int i = 0; i < 4; ++i) bw[i] = pick_half(vf[st][2 * i][t >> 1], vf[st][2 * i + 1][t >> 1], t & 1);
            const half8 vb = __builtin_bit_cast(half8, bw);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, o[t], 0, 0, 0);
        }
    }
}

__device__ __forceinline__ void attn_wave(const u32x4 (&kf)[4][4], const u32x4 (&vf)[2][8], const half8 (&qh)[4],
                                          const half8 (&ql)[4], int cbase, bool qvalid, int qpos, int g, float& m,
                                          float& l, floatx4 (&o)[8], bool full) {
    floatx4 s[4];
    attn_scores(kf, qh, ql, cbase, qvalid, qpos, g, m, l, s, full);
    attn_pv(vf, s, o);
}

struct AttnShared {
    __attribute__((aligned(16))) float o[4][16][ATT_D + 4];  // (rows of 528 bytes: 16-byte pieces stay aligned)
    float m[4][16], l[4][16];
};

// The 4 wavefronts' partials combined in wavefront order into the chunk's partial of thread (query qq, dims d0 ..
// d0 + 7): M = the max, L = the rescaled sum, acc = the rescaled outputs. Only the group's nq = rows x G queries are
// exchanged (lane part g holds queries 4g .. 4g + 3; a decode row's G = 4 queries are lane part 0's): each lane writes
// its 8 dims of a query as two 16-byte pieces, each thread reads its query's 8 dims of each wavefront the same way.
// The threads of queries past nq read LDS nobody wrote this round and compute values nobody stores. Ends with the
// workgroup's LDS reads done only when the caller syncs again.
__device__ __forceinline__ void attn_combine(AttnShared& sh, int wave, int n, int g, int nq, float m, float l,
                                             const floatx4 (&o)[8], int qq, int d0, float& M, float& L,
                                             float (&acc)[8]) {
    if (g == 0) {
        sh.m[wave][n] = m;
        sh.l[wave][n] = l;
    }
    if (4 * g < nq)
        for (int v = 0; v < 4; ++v) {
            float* row = &sh.o[wave][4 * g + v][8 * n];
            *(float4*) row = (float4){o[0][v], o[1][v], o[2][v], o[3][v]};
            *(float4*) (row + 4) = (float4){o[4][v], o[5][v], o[6][v], o[7][v]};
        }
    __syncthreads();
    M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sh.m[w][qq]);
    float e[4];
    L = 0.0f;
    for (int w = 0; w < 4; ++w) {
        e[w] = sh.m[w][qq] == -INFINITY ? 0.0f : __expf(sh.m[w][qq] - M);
        L += sh.l[w][qq] * e[w];
    }
    float ow[4][8];
    for (int w = 0; w < 4; ++w) {
        const float4 a = *(const float4*) &sh.o[w][qq][d0], b = *(const float4*) &sh.o[w][qq][d0 + 4];
        ow[w][0] = a.x, ow[w][1] = a.y, ow[w][2] = a.z, ow[w][3] = a.w;
        ow[w][4] = b.x, ow[w][5] = b.y, ow[w][6] = b.z, ow[w][7] = b.w;
    }
    for (int d = 0; d < 8; ++d) {
        float s = 0.0f;
        for (int w = 0; w < 4; ++w) s += ow[w][d] * e[w];
        acc[d] = s;
    }
}

// Chunk partials folded in chunk order into a row's running (M, L, o) (nd dims): the one arithmetic both the merge and
// the whole-context kernel use, contraction off so both round alike. A chunk with no cell for the row (mc = -inf) is
// skipped.
template <int ND>
__device__ __forceinline__ void attn_fold(float& M, float& L, float (&o)[ND], float mc, float lc, const float (&ov)[ND]) {
#pragma clang fp contract(off)
    if (mc == -INFINITY) return;
    const float mn = fmaxf(M, mc);
    const float e0 = M == -INFINITY ? 0.0f : __expf(M - mn), e1 = __expf(mc - mn);
    for (int d = 0; d < ND; ++d) o[d] = o[d] * e0 + ov[d] * e1;
    L = L * e0 + lc * e1;
    M = mn;
}

// A row's normalised output dims (nd of them, fold done): o / L
template <int ND>
__device__ __forceinline__ void attn_finish(float L, float (&o)[ND]) {
    const float il = L > 0.0f ? 1.0f / L : 0.0f;
    for (int d = 0; d < ND; ++d) o[d] *= il;
}

// the group of a shared item's member m (0: the item's own group; -1: none), by selects (m may differ per lane)
__device__ __forceinline__ int attn_member(const AttnItem& it, int m) {
    static_assert(ATT_SHARE_MAX == 4, "three shared members after the item's own group");
    return m == 0 ? it.group : m == 1 ? it.share[0] : m == 2 ? it.share[1] : m == 3 ? it.share[2] : -1;
}

// One work item = (query group, chunk), or a shared chunk of up to ATT_SHARE_MAX one-row groups; grid.y = KV head.
// Writes the chunk's partial (acc[128], m, l) of every query of the item's rows; k_attn_merge folds them. A query's
// partial depends on its own column only, so it is the same whichever item computes it.
// (every thread of the workgroup reaches the end)
__device__ __forceinline__ void attn_part_item(const AttnArgs& a, const AttnItem it, const int kvh, AttnShared& sh) {
    const AttnGroup gr = it.g;
    const int G = a.H / a.KVH;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const bool shared = it.share[0] >= 0;  // (uniform)
    int nshare = 1;
    if (shared)
        while (nshare < ATT_SHARE_MAX && nshare * G < 16 && attn_member(it, nshare) >= 0) ++nshare;
    // the pages and the cells' bound come from the item's own group (a shared chunk lies wholly below every member's
    // position, on the same pages)
    const int pos_last = gr.pos0 + gr.nrows - 1;
    const int cbase = it.chunk * ATT_CHUNK + 64 * wave;  // this wavefront's first cell
    // this lane's query (as a B column of S^T and the A row of O): n = row * G + head-in-group, the row being a row of
    // the item's group, or (shared) the one row of member n / G
    const int qhead = kvh * G + n % G;
    int qstep, qpos;  // the query's step row and position
    bool qvalid;
    if (shared) {
        const int mq = n / G;
        const AttnGroup& gm = a.groups[attn_member(it, min(mq, nshare - 1))];
        qstep = gm.row0;
        qpos = gm.pos0;
        qvalid = mq < nshare;
    } else {
        const int qrow = n / G;
        qvalid = qrow < gr.nrows;
        qstep = gr.row0 + (qvalid ? qrow : 0);
        qpos = gr.pos0 + qrow;
    }
    int p_lo, p_hi;
    attn_pages(a, a.pt + (size_t) gr.seq * a.max_pages, cbase, pos_last, p_lo, p_hi);
    u32x4 kf[4][4], vf[2][8];
    attn_issue(a, kvh, cbase, pos_last, p_lo, p_hi, true, n, g, kf, vf);
    half8 qh[4], ql[4];
    attn_qfrag_row(a, qstep, qhead, qvalid, g, qh, ql);
    // (a shared chunk lies wholly below every member's position; otherwise the group's first row is its lowest)
    const bool full = shared || cbase + 63 <= gr.pos0;
    float m, l;
    floatx4 o[8];
    attn_wave(kf, vf, qh, ql, cbase, qvalid, qpos, g, m, l, o, full);
    // thread -> (query qq, 8 dims)
    const int qq = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
    float M, L, acc[8];
    attn_combine(sh, wave, n, g, (shared ? nshare : gr.nrows) * G, m, l, o, qq, d0, M, L, acc);
    const int row = qq / G, head = kvh * G + qq % G;
    if (row < (shared ? nshare : gr.nrows)) {
        const int orow = shared ? a.groups[attn_member(it, row)].row0 : gr.row0 + row;
        float* dst = a.part + (((size_t) orow * a.H + head) * a.max_chunks + it.chunk) * (ATT_D + 2);
        *(float2*) (dst + d0) = (float2){acc[0], acc[1]};  // (a partial is 130 floats: 8-byte aligned)
        *(float2*) (dst + d0 + 2) = (float2){acc[2], acc[3]};
        *(float2*) (dst + d0 + 4) = (float2){acc[4], acc[5]};
        *(float2*) (dst + d0 + 6) = (float2){acc[6], acc[7]};
        if ((threadIdx.x & 15) == 0) *(float2*) (dst + ATT_D) = (float2){M, L};
    }
}
// grid (KV head, item): see attention_items
// The launches' hot arguments come first as scalars, which the hardware preloads into SGPRs at wavefront start
// (-amdgpu-kernarg-preload-count): the item, group, page-table and cell loads are issued without waiting for the
// argument block; the rest of AttnArgs is read from it as before.
#define AP_ARGS(a) (a).items, (a).groups, (a).pt, (a).kpool, (a).vpool, (a).q, (a).H, (a).KVH, (a).page_cells, (a).max_pages, (a)
#define AM_ARGS(a) (a).mrows, (a).row_pos, (a).part, (a).out, (a).xa, (a).H, (a).KVH, (a).max_chunks, (a).ldo, (a)
__global__ __launch_bounds__(256) void k_attn_part(const AttnItem* items_, const AttnGroup* groups_, const int32_t* pt_,
                                                   const uint16_t* kpool_, const uint16_t* vpool_, const float* q_,
                                                   int H_, int KVH_, int page_cells_, int max_pages_, AttnArgs a) {
    a.items = items_, a.groups = groups_, a.pt = pt_, a.kpool = kpool_, a.vpool = vpool_, a.q = q_;
    a.H = H_, a.KVH = KVH_, a.page_cells = page_cells_, a.max_pages = max_pages_;
    __shared__ AttnShared sh;
    attn_part_item(a, a.items[blockIdx.y], blockIdx.x, sh);
}

// The Q8_0 operand of the o-projection from a row's normalised outputs (ggml x86 quantize_row_q8_0, exactly as the
// activation quantizer): this lane's 8 dims e0 .. e0 + 7 (e0 = 8 i, i = 0..3) of block blk, whose 4 lanes are xor
// neighbours 1 and 2; written in the operand's fragment order (q / 16 for elements 16..31) with the block's scale and
// corrections from the block's first lane.
__device__ __forceinline__ void attn_xa8(uint8_t* xa, int K, int r, int blk, int e0, const float (&o)[8]) {
    float amax = 0.0f;
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(o[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float d = amax / 127.f;
    const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    const bool hi = e0 >= 16;
    const float sc = hi ? 0.0625f : 1.0f;
    float q[8], sq = 0.0f;
    for (int j = 0; j < 8; ++j) {
        q[j] = __builtin_rintf(o[j] * id);
        sq += q[j];
    }
    uint8_t* rec = xa + xa_rec_off(K, r, blk);
    const int gg = (e0 & 15) / 4;  // elements e0 .. e0 + 3 at lane part gg, e0 + 4 .. e0 + 7 at gg + 1
    for (int h = 0; h < 2; ++h)
        *(half4v*) (rec + (blk & 3) * 1024 + 16 * ((r & 15) + 16 * (gg + h)) + (hi ? 8 : 0)) =
            (half4v){(_Float16) (q[4 * h] * sc), (_Float16) (q[4 * h + 1] * sc), (_Float16) (q[4 * h + 2] * sc),
                     (_Float16) (q[4 * h + 3] * sc)};
    float slo = hi ? 0.0f : sq, shi = hi ? sq : 0.0f;
    slo += __shfl_xor(slo, 1);
    shi += __shfl_xor(shi, 1);
    slo += __shfl_xor(slo, 2);
    shi += __shfl_xor(shi, 2);
    if (e0 == 0) {
        *(float*) (rec + XA_DX_OFF + (blk & 3) * 64 + 4 * (r & 15)) = (float) (_Float16) d;
        *(float*) (rec + XA_CORR_OFF + (blk & 3) * 64 + 4 * (r & 15)) = -(1032.0f * slo + 72.0f * shi);
        *(float*) (rec + XA_CORR8_OFF + (blk & 3) * 64 + 4 * (r & 15)) = -1152.0f * (slo + shi);
    }
}

// One work item = a whole query group (every chunk of its context); grid.y = KV head. 8 wavefronts: waves 0-3 take
// chunk c and waves 4-7 chunk c + 1 of each pair, each half combining its chunk's partial exactly as k_attn_part does;
// the first half's threads then fold the two partials in chunk order into their running (M, L, o) (query, 8 dims) as
// k_attn_merge would, and finally write the rows' outputs (and the o-projection's operand) themselves: no partials,
// no merge. A pair's second chunk past the context (odd chunk counts) reads nothing and has no cell.
struct AttnPairShared {
    AttnShared h[2];
    float x[257][10];  // the second half's combined partials: acc[8], M, L (row 256: the first half's dummy writes)
};
__global__ __launch_bounds__(512) void k_attn_whole(AttnArgs a) {
    __shared__ AttnPairShared sh;
    const AttnItem it = a.items[blockIdx.y];  // (grid: KV head, item)
    const AttnGroup gr = it.g;
    const int kvh = blockIdx.x;
    const int G = a.H / a.KVH;
    const int lane = threadIdx.x & 63, w8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = w8 >> 2, wave = w8 & 3, th = threadIdx.x & 255;
    const int n = lane & 15, g = lane >> 4;
    const int pos_last = gr.pos0 + gr.nrows - 1;
    const int qrow = n / G, qhead = kvh * G + n % G;
    const bool qvalid = qrow < gr.nrows;
    const int qpos = gr.pos0 + qrow;
    const int32_t* ptrow = a.pt + (size_t) gr.seq * a.max_pages;
    const int nch = it.nchunk;
    const int qq = th >> 4, d0 = (th & 15) * 8;
    float RM = -INFINITY, RL = 0.0f, RO[8];
    for (int d = 0; d < 8; ++d) RO[d] = 0.0f;
    // chunk c0 + half of each pair; the next pair's K loads go out as soon as the scores have used K, its V loads as
    // soon as P . V has used V, so they are in flight through the softmax, the combine and the fold. Past the context
    // (live false) the same loads read nothing, so the issue sequence has no branch.
    u32x4 kf[4][4], vf[2][8];
    auto rsrc_of = [&](int c0, int& cbase, int& plast) {
        const int c = c0 + half;
        const bool live = c < nch;
        cbase = (live ? c : 0) * ATT_CHUNK + 64 * wave;
        plast = live ? pos_last : -1;
        int p_lo, p_hi;
        attn_pages(a, ptrow, cbase, plast, p_lo, p_hi);
        return attn_rsrc(a, kvh, p_lo, p_hi, live);
    };
    int cb, pl;
    {
        const AttnRsrc r0 = rsrc_of(0, cb, pl);
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_k(a, r0, cb, pl, n, g, kf);  // K before V, as in the loop: the wait for K leaves V in flight
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_v(a, r0, cb, pl, n, g, vf);
        __builtin_amdgcn_sched_barrier(0);
    }
    half8 qh[4], ql[4];  // (loaded and split while the first pair's cells are in flight)
    attn_qfrag(a, gr, qrow, qhead, qvalid, g, qh, ql);
    for (int c0 = 0; c0 < nch; c0 += 2) {  // (uniform trips: every wavefront meets every barrier)
        const int c = c0 + half;
        const bool live = c < nch;
        const int cbase = c * ATT_CHUNK + 64 * wave;
        int ncb, npl;
        const AttnRsrc rn = rsrc_of(c0 + 2, ncb, npl);
        float m, l;
        floatx4 sc[4], o[8];
        __builtin_amdgcn_sched_barrier(0);
        attn_scores(kf, qh, ql, cbase, qvalid && live, qpos, g, m, l, sc, live && cbase + 63 <= gr.pos0);
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_k(a, rn, ncb, npl, n, g, kf);
        __builtin_amdgcn_sched_barrier(0);
        attn_pv(vf, sc, o);
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_v(a, rn, ncb, npl, n, g, vf);
        __builtin_amdgcn_sched_barrier(0);
        float M, L, acc[8];
        attn_combine(sh.h[half], wave, n, g, gr.nrows * G, m, l, o, qq, d0, M, L, acc);
        // (no branch on the half: the second half writes its partial and also folds, into a state never used)
        float* xw = sh.x[half ? th : 256];
        for (int d = 0; d < 8; ++d) xw[d] = acc[d];
        xw[8] = M;
        xw[9] = L;
        __syncthreads();
        attn_fold<8>(RM, RL, RO, M, L, acc);
        float acc1[8];
        for (int d = 0; d < 8; ++d) acc1[d] = sh.x[th][d];
        attn_fold<8>(RM, RL, RO, sh.x[th][8], sh.x[th][9], acc1);
        // (no barrier here: the next pair writes sh.h after every thread's combine reads, which precede the barrier
        // above, and sh.x after its combine's barrier, which every thread reaches only once its fold has read sh.x)
    }
    const int row = qq / G, head = kvh * G + qq % G;
    if (half != 0 || row >= gr.nrows) return;
    const int r = gr.row0 + row;
    attn_finish<8>(RL, RO);
    if (a.out) {
        float* out = a.out + (size_t) r * a.ldo + (size_t) head * ATT_D + d0;
        *(float4*) out = (float4){RO[0], RO[1], RO[2], RO[3]};
        *(float4*) (out + 4) = (float4){RO[4], RO[5], RO[6], RO[7]};
    }
    if (a.xa) attn_xa8(a.xa, a.H * ATT_D, r, head * 4 + d0 / 32, d0 & 31, RO);
}

// One work item = a run of nmem consecutive query groups of one sequence (prompt rows), every chunk of the last
// group's context; grid.y = KV head. The whole-group kernel's walk (waves 0-3 on chunk c, 4-7 on chunk c + 1 of each
// pair, each half combining its chunk's partial as k_attn_part does, the first half folding the two in chunk order),
// with the pair's K/V cells held in registers for every group of the run in turn: each group's queries (staged in LDS
// as hi + lo, as attn_qfrag_row splits them) take the MFMA columns, its rows' masks are its own, and its running
// (M, L, o) lives in LDS between pairs. A cell past a group's rows but within the run's has a real value where that
// group's own item would read zeros; its score is -inf and its p exactly 0 either way, so every group's output is the
// one its own whole-group or chunk items give, bit for bit. Outputs and the o-projection's operand are written here.
struct AttnRunShared {
    AttnShared h[2];
    float x[257][10];                 // the second half's combined partials (row 256: the first half's dummy writes)
    float st[ATT_RUN_MAX][10][256];   // each group's running o[8], M, L per first-half thread
    __attribute__((aligned(16))) _Float16 q[ATT_RUN_MAX][2][16][ATT_D + 8];  // each group's queries: hi, lo
};
__global__ __launch_bounds__(512) void k_attn_run(AttnArgs a) {
    __shared__ AttnRunShared sh;
    const AttnItem it = a.runs[blockIdx.y];  // (grid: KV head, run)
    const int kvh = blockIdx.x;
    const int G = a.H / a.KVH;
    const int lane = threadIdx.x & 63, w8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = w8 >> 2, wave = w8 & 3, th = threadIdx.x & 255;
    const int n = lane & 15, g = lane >> 4;
    const int nm = it.nmem;
    const AttnGroup glast = a.groups[it.group + nm - 1];
    const int pos_last = glast.pos0 + glast.nrows - 1;  // the run's last cell
    const int32_t* ptrow = a.pt + (size_t) glast.seq * a.max_pages;
    const int nch = it.nchunk;
    const int qq = th >> 4, d0 = (th & 15) * 8;
    {  // the groups' queries: thread t takes dims 4 (t % 32) .. + 3 of query column t / 32 of each group
        const int qn = threadIdx.x >> 5, dd = 4 * (threadIdx.x & 31);
        for (int m = 0; m < nm; ++m) {
            const AttnGroup gm = a.groups[it.group + m];
            const int row = qn / G;
            const bool ok = row < gm.nrows;
            const float4 v = *(const float4*) (a.q + (size_t) (gm.row0 + (ok ? row : 0)) * a.ldq +
                                               (size_t) (kvh * G + qn % G) * ATT_D + dd);
            const float xs[4] = {v.x, v.y, v.z, v.w};
            for (int j = 0; j < 4; ++j) {
                const float x = ok ? xs[j] * a.scale : 0.0f;
                const _Float16 h = (_Float16) x;
                sh.q[m][0][qn][dd + j] = h;
                sh.q[m][1][qn][dd + j] = (_Float16) (x - (float) h);
            }
        }
        if (half == 0)
            for (int m = 0; m < ATT_RUN_MAX; ++m) {
                for (int d = 0; d < 8; ++d) sh.st[m][d][th] = 0.0f;
                sh.st[m][8][th] = -INFINITY;
                sh.st[m][9][th] = 0.0f;
            }
    }
    __syncthreads();
    u32x4 kf[4][4], vf[2][8];
    auto rsrc_of = [&](int c0, int& cbase, int& plast) {
        const int c = c0 + half;
        const bool live = c < nch;
        cbase = (live ? c : 0) * ATT_CHUNK + 64 * wave;
        plast = live ? pos_last : -1;
        int p_lo, p_hi;
        attn_pages(a, ptrow, cbase, plast, p_lo, p_hi);
        return attn_rsrc(a, kvh, p_lo, p_hi, live);
    };
    int cb, pl;
    {
        const AttnRsrc r0 = rsrc_of(0, cb, pl);
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_k<0>(a, r0, cb, pl, n, g, kf);
        __builtin_amdgcn_sched_barrier(0);
        attn_issue_v<0>(a, r0, cb, pl, n, g, vf);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int c0 = 0; c0 < nch; c0 += 2) {  // (uniform trips: every wavefront meets every barrier)
        const int c = c0 + half;
        const bool live = c < nch;
        const int cbase = c * ATT_CHUNK + 64 * wave;
        int ncb, npl;
        const AttnRsrc rn = rsrc_of(c0 + 2, ncb, npl);
        // group m of the run on this pair; the last one issues the next pair's loads (K once its scores have used K,
        // V once P . V has used V), so they are in flight through its softmax, combine and fold
        auto member = [&](int m, auto last) {
            const AttnGroup gm = a.groups[it.group + m];
            half8 qh[4], ql[4];
            for (int t = 0; t < 4; ++t) {
                qh[t] = *(const half8*) &sh.q[m][0][n][32 * t + 8 * g];
                ql[t] = *(const half8*) &sh.q[m][1][n][32 * t + 8 * g];
            }
            const int qrow = n / G;
            const bool qvalid = qrow < gm.nrows;
            float ml, ll;
            floatx4 sc[4], o[8];
            __builtin_amdgcn_sched_barrier(0);
            attn_scores(kf, qh, ql, cbase, qvalid && live, gm.pos0 + qrow, g, ml, ll, sc, live && cbase + 63 <= gm.pos0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(last)::value) attn_issue_k<0>(a, rn, ncb, npl, n, g, kf);
            __builtin_amdgcn_sched_barrier(0);
            attn_pv(vf, sc, o);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(last)::value) attn_issue_v<0>(a, rn, ncb, npl, n, g, vf);
            __builtin_amdgcn_sched_barrier(0);
            float M, L, acc[8];
            attn_combine(sh.h[half], wave, n, g, gm.nrows * G, ml, ll, o, qq, d0, M, L, acc);
            float* xw = sh.x[half ? th : 256];
            for (int d = 0; d < 8; ++d) xw[d] = acc[d];
            xw[8] = M;
            xw[9] = L;
            __syncthreads();
            // (the second half folds a copy it never stores)
            float RM = sh.st[m][8][th], RL = sh.st[m][9][th], RO[8];
            for (int d = 0; d < 8; ++d) RO[d] = sh.st[m][d][th];
            attn_fold<8>(RM, RL, RO, M, L, acc);
            float acc1[8];
            for (int d = 0; d < 8; ++d) acc1[d] = sh.x[th][d];
            attn_fold<8>(RM, RL, RO, sh.x[th][8], sh.x[th][9], acc1);
            if (half == 0) {  // (a thread's own slots: no barrier needed for them)
                for (int d = 0; d < 8; ++d) sh.st[m][d][th] = RO[d];
                sh.st[m][8][th] = RM;
                sh.st[m][9][th] = RL;
            }
            // (no barrier here: the next group writes sh.h after every thread's combine reads, which precede the
            // barrier above, and sh.x after its combine's barrier, which every thread reaches only once its fold has
            // read sh.x)
        };
        for (int m = 0; m + 1 < nm; ++m) member(m, std::false_type{});
        member(nm - 1, std::true_type{});
    }
    if (half != 0) return;
    const int row = qq / G, head = kvh * G + qq % G;
    for (int m = 0; m < nm; ++m) {
        const AttnGroup gm = a.groups[it.group + m];
        if (row >= gm.nrows) continue;  // (a block's 4 lanes share the row: attn_xa8's shuffles stay within them)
        float RL = sh.st[m][9][th], RO[8];
        for (int d = 0; d < 8; ++d) RO[d] = sh.st[m][d][th];
        attn_finish<8>(RL, RO);
        const int r = gm.row0 + row;
        if (a.out) {
            float* out = a.out + (size_t) r * a.ldo + (size_t) head * ATT_D + d0;
            *(float4*) out = (float4){RO[0], RO[1], RO[2], RO[3]};
            *(float4*) (out + 4) = (float4){RO[4], RO[5], RO[6], RO[7]};
        }
        if (a.xa) attn_xa8(a.xa, a.H * ATT_D, r, head * 4 + d0 / 32, d0 & 31, RO);
    }
}

// per (row, head) of the rows the partial kernel split (a.mrows): the chunks' partials folded in chunk order (attn_fold);
// out = acc / l. One wavefront, 2 dims a lane; the loads of 8 chunks are issued together (chunk index clamped, no load
// behind a branch), then folded in order. With a.xa the head's 128 outputs (4 Q8_0 blocks of the o-projection's input
// row) are also quantized there, exactly as the activation quantizer does (ggml x86 quantize_row_q8_0), into the xa
// operand of K = H * 128.
#define MERGE_BATCH 16  // chunk partials a lane loads before folding them (the fold's completers)
// row r, head h by one wavefront (lane: dims 2 lane, 2 lane + 1). L2: the partials were stored in this launch by other
// workgroups of this XCD (the caller has dropped its L1 lines: the loads read the XCD's L2)
template <bool L2, int MB = MERGE_BATCH>
__device__ __forceinline__ void attn_merge_one(const AttnArgs& a, const int r, const int h, const int lane) {
    // the chunk count (the row's position) is loaded beside the first round's partials: their addresses are clamped
    // to the (row, head)'s max_chunks slots, not to its chunks, so no load waits for it (slots past the row's chunks
    // are loaded and not folded); the loads are buffer loads, all issued before any is folded (as plain loads, the
    // uniform (m, l) pairs became scalar loads, each waited for in the fold)
    const int rp = (int) __builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(a.row_pos + r, 4), 0, 0, 0);
    const float* p0 = a.part + ((size_t) r * a.H + h) * a.max_chunks * (ATT_D + 2);
    // (L2: a resource over the row's partials; offsets below 2^31 bytes)
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(p0, (uint32_t) (a.max_chunks * (ATT_D + 2) * 4));
    float M = -INFINITY, L = 0.0f, o[2] = {0.0f, 0.0f};
    float2 ov[MB], ml[MB];
    auto load = [&](int c0) {
        for (int j = 0; j < MB; ++j) {
            const int pc = min(c0 + j, a.max_chunks - 1) * (ATT_D + 2);
            ov[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(pr, (pc + 2 * lane) * 4, 0, L2 ? 1 : 0));
            ml[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(pr, (pc + ATT_D) * 4, 0, L2 ? 1 : 0));
        }
    };
    auto fold = [&](int c0, int nc) {
#pragma unroll
        for (int j = 0; j < MB; ++j) {  // (a fixed trip count keeps ov and ml in registers)
            if (c0 + j >= nc) continue;  // past the row's chunks
            const float v2[2] = {ov[j].x, ov[j].y};
            attn_fold<2>(M, L, o, ml[j].x, ml[j].y, v2);
        }
    };
    int rpv = rp;
    load(0);
    asm volatile("" : "+v"(rpv));  // (rpv stays where the load put it until the first round's loads are issued)
    const int nc = rpv / ATT_CHUNK + 1;
    fold(0, nc);
    for (int c0 = MB; c0 < nc; c0 += MB) {  // (contexts up to 4096 cells: one round of loads)
        load(c0);
        fold(c0, nc);
    }
    attn_finish<2>(L, o);
    const float o0 = o[0], o1 = o[1];
    if (a.out) {
        float* out = a.out + (size_t) r * a.ldo + (size_t) h * ATT_D;
        out[2 * lane] = o0;
        out[2 * lane + 1] = o1;
    }
    if (a.xa) {
        // block b = lane / 16 holds dims 32 b + 2 (lane % 16) and + 1: elements e, e + 1 of block 4 h + b, stored in
        // the operand's fragment order (q / 16 for elements 16..31), with the block's scale and corrections
        float amax = fmaxf(fabsf(o0), fabsf(o1));
        for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        const int b = lane >> 4, e = 2 * (lane & 15);
        const bool hi = e >= 16;
        const int gg = (hi ? e - 16 : e) / 4, j = (hi ? 4 : 0) + e % 4;
        const int K = a.H * ATT_D, blk = h * 4 + b;
        const float q0 = __builtin_rintf(o0 * id), q1 = __builtin_rintf(o1 * id);
        const float sc = hi ? 0.0625f : 1.0f;
        uint8_t* rec = a.xa + xa_rec_off(K, r, blk);
        *(half2v*) (rec + b * 1024 + 16 * ((r & 15) + 16 * gg) + 2 * j) = (half2v){(_Float16) (q0 * sc), (_Float16) (q1 * sc)};
        float slo = hi ? 0.0f : q0 + q1, shi = hi ? q0 + q1 : 0.0f;
        for (int off = 1; off < 16; off <<= 1) {
            slo += __shfl_xor(slo, off);
            shi += __shfl_xor(shi, off);
        }
        if ((lane & 15) == 0) {
            *(float*) (rec + XA_DX_OFF + b * 64 + 4 * (r & 15)) = (float) (_Float16) d;
            *(float*) (rec + XA_CORR_OFF + b * 64 + 4 * (r & 15)) = -(1032.0f * slo + 72.0f * shi);
            *(float*) (rec + XA_CORR8_OFF + b * 64 + 4 * (r & 15)) = -1152.0f * (slo + shi);
        }
    }
}
// XA (KV head count a multiple of 8): a 1-D grid whose workgroup L, dealt to XCD L mod 8, takes a (row, head) of a KV
// head k with k = L (mod 8): k_attn_part's grid (KV head fastest) dealt every item of KV head k to XCD k mod 8, so the
// merge reads its partials where they were written. Otherwise (row, head) = (blockIdx.x, blockIdx.y).
template <int MB, bool XA>
__global__ __launch_bounds__(64) void k_attn_merge(const int32_t* mrows_, const int32_t* row_pos_, float* part_,
                                                   float* out_, uint8_t* xa_, int H_, int KVH_, int max_chunks_,
                                                   int ldo_, AttnArgs a) {
    a.mrows = mrows_, a.row_pos = row_pos_, a.part = part_, a.out = out_, a.xa = xa_;
    a.H = H_, a.KVH = KVH_, a.max_chunks = max_chunks_, a.ldo = ldo_;
    int row = blockIdx.x, h = blockIdx.y;
    if constexpr (XA) {
        const int L = blockIdx.x, kx = L & 7, q = L >> 3, hx = a.H >> 3, G = a.H / a.KVH, t = q % hx;
        row = q / hx;
        h = ((t / G) * 8 + kx) * G + t % G;
    }
    attn_merge_one<false, MB>(a, a.mrows[row], h, threadIdx.x);
}

// The chunk items and their merge in one launch (plain chunk items: no shared chunks, runs or whole groups). Unit
// (group g, KV head h) owns the group's nc chunk workgroups. The 1-D grid keeps the two-launch order (KV head, then
// group, then chunk: measured 62.4 against 58.8 us for chunk-major) with 8 groups interleaved, so that a unit's linear
// ids are equal modulo the XCD count nx: chunk c of (h, g) at nx ((h S + g / nx) NC + c) + g % nx (S = group slots a
// head, NC = the most chunks of a group), and the hardware's in-turn dealing puts a unit's workgroups on one XCD. Each
// stores its chunk's partials as k_attn_part does, then counts itself in the unit's 64-bit counter (bits 0-7 the
// count, 7 bits an XCD from bit 8: a unit found on two XCDs sets *xerr); the count's completer folds the unit's (row,
// head) pairs, a wavefront each, as k_attn_merge does, its loads through the XCD's L2, and takes the count back.
__global__ __launch_bounds__(256) void k_attn_fold(AttnArgs a) {
    __shared__ AttnShared sh;
    __shared__ int s_last;
    const int nx = a.nxcd, S = (a.n_groups + nx - 1) / nx, NC = a.fold_chunks;
    const int L = (int) blockIdx.x, q = L / nx, c = q % NC, t = q / NC;
    const int gi = (t % S) * nx + L % nx, kvh = t / S;
    if (gi >= a.n_groups) return;  // (a padding slot)
    const int u = gi * a.KVH + kvh;
    const AttnGroup gr = a.groups[gi];
    const int nc = (gr.pos0 + gr.nrows - 1) / ATT_CHUNK + 1;
    if (c >= nc) return;  // (past the group's chunks)
    const AttnItem it = {gi, c, 1, {-1, -1, -1}, 1, a.groups[gi]};
    attn_part_item(a, it, kvh, sh);
    __builtin_amdgcn_s_waitcnt(0);  // the partials have reached the L2
    __syncthreads();
    uint64_t* cnt = a.cnt + (size_t) u * CNT_STRIDE;
    uint64_t done = 0;
    if (threadIdx.x == 0) {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        const int f = 8 + 7 * (int) (xcc & 7);
        const uint64_t add = 1ull + (1ull << f);
        const uint64_t n = __hip_atomic_fetch_add(cnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
        s_last = (int) (n & 255) == nc;
        if (s_last) {
            if ((int) ((n >> f) & 127) != nc) __hip_atomic_fetch_or(a.xerr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            done = n;
        }
    }
    __syncthreads();
    if (!s_last) return;
    l1_drop();
    const int G = a.H / a.KVH, wave = threadIdx.x >> 6;
    for (int p = wave; p < gr.nrows * G; p += 4) attn_merge_one<true>(a, gr.row0 + p / G, kvh * G + p % G, threadIdx.x & 63);
    if (threadIdx.x == 0) __hip_atomic_fetch_add(cnt, (uint64_t) 0 - done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int attention_runs(const AttnArgs& a, hipStream_t st) {
    if (a.n_runs <= 0) return 0;
    if (a.H % a.KVH != 0 || 16 % (a.H / a.KVH) != 0) return -1;
    hipLaunchKernelGGL(k_attn_run, dim3(a.KVH, a.n_runs), dim3(512), 0, st, a);
    return 0;
}
int attention_items(const AttnArgs& a, hipStream_t st) {
    if (a.n_items <= 0) return 0;
    if (a.H % a.KVH != 0 || 16 % (a.H / a.KVH) != 0) return -1;
    if (a.fold) {  // (the plan's chunk items in the fold's order, and their merge)
        if (a.whole || a.n_runs > 0 || !a.cnt || !a.xerr || a.nxcd < 1 || a.n_groups < 1 || a.fold_chunks < 1 ||
            a.fold_chunks > 127)
            return -1;
        const int S = (a.n_groups + a.nxcd - 1) / a.nxcd;
        hipLaunchKernelGGL(k_attn_fold, dim3(a.nxcd * S * a.KVH * a.fold_chunks), dim3(256), 0, st, a);
        return 0;
    }
    // The grid's x is the KV head: a launch deals its workgroups out by linear id, so the KV heads of one item (the
    // same cells of every head: adjacent blocks of each page) run together. Measured on MI355X against item-major
    // grids: configs[2]'s chunk items 55.2 -> 51.3 us a layer (with the item order of attn_plan), configs[1] 60.2 ->
    // 56.8 us; the run items (prompt rows) unchanged.
    if (a.whole) hipLaunchKernelGGL(k_attn_whole, dim3(a.KVH, a.n_items), dim3(512), 0, st, a);
    else hipLaunchKernelGGL(k_attn_part, dim3(a.KVH, a.n_items), dim3(256), 0, st, AP_ARGS(a));
    return 0;
}
int attention_merge(const AttnArgs& a, hipStream_t st) {
    if (a.n_items <= 0 || a.whole || a.n_mrows <= 0 || a.fold) return 0;
    // a row's chunk partials in one round of loads, as few clamped copies as the instances allow (configs[2]'s 9
    // chunks: 10 a round, decode 7,885 -> 7,918 tok/s against 16; configs[1]'s up to 16 chunks: 16)
    const int mc = a.max_chunks;
    const bool xa = a.KVH % 8 == 0;
    const dim3 grid = xa ? dim3(a.n_mrows * a.H) : dim3(a.n_mrows, a.H);
#define MERGE(MB_)                                                                               \
    do {                                                                                         \
        if (xa) hipLaunchKernelGGL((k_attn_merge<MB_, true>), grid, dim3(64), 0, st, AM_ARGS(a));         \
        else hipLaunchKernelGGL((k_attn_merge<MB_, false>), grid, dim3(64), 0, st, AM_ARGS(a));           \
    } while (0)
    if (mc <= 8) MERGE(8);
    else if (mc <= 10) MERGE(10);
    else if (mc <= 12) MERGE(12);
    else if (mc <= 16) MERGE(16);
    else MERGE(20);
#undef MERGE
    return 0;
}
int paged_attention(const AttnArgs& a, hipStream_t st) {
    int rc = attention_runs(a, st);
    if (!rc) rc = attention_items(a, st);
    return rc ? rc : attention_merge(a, st);
}

// The work list (see sn_kernels_internal.h). Whole groups when they make one round of workgroups on the 256 CUs
// (240 .. 256), no group's context is over 9/8 of the mean, and the contexts are long: at least 10 chunks on average,
// or 5 with 32-cell pages. Measured on MI355X (32 sequences, K/V beyond the Infinity Cache), whole groups beat chunk
// items plus merge by 10-20% at 12-16 chunks and at 32-cell pages when the contexts are alike, and lose 2-8% at 4 and
// 8 chunks of 64-cell pages and whenever the groups are not one round (16 or 48 sequences). A whole-group launch lasts
// as long as its longest context: at contexts U[256, 4096] (longest 1.7x the mean) it took 81.5 us against 66.0 for
// chunk items. Otherwise one item per (group, 256-cell chunk) and the merge folds every row's chunks. Prompt rows: run
// items first (see sn_kernels_internal.h), the rule above then over the groups outside them.
void attn_plan(int R, const int32_t* seq, const int32_t* pos, int H, int KVH, int page_cells, AttnPlan& p, int mode,
               const int32_t* pt, int max_pages) {
    const int gmax = 16 / (H / KVH);
    p.groups.clear();
    p.items.clear();
    p.runs.clear();
    p.mrows.clear();
    p.max_chunk = 0;
    for (int r = 0; r < R;) {
        int n = 1;
        while (r + n < R && n < gmax && seq[r + n] == seq[r] && pos[r + n] == pos[r] + n) ++n;
        p.groups.push_back({r, n, seq[r], pos[r]});
        p.max_chunk = std::max(p.max_chunk, (pos[r] + n - 1) / ATT_CHUNK + 1);
        r += n;
    }
    const int ng = (int) p.groups.size();
    const AttnItem none = {0, 0, 0, {-1, -1, -1}, 1};
    // run items: a sequence's consecutive groups at consecutive positions, every one but the last full
    std::vector<char> in_run(ng, 0);
    if (mode == -1 || mode == 2) {
        std::vector<AttnItem> runs;
        for (int gi = 0; gi < ng;) {
            int n = 1;
            while (gi + n < ng && p.groups[gi + n].seq == p.groups[gi].seq && p.groups[gi + n - 1].nrows == gmax &&
                   p.groups[gi + n].pos0 == p.groups[gi + n - 1].pos0 + gmax)
                ++n;
            if (n >= 2)
                for (int j = 0; j < n; j += ATT_RUN_MAX) {
                    AttnItem it = none;
                    it.group = gi + j;
                    it.nmem = std::min(ATT_RUN_MAX, n - j);
                    const AttnGroup& gl = p.groups[gi + j + it.nmem - 1];
                    it.nchunk = (gl.pos0 + gl.nrows - 1) / ATT_CHUNK + 1;
                    runs.push_back(it);
                }
            gi += n;
        }
        if (!runs.empty() && (mode == 2 || (long) runs.size() * KVH >= ATT_RUN_MIN_WG)) {
            p.runs = runs;
            for (const AttnItem& it : runs)
                for (int j = 0; j < it.nmem; ++j) in_run[it.group + j] = 1;
        }
    }
    // the other groups: whole groups or chunk items
    int tot = 0, mx = 0, nrest = 0;
    for (int gi = 0; gi < ng; ++gi) {
        if (in_run[gi]) continue;
        const AttnGroup& gr = p.groups[gi];
        const int nc = (gr.pos0 + gr.nrows - 1) / ATT_CHUNK + 1;
        tot += nc;
        mx = std::max(mx, nc);
        ++nrest;
    }
    const long wg = (long) nrest * KVH;
    const bool long_ctx = tot >= (page_cells == 32 ? 5L : 10L) * nrest;
    p.whole = mode == 0 || mode == 1 ? mode == 1
              : nrest > 0 && wg >= ATT_WHOLE_MIN_WG && wg <= ATT_WHOLE_MAX_WG && 8L * mx * nrest <= 9L * tot && long_ctx;
    // shared chunks: a one-row group's chunk that lies wholly below its position, keyed by the chunk's pages
    std::vector<std::vector<int>> taken(ng);  // per group, its chunks that went into shared items
    if (!p.whole && pt && max_pages > 0) {
        const int members = std::min(ATT_SHARE_MAX, 16 / (H / KVH));
        const int ppc = ATT_CHUNK / page_cells;  // pages a chunk
        std::map<std::vector<int32_t>, std::vector<int>> by_pages;  // pages + chunk -> groups
        for (int gi = 0; gi < ng; ++gi) {
            const AttnGroup& gr = p.groups[gi];
            if (gr.nrows != 1 || in_run[gi]) continue;
            for (int c = 0; (c + 1) * ATT_CHUNK - 1 <= gr.pos0; ++c) {
                std::vector<int32_t> k(ppc + 1);
                bool ok = true;
                for (int j = 0; j < ppc; ++j) {
                    k[j] = pt[(size_t) gr.seq * max_pages + c * ppc + j];
                    ok = ok && k[j] >= 0;
                }
                k[ppc] = c;
                if (ok) by_pages[k].push_back(gi);
            }
        }
        for (auto& kv : by_pages) {
            const std::vector<int>& gs = kv.second;
            const int c = kv.first.back();
            for (size_t i = 0; i + 1 < gs.size(); i += members) {  // (a last lone group keeps its own item)
                const int cnt = (int) std::min<size_t>(members, gs.size() - i);
                AttnItem it = none;
                it.group = gs[i];
                it.chunk = c;
                it.nchunk = 1;
                for (int j = 1; j < cnt; ++j) it.share[j - 1] = gs[i + j];
                p.items.push_back(it);
                for (int j = 0; j < cnt; ++j) taken[gs[i + j]].push_back(c);
            }
        }
    }
    for (int gi = 0; gi < ng; ++gi) {
        if (in_run[gi]) continue;
        const AttnGroup& gr = p.groups[gi];
        const int nc = (gr.pos0 + gr.nrows - 1) / ATT_CHUNK + 1;
        if (p.whole) {
            AttnItem it = none;
            it.group = gi, it.nchunk = nc;
            p.items.push_back(it);
        } else {
            for (int c = 0; c < nc; ++c) {
                if (std::find(taken[gi].begin(), taken[gi].end(), c) != taken[gi].end()) continue;
                AttnItem it = none;
                it.group = gi, it.chunk = c, it.nchunk = 1;
                p.items.push_back(it);
            }
            for (int i = 0; i < gr.nrows; ++i) p.mrows.push_back(gr.row0 + i);
        }
    }
    for (auto& it : p.items) it.g = p.groups[it.group];
    for (auto& it : p.runs) it.g = p.groups[it.group];
    // chunk items with more cells first (a context's short last chunk at the end of the launch): configs[2] 51.9 ->
    // 51.3 us a layer, configs[3]'s verify groups 33.3 -> 32.4 us; the results do not depend on the order
    if (!p.whole) {
        auto work = [&](const AttnItem& it) {
            const AttnGroup& gr = p.groups[it.group];
            return std::min(ATT_CHUNK, gr.pos0 + gr.nrows - it.chunk * ATT_CHUNK);
        };
        std::stable_sort(p.items.begin(), p.items.end(),
                         [&](const AttnItem& x, const AttnItem& y) { return work(x) > work(y); });
    }
}
