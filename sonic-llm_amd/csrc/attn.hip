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

__global__ __launch_bounds__(256) void k_attn_part(AttnArgs a) {
    __shared__ float s_o[4][16][ATT_D + 4];
    __shared__ float s_m[4][16], s_l[4][16];

    const AttnItem it = a.items[blockIdx.x];
    const AttnGroup gr = a.groups[it.group];
    const int kvh = blockIdx.y;
    const int G = a.H / a.KVH;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int pos_last = gr.pos0 + gr.nrows - 1;
    const int cbase = it.chunk * ATT_CHUNK + 64 * wave;  // this wavefront's first cell
    const size_t head_stride = (size_t) a.page_cells * ATT_D;

    // this lane's query (as a B column of S^T and the A row of O): n = row * G + head-in-group
    const int qrow = n / G, qhead = kvh * G + n % G;
    const bool qvalid = qrow < gr.nrows;
    const int qpos = gr.pos0 + qrow;

    // Q^T fragments: MFMA t covers dims 32t .. 32t+31; lane (n, g) holds dims 32t + 8g .. +7 of query n. Loaded as
    // 16-byte pieces from a valid row (an unused column reads the group's first row) and zeroed by a select, so no load
    // sits behind a branch.
    half8 qh[4], ql[4];
    {
        const float* qp = a.q + (size_t) (gr.row0 + (qvalid ? qrow : 0)) * a.ldq + (size_t) qhead * ATT_D;
        for (int t = 0; t < 4; ++t) {
            const float4 x0 = *(const float4*) (qp + 32 * t + 8 * g), x1 = *(const float4*) (qp + 32 * t + 8 * g + 4);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            for (int j = 0; j < 8; ++j) split_hl(qvalid ? xs[j] * a.scale : 0.0f, qh[t], ql[t], j);
        }
    }

    // The wavefront's 64 cells lie in one page (64-cell pages) or two (32-cell pages): their page ids are uniform, read
    // once. Every K and V load of the wavefront is issued here, before any arithmetic, so the whole 32 KB is in flight
    // at once (V does not depend on the scores).
    const int32_t* ptrow = a.pt + (size_t) gr.seq * a.max_pages;
    const int pc = a.page_cells;
    const int p_lo = cbase <= pos_last ? ptrow[cbase / pc] : 0;
    const int p_hi = cbase + 32 <= pos_last ? ptrow[(cbase + 32) / pc] : p_lo;
    const uint16_t* kbase0 = a.kpool + ((size_t) p_lo * a.KVH + kvh) * head_stride;
    const uint16_t* kbase1 = a.kpool + ((size_t) p_hi * a.KVH + kvh) * head_stride;
    const uint16_t* vbase0 = a.vpool + ((size_t) p_lo * a.KVH + kvh) * head_stride;
    const uint16_t* vbase1 = a.vpool + ((size_t) p_hi * a.KVH + kvh) * head_stride;
    auto cell_off = [&](int c) { return (size_t) (c % pc) * ATT_D; };  // c - cbase < 64
    // Cells past the group's last position are read from the same pages (memory that exists: a page holds whole
    // cells) and then zeroed by a select (a masked cell's p is exactly 0, and 0 * V must not meet a NaN).
    u32x4 kf[4][4], vf[2][8];
    const u32x4 z4 = {0u, 0u, 0u, 0u};
    for (int jg = 0; jg < 4; ++jg) {
        const int c = cbase + 16 * jg + n;
        const uint16_t* kp = (c - cbase < 32 ? kbase0 : kbase1) + cell_off(c);
        for (int t = 0; t < 4; ++t) kf[jg][t] = *(const u32x4*) (kp + 32 * t + 8 * g);
    }
    for (int st = 0; st < 2; ++st)
        for (int jj = 0; jj < 2; ++jj)
            for (int v = 0; v < 4; ++v) {
                const int c = cbase + 32 * st + 16 * jj + 4 * g + v;
                vf[st][4 * jj + v] = *(const u32x4*) ((st == 0 ? vbase0 : vbase1) + cell_off(c) + 8 * n);
            }
    for (int jg = 0; jg < 4; ++jg)
        if (cbase + 16 * jg + n > pos_last)
            for (int t = 0; t < 4; ++t) kf[jg][t] = z4;
    for (int st = 0; st < 2; ++st)
        for (int jj = 0; jj < 2; ++jj)
            for (int v = 0; v < 4; ++v)
                if (cbase + 32 * st + 16 * jj + 4 * g + v > pos_last) vf[st][4 * jj + v] = z4;

    // ---- scores for the wavefront's 64 cells: 4 groups of 16 cells
    floatx4 s[4];
    for (int jg = 0; jg < 4; ++jg) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int t = 0; t < 4; ++t) {
            const half8 kh = __builtin_bit_cast(half8, kf[jg][t]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[t], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[t], acc, 0, 0, 0);
        }
        s[jg] = acc;  // lane (n, g): cells cbase + 16 jg + 4 g + v, query n
    }

    // ---- the wavefront's softmax statistics per query (lanes n, n+16, n+32, n+48 share query n)
    float m = -INFINITY;
    for (int jg = 0; jg < 4; ++jg)
        for (int v = 0; v < 4; ++v) {
            const int c = cbase + 16 * jg + 4 * g + v;
            const bool ok = qvalid && c <= qpos;
            s[jg][v] = ok ? s[jg][v] : -INFINITY;
            m = fmaxf(m, s[jg][v]);
        }
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    float l = 0.0f;
    for (int jg = 0; jg < 4; ++jg)
        for (int v = 0; v < 4; ++v) {
            const float p = m == -INFINITY ? 0.0f : __expf(s[jg][v] - m);
            s[jg][v] = p;
            l += p;
        }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    // ---- O = P . V over two steps of 32 cells; MFMA t covers output dims {8 c + t : c = 0..15}
    floatx4 o[8];
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

    // ---- the 4 wavefronts combined in wavefront order
    if (g == 0) {
        s_m[wave][n] = m;
        s_l[wave][n] = l;
    }
    for (int t = 0; t < 8; ++t)
        for (int v = 0; v < 4; ++v) s_o[wave][4 * g + v][8 * n + t] = o[t][v];
    __syncthreads();
    // thread -> (query qq, 8 dims)
    const int qq = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
    const int row = qq / G, head = kvh * G + qq % G;
    if (row >= gr.nrows) return;
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][qq]);
    float e[4], L = 0.0f;
    for (int w = 0; w < 4; ++w) {
        e[w] = s_m[w][qq] == -INFINITY ? 0.0f : __expf(s_m[w][qq] - M);
        L += s_l[w][qq] * e[w];
    }
    float* dst = a.part + (((size_t) (gr.row0 + row) * a.H + head) * a.max_chunks + it.chunk) * (ATT_D + 2);
    for (int d = 0; d < 8; ++d) {
        float acc = 0.0f;
        for (int w = 0; w < 4; ++w) acc += s_o[w][qq][d0 + d] * e[w];
        dst[d0 + d] = acc;
    }
    if ((threadIdx.x & 15) == 0) {
        dst[ATT_D] = M;
        dst[ATT_D + 1] = L;
    }
}

// per (row, head): the chunks' partials in chunk order; out = acc / l. One wavefront, 2 dims a lane; the loads of 8
// chunks are issued together (chunk index clamped, no load behind a branch), then combined in order. With a.xa the
// head's 128 outputs (4 Q8_0 blocks of the o-projection's input row) are also quantized there, exactly as the
// activation quantizer does (ggml x86 quantize_row_q8_0), into the xa operand of K = H * 128.
__global__ __launch_bounds__(64) void k_attn_merge(AttnArgs a) {
    const int r = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int nc = a.row_pos[r] / ATT_CHUNK + 1;
    const float* p0 = a.part + ((size_t) r * a.H + h) * a.max_chunks * (ATT_D + 2);
    float M = -INFINITY, L = 0.0f, o0 = 0.0f, o1 = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 8) {
        float2 ov[8], ml[8];
        for (int j = 0; j < 8; ++j) {
            const float* pc = p0 + (size_t) (c0 + j < nc ? c0 + j : nc - 1) * (ATT_D + 2);
            ov[j] = *(const float2*) (pc + 2 * lane);
            ml[j] = *(const float2*) (pc + ATT_D);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // (a fixed trip count keeps ov and ml in registers)
            const float mc = ml[j].x, lc = ml[j].y;
            if (c0 + j >= nc || mc == -INFINITY) continue;  // past the row's chunks, or a chunk with no cell for it
            const float mn = fmaxf(M, mc);
            const float e0 = M == -INFINITY ? 0.0f : __expf(M - mn), e1 = __expf(mc - mn);
            o0 = o0 * e0 + ov[j].x * e1;
            o1 = o1 * e0 + ov[j].y * e1;
            L = L * e0 + lc * e1;
            M = mn;
        }
    }
    const float il = L > 0.0f ? 1.0f / L : 0.0f;
    o0 *= il;
    o1 *= il;
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

int paged_attention(const AttnArgs& a, hipStream_t st) {
    if (a.n_items <= 0) return 0;
    if (a.H % a.KVH != 0 || 16 % (a.H / a.KVH) != 0) return -1;
    hipLaunchKernelGGL(k_attn_part, dim3(a.n_items, a.KVH), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_attn_merge, dim3(a.n_rows, a.H), dim3(64), 0, st, a);
    return 0;
}
