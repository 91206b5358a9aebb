// 17..32 tokens of the dual GEMM for gfx950, any K % 128 == 0: K cut in
// 1024-column slices over the grid, partials added in slice order by a
// second launch when there is more than one slice.  One launch may take up
// to four layers that read the same activations (q / k / v, gate / up).
//
// Same formula as /root/reference/src/dual_gemm.cu:176-225.  With 32 tokens
// the activations of all of K (256 KB at K = 4096) fit neither one
// workgroup's LDS nor its registers, and a 16-row block alone carries too
// little weight (32 KB) to pay for reading them; so each workgroup takes
// one slice of K (8 chunks, the ortho plan's slice record cell) and a run
// of 64-row groups (of one or more layers), and keeps the slice's
// activations in registers for the whole launch:
//
//  * 8 waves, two per SIMD.  The slice's activations are read once with
//    coalesced loads and staged row-major in LDS; wave w takes chunks
//    2 (w % 4), + 1 of the slice (its MFMA A operands, 32 tokens x 256
//    columns: 64 registers, read back from LDS once; the space is then
//    reused) and rows 32 (w / 4) .. + 31 of each group: per group it streams
//    32 rows x 256 columns of weights (nontemporal, one group ahead: issued
//    further ahead they delay the activations' loads), converts each word
//    into 8 exact biased FP16 integers (five bit operations; BF16
//    activations: the exact BF16 integers q + 136) and feeds
//    v_mfma_f32_16x16x32_f16 for both token tiles.  The bias (1032 per even
//    and 72 per odd column, 136 per column in BF16) times the activation sums
//    is formed once per launch by MFMAs of the A operands against a constant
//    B (the conversion of q = 0) and kept, negated, in 16 registers: it
//    starts each chunk's MFMA chain, so the chain yields the chunk's partial
//    without the bias and one FMA applies the group scale.
//  * The four waves of a row half hold the slice's four chunk pairs; their
//    partials meet in LDS and are added in wave order (deterministic).
//  * Ortho term (alpha > 0, planned): the same loads are staged a second
//    time, transposed (a column's 32 tokens contiguous).  Per group, wave w
//    stages the slice record of 16-row block 2 (w / 4) + (w % 4) / 2 in its
//    own LDS region and sums v * x for the tokens of tile w % 2, four lanes
//    per row: entries in pairs, each token's two products by one
//    v_dot2_f32_f16 (BF16 activations: one FMA per product).  The quad's
//    sums go to LDS and are added, times alpha, when the partials meet.  A
//    block whose entries did not fit its record (or another layer's plan)
//    reads the rows' CSR, filtered to the slice's columns.
//  * One slice (K <= 1024): the workgroup writes y (+ bias).  Else each
//    writes its FP32 partial [slice][M][N] and split_reduce_kernel adds the
//    slices in order and rounds (+ bias), for every layer of the launch.
//    (An in-kernel hand-off through device-scope fences, the last
//    workgroup of a group adding the slices, measured 10x slower: the
//    fences write back and invalidate the L2 of every XCD.)
#include <algorithm>
#include <atomic>

#include "orth_common.h"

namespace orth {

int plan_srec_words(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip
int64_t plan_srec_at(int64_t N, int64_t K, int64_t nnz);

constexpr int kSpW = 8;             // waves per workgroup
constexpr int kSpNT = 64 * kSpW;
constexpr int kSpRows = 64;         // rows per group
constexpr int kSpMT = 32;           // tokens (two MFMA tiles)
constexpr int kSpRS = 36;           // row stride of the LDS partial and sparse-sum buffers, in floats
constexpr int kSpCols = 1024;       // columns per slice
constexpr int kSpXS = kSpCols + 8;  // row stride of the row-major staging, in halves
constexpr int kSpMaxLayers = 4;     // layers one launch may take
static const int64_t kSpLdsMax = 160 * 1024;

// The per-layer part of a launch.
struct SplitLayer {
    const uint8_t *q;
    const f16 *scales;
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int32_t nnz;
    void *y;               // one slice: the output [M][N]
    float *part;           // more slices: [S][M][N]
    const void *bias;
    int bias_dtype;
    int64_t N;
    int nb16;              // 16-row blocks
    float alpha;
    const uint32_t *srec;  // plan slice records, swords words per (16-row block, slice)
};

struct SplitArgs {
    SplitLayer L[kSpMaxLayers];
    int nlayers;
    int gofs[kSpMaxLayers + 1];  // groups of layer l: [gofs[l], gofs[l + 1])
    int ngroups;        // scale groups per row (every layer)
    int gshift;         // scale group of chunk c: c >> gshift
    const f16 *x;       // FP16 or BF16 bits
    int M;
    int K;
    int nchunks;
    int S;              // slices
    int wps;            // workgroups per slice
    int ngrp;           // 64-row groups of all layers
    int lds_xt, lds_red, lds_sp, lds_rec;  // byte offsets of the LDS regions
    int swords;         // record words (every layer)
};

// SPARSE: 0 no ortho term, 1 / 2 slice records of 256 / 512 words.
// XB: BF16 activations and output.
template <int SPARSE, bool XB>
__global__ void __launch_bounds__(kSpNT) split_kernel(SplitArgs a) {
    constexpr int NTT = 2;
    constexpr int RS = kSpRS;
    constexpr int ER = SPARSE ? SPARSE : 1;  // 16-byte record loads per lane
    static_assert(kSpMaxLayers == 4, "the layer pick below takes up to four layers");

    extern __shared__ __align__(16) unsigned char smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem);                    // [32 tokens][kSpXS] row-major (prologue)
    f16 *xt = reinterpret_cast<f16 *>(smem + a.lds_xt);
    float *red = reinterpret_cast<float *>(smem + a.lds_red);    // [4 pairs][64 rows][RS]
    float *sp = reinterpret_cast<float *>(smem + a.lds_sp);      // [64 rows][RS]
    // column c of the transposed slice: its 32 tokens, 16 bytes of padding
    // after every 8 columns (the lanes' 16-byte writes spread over the banks)
    auto xt_col = [&](int c) -> const f16 * { return xt + c * kSpMT + (c >> 3) * 8; };

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int nl = lane & 15;  // B column (weight row) and A row (token within a tile)
    const int g = lane >> 4;   // which 32 columns of a chunk
    const int kq = wave & 3;   // chunk pair of the slice
    const int rh = wave >> 2;  // row half of a group
    const int s = (int)(blockIdx.x % (unsigned)a.S);
    const int wgj = (int)(blockIdx.x / (unsigned)a.S);
    const int K = a.K;
    const int cs0 = 8 * s;                            // first chunk of the slice
    const int col0 = cs0 * 128;
    const int scols = min(8, a.nchunks - cs0) * 128;  // columns of the slice
    const int cw = cs0 + 2 * kq;                      // the wave's first chunk
    const int cv = max(0, min(2, a.nchunks - cw));    // its valid chunks (uniform)
    const int clast = a.nchunks - 1;

    // a group's layer and its group within the layer.  Constant indices
    // only: an index computed at run time into the argument struct would
    // move the whole struct to scratch memory.
    auto layer_of = [&](int gi, int &lg) -> SplitLayer {
        const int l = (gi >= a.gofs[1] ? 1 : 0) + (a.nlayers > 2 && gi >= a.gofs[2] ? 1 : 0) +
                      (a.nlayers > 3 && gi >= a.gofs[3] ? 1 : 0);
        lg = gi - (l == 0 ? 0 : (l == 1 ? a.gofs[1] : (l == 2 ? a.gofs[2] : a.gofs[3])));
        return l == 0 ? a.L[0] : (l == 1 ? a.L[1] : (l == 2 ? a.L[2] : a.L[3]));
    };

    // ---- loads at entry: the slice's activations, coalesced (lane: columns
    //      8 (l % 16) .. of the wave's 128, tokens 8 (l / 16) ..: each
    //      instruction reads 256 contiguous bytes of four token rows), then
    //      the first group's weights, scales and record
    const int scg = lane & 15, sth = lane >> 4;
    const int scol = 128 * wave + 8 * scg;  // slice-local column of the staging lane
    u32x4 xr[8];
#pragma unroll
    for (int t = 0; t < 8; t++)
        xr[t] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)min(8 * sth + t, a.M - 1) * K +
                                                 min(col0 + scol, K - 8));

    // per-group loads: weights (lane: row nl of row tile rt, 16 bytes at 16 g
    // of the chunk's 64), group scales and the wave's block record
    const int bi = 2 * rh + (kq >> 1);  // the wave's 16-row block of a group (sparse term)
    struct Buf {
        u32x4 w[2][2];
        uint32_t sc[2][2];
        u32x4 r[ER];
    };
    auto issue = [&](int gi, Buf &b) {
        int lg = 0;
        const SplitLayer L = layer_of(gi, lg);
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            const int64_t row = min((int64_t)lg * kSpRows + 32 * rh + 16 * rt + nl, L.N - 1);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int c = min(cw + p, clast);
                b.w[rt][p] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(L.q + row * (int64_t)(K >> 1) + c * 64 + 16 * g));
                b.sc[rt][p] = __builtin_bit_cast(uint16_t, L.scales[row * a.ngroups + (c >> a.gshift)]);
            }
        }
        if (SPARSE) {
            const int64_t blk = min((int64_t)lg * 4 + bi, (int64_t)L.nb16 - 1);
            const uint32_t *rb = L.srec + (blk * a.S + s) * (int64_t)a.swords;
#pragma unroll
            for (int e = 0; e < ER; e++)
                b.r[e] = *reinterpret_cast<const u32x4 *>(rb + min(4 * (lane + 64 * e), a.swords - 4));
        }
    };
    Buf cur, nxt;
    issue(wgj, cur);

    // ---- staging (tokens past M and columns past K zero): row-major in the
    //      interleaved k order, read back below as the A operands; and, for
    //      the ortho term, transposed
#pragma unroll
    for (int t = 0; t < 8; t++)
        if (8 * sth + t >= a.M || col0 + scol >= K) xr[t] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; t++)
        *reinterpret_cast<u32x4 *>(xs + (8 * sth + t) * kSpXS + scol) = permute_x8(xr[t]);
    if (SPARSE) {
#pragma unroll
        for (int jc = 0; jc < 8; jc++) {
            uint32_t wd[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                wd[u] = __builtin_amdgcn_perm(xr[2 * u + 1][jc >> 1], xr[2 * u][jc >> 1],
                                              (jc & 1) ? 0x07060302u : 0x05040100u);
            const int c = scol + jc;
            *reinterpret_cast<u32x4 *>(xt + c * kSpMT + (c >> 3) * 8 + 8 * sth) = u32x4{wd[0], wd[1], wd[2], wd[3]};
        }
    }
    __syncthreads();  // the slice is in LDS, both ways

    // ---- the wave's A operands for the whole launch: tile t, token 16 t +
    //      nl, chunk cw + p, k step kk (columns 32 g + 8 kk ..)
    u32x4 afr[NTT][2][4];
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int p = 0; p < 2; p++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                afr[t][p][kk] = *reinterpret_cast<const u32x4 *>(xs + (16 * t + nl) * kSpXS + (2 * kq + p) * 128 +
                                                                 32 * g + 8 * kk);
    auto mfma = [](const u32x4 &av, const uint32_t b[4], f32x4 c) -> f32x4 {
        if constexpr (XB)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                           __builtin_bit_cast(bf16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                          __builtin_bit_cast(f16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                          c, 0, 0, 0);
    };
    // the conversion of q = 0: every column's bias.  Its sums per chunk and
    // token (the same in every column of the product), negated, start each
    // chunk's MFMA chain below: the chain then yields the partial with the
    // bias removed, and only the group scale is left to apply.
    const uint32_t kb[4] = {XB ? 0x43084308u : 0x64086408u, XB ? 0x43084308u : 0x54805480u,
                            XB ? 0x43084308u : 0x64086408u, XB ? 0x43084308u : 0x54805480u};
    f32x4 nbias[2][NTT];
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int p = 0; p < 2; p++) {
            f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; kk++) z = mfma(afr[t][p][kk], kb, z);
            nbias[p][t] = -z;
        }
    __syncthreads();  // every wave has its A operands: the row-major copy's space is reused below

    uint32_t *er = reinterpret_cast<uint32_t *>(smem + a.lds_rec) + wave * a.swords;
    const int qr = lane >> 2, qe = lane & 3;  // sparse term: row of the block, lane of its quad
    const int th = kq & 1;                    // sparse term: the wave's token tile

    // ---- group gi from cur; MORE: the next group's loads into nxt first,
    //      and cur takes them at the end (the copy waits for them, which the
    //      next group needs at once anyway)
    auto group = [&](int gi, auto more_c) {
        constexpr bool MORE = decltype(more_c)::value;
        if (MORE) issue(gi + a.wps, nxt);
        int lg = 0;
        const SplitLayer L = layer_of(gi, lg);

        // ---- sparse sums of the wave's block and token tile
        if (SPARSE) {
#pragma unroll
            for (int e = 0; e < ER; e++) {
                const int o = 4 * (lane + 64 * e);
                if (o < a.swords) *reinterpret_cast<u32x4 *>(er + o) = cur.r[e];
            }
            __builtin_amdgcn_wave_barrier();  // (same wave: LDS keeps the order)
            const int64_t blk = (int64_t)lg * 4 + bi;
            const int64_t row = blk * 16 + qr;
            float sacc[16];
#pragma unroll
            for (int m = 0; m < 16; m++) sacc[m] = 0.f;
            // a pair of entries (their columns' 16 tokens xa, xb; values as
            // the FP16 pair vp): each token's two products
            auto products = [&](const u32x4 (&ua)[2], const u32x4 (&ub)[2], uint32_t vp) {
                const uint32_t xa[8] = {ua[0].x, ua[0].y, ua[0].z, ua[0].w, ua[1].x, ua[1].y, ua[1].z, ua[1].w};
                const uint32_t xb[8] = {ub[0].x, ub[0].y, ub[0].z, ub[0].w, ub[1].x, ub[1].y, ub[1].z, ub[1].w};
                if constexpr (XB) {
                    const float va = (float)__builtin_bit_cast(f16, (uint16_t)(vp & 0xffffu));
                    const float vb = (float)__builtin_bit_cast(f16, (uint16_t)(vp >> 16));
#pragma unroll
                    for (int w = 0; w < 8; w++) {
                        sacc[2 * w] = __builtin_fmaf(va, bf16_bits_to_f32((uint16_t)(xa[w] & 0xffffu)), sacc[2 * w]);
                        sacc[2 * w + 1] = __builtin_fmaf(va, bf16_bits_to_f32((uint16_t)(xa[w] >> 16)), sacc[2 * w + 1]);
                        sacc[2 * w] = __builtin_fmaf(vb, bf16_bits_to_f32((uint16_t)(xb[w] & 0xffffu)), sacc[2 * w]);
                        sacc[2 * w + 1] = __builtin_fmaf(vb, bf16_bits_to_f32((uint16_t)(xb[w] >> 16)), sacc[2 * w + 1]);
                    }
                } else {
                    const f16x2 v2 = __builtin_bit_cast(f16x2, vp);
#pragma unroll
                    for (int w = 0; w < 8; w++) {
                        const uint32_t lo = __builtin_amdgcn_perm(xb[w], xa[w], 0x05040100u);  // token 2w: (xa, xb)
                        const uint32_t hi = __builtin_amdgcn_perm(xb[w], xa[w], 0x07060302u);  // token 2w + 1
                        sacc[2 * w] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, lo), v2, sacc[2 * w], false);
                        sacc[2 * w + 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, hi), v2, sacc[2 * w + 1], false);
                    }
                }
            };
            auto pair = [&](int ca, int cb, uint32_t vp) {
                const u32x4 *pa = reinterpret_cast<const u32x4 *>(xt_col(ca) + 16 * th);
                const u32x4 *pb = reinterpret_cast<const u32x4 *>(xt_col(cb) + 16 * th);
                const u32x4 ua[2] = {pa[0], pa[1]}, ub[2] = {pb[0], pb[1]};
                products(ua, ub, vp);
            };
            const bool ok = (er[0] == plan_cell_tag(kCellSlice, L.N, K, L.nnz, a.swords, blk, s)) &
                            (er[1] == 0u);  // (uniform)
            if (ok) {
                const uint32_t hw = er[2 + qr];
                const int32_t lo = (int32_t)(hw & 0xffffu);
                const int32_t hi = row < L.N ? (int32_t)(hw >> 16) : lo;
                const uint32_t *ee = er + kCellHdrWords;
                // two pairs per pass (entries j0 + 4 u, u < 4): every LDS
                // read of the pass is issued before the products, one round
                // trip for the record words and one for the activations
                for (int32_t j0 = lo + qe; j0 < hi; j0 += 16) {
                    uint32_t w[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) w[u] = ee[min(j0 + 4 * u, hi - 1)];
                    uint32_t vp[2];
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const bool va = j0 + 8 * h < hi, vb = j0 + 8 * h + 4 < hi;
                        vp[h] = (va ? (w[2 * h] >> 16) : 0u) | (vb ? (w[2 * h + 1] & 0xffff0000u) : 0u);
                    }
                    u32x4 xv[4][2];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const u32x4 *pc = reinterpret_cast<const u32x4 *>(xt_col((int)(w[u] & 0xffffu)) + 16 * th);
                        xv[u][0] = pc[0];
                        xv[u][1] = pc[1];
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int h = 0; h < 2; h++) products(xv[2 * h], xv[2 * h + 1], vp[h]);
                }
            } else {
                int32_t fs = 0, fe = 0;
                csr_row_range(L.row_ptr, min(row, L.N - 1), L.nnz, fs, fe);
                if (row >= L.N) fe = fs;
                for (int32_t jj = fs + qe; jj < fe; jj += 4) {
                    const int32_t c = L.col[jj] - col0;
                    const bool okc = c >= 0 && c < scols;
                    const uint32_t v = okc ? (uint32_t)__builtin_bit_cast(uint16_t, L.vals[jj]) : 0u;
                    pair(okc ? c : 0, 0, v);
                }
            }
            // quad sums (fixed order), to LDS
#pragma unroll
            for (int m = 0; m < 16; m++) {
                float v = sacc[m];
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
                sacc[m] = v;
            }
            if (qe == 0) {
                float *dst = sp + (16 * bi + qr) * RS + 16 * th;
#pragma unroll
                for (int m = 0; m < 16; m += 4)
                    *reinterpret_cast<f32x4 *>(dst + m) = f32x4{sacc[m], sacc[m + 1], sacc[m + 2], sacc[m + 3]};
            }
        }

        // ---- dense term: row tiles x chunks, both token tiles; each chunk's
        //      chain starts at minus its bias sums and takes its group scale
        f32x4 acc[2][NTT];
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int t = 0; t < NTT; t++) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                if (p < cv) {  // uniform
                    const uint32_t u[4] = {cur.w[rt][p].x, cur.w[rt][p].y, cur.w[rt][p].z, cur.w[rt][p].w};
                    f32x4 part[NTT];
#pragma unroll
                    for (int t = 0; t < NTT; t++) part[t] = nbias[p][t];
#pragma unroll
                    for (int kk = 0; kk < 4; kk++) {
                        uint32_t bw[4];
                        if constexpr (XB) int4x8_to_bf16_biased(u[kk], bw);
                        else int4x8_to_f16_biased(u[kk], bw);
#pragma unroll
                        for (int t = 0; t < NTT; t++) part[t] = mfma(afr[t][p][kk], bw, part[t]);
                    }
                    const float scl = (float)__builtin_bit_cast(f16, (uint16_t)cur.sc[rt][p]);
#pragma unroll
                    for (int t = 0; t < NTT; t++)
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[rt][t][i] = __builtin_fmaf(scl, part[t][i], acc[rt][t][i]);
                }
            }
        }
        // ---- partials to LDS: lane (row nl of tile rt, tokens 16 t + 4 g ..)
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int t = 0; t < NTT; t++)
                *reinterpret_cast<f32x4 *>(red + (kq * kSpRows + 32 * rh + 16 * rt + nl) * RS + 16 * t + 4 * g) =
                    acc[rt][t];
        __syncthreads();  // every wave's partials and sparse sums are in LDS

        // ---- thread (row tid % 64, tokens 4 (tid / 64) ..): the four chunk
        //      pairs in order, + alpha * sparse; y or the slice's partial
        {
            const int crow = tid & 63, tq = tid >> 6;
            const int64_t n = (int64_t)lg * kSpRows + crow;
            f32x4 v = *reinterpret_cast<const f32x4 *>(red + crow * RS + 4 * tq);
#pragma unroll
            for (int w = 1; w < 4; w++) v += *reinterpret_cast<const f32x4 *>(red + (w * kSpRows + crow) * RS + 4 * tq);
            if (SPARSE) {
                const f32x4 e = *reinterpret_cast<const f32x4 *>(sp + crow * RS + 4 * tq);
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] += L.alpha * e[i];
            }
            if (n < L.N) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 4 * tq + i;
                    if (m < a.M) {
                        if (a.S == 1) {
                            if constexpr (XB) static_cast<uint16_t *>(L.y)[(int64_t)m * L.N + n] = out_bf16(v[i], L.bias, L.bias_dtype, n);
                            else static_cast<f16 *>(L.y)[(int64_t)m * L.N + n] = out_f16(v[i], L.bias, L.bias_dtype, n);
                        } else {
                            L.part[((int64_t)s * a.M + m) * L.N + n] = v[i];
                        }
                    }
                }
            }
        }
        __syncthreads();  // the buffers are read before the next group writes them
        if (MORE) cur = nxt;
    };
    // the workgroup's groups: wgj, wgj + wps, ... (the host gives every
    // workgroup at least one)
    const int its = (a.ngrp - wgj + a.wps - 1) / a.wps;  // (uniform)
    int gi = wgj;
    for (int i = 0; i < its - 1; i++, gi += a.wps) group(gi, std::integral_constant<bool, true>{});
    group(gi, std::integral_constant<bool, false>{});
}

// y = part[0] + part[1] + ... + part[S - 1] (in that order), rounded (+ bias),
// for every layer of a launch: workgroups [rb0[l], rb0[l + 1]) take layer l;
// thread t takes 4 consecutive outputs of one token (N % 4 == 0; else one).
// The slices' loads are issued four at a time (addresses clamped), so that
// 11 slices cost three memory round trips, not eleven.
struct SplitReduceArgs {
    const float *part[kSpMaxLayers];
    void *y[kSpMaxLayers];
    const void *bias[kSpMaxLayers];
    int bias_dtype[kSpMaxLayers];
    int64_t N[kSpMaxLayers];
    int vec4[kSpMaxLayers];
    int rb0[kSpMaxLayers + 1];
    int nlayers;
    int M;
    int S;
    int xb;
};

__global__ void __launch_bounds__(256) split_reduce_kernel(SplitReduceArgs r) {
    constexpr int U = 4;
    int bid = (int)blockIdx.x;
    const int l = (bid >= r.rb0[1] ? 1 : 0) + (r.nlayers > 2 && bid >= r.rb0[2] ? 1 : 0) +
                  (r.nlayers > 3 && bid >= r.rb0[3] ? 1 : 0);
    // (constant indices only, as in split_kernel)
#define ORTH_PICK(f) (l == 0 ? r.f[0] : (l == 1 ? r.f[1] : (l == 2 ? r.f[2] : r.f[3])))
    const float *part = ORTH_PICK(part);
    void *y = ORTH_PICK(y);
    const void *bias = ORTH_PICK(bias);
    const int bias_dtype = ORTH_PICK(bias_dtype);
    const int64_t N = ORTH_PICK(N);
    const int vec4 = ORTH_PICK(vec4);
    bid -= ORTH_PICK(rb0);
#undef ORTH_PICK
    const int S = r.S, xb = r.xb;
    const int64_t MN = (int64_t)r.M * N;
    const int64_t t = (int64_t)bid * 256 + threadIdx.x;
    if (vec4) {
        const int64_t o = 4 * t;
        if (o >= MN) return;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += U) {
            f32x4 w[U];
#pragma unroll
            for (int u = 0; u < U; u++) w[u] = *reinterpret_cast<const f32x4 *>(part + min(s0 + u, S - 1) * MN + o);
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u == 0) v = w[u];
                else if (s0 + u < S) v += w[u];
            }
        }
        const int64_t n = o % N;
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            h[e] = xb ? (uint32_t)out_bf16(v[e], bias, bias_dtype, n + e)
                      : (uint32_t)__builtin_bit_cast(uint16_t, out_f16(v[e], bias, bias_dtype, n + e));
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + o) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
        if (t >= MN) return;
        float v = 0.f;
        for (int s0 = 0; s0 < S; s0 += U) {
            float w[U];
#pragma unroll
            for (int u = 0; u < U; u++) w[u] = part[min(s0 + u, S - 1) * MN + t];
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u == 0) v = w[u];
                else if (s0 + u < S) v += w[u];
            }
        }
        if (xb) static_cast<uint16_t *>(y)[t] = out_bf16(v, bias, bias_dtype, t % N);
        else static_cast<f16 *>(y)[t] = out_f16(v, bias, bias_dtype, t % N);
    }
}

// ------------------------------------------------------------------ host

struct SplitShape {
    int sparse, lds, grid, swords, gshift;
    bool xb;
};

// One layer's part of the shape (sparse class, record size, scale layout):
// what every layer of a launch must share.
static bool split_layer_shape(const ForwardArgs &a, const void *plan, SplitShape &sh) {
    if (a.M < 1 || a.M > kSpMT) return false;
    if ((a.io_dtype != ORTH_DT_F16 && a.io_dtype != ORTH_DT_BF16) || a.scale_dtype != ORTH_DT_F16) return false;
    sh.xb = a.io_dtype == ORTH_DT_BF16;
    if (a.K % 128 != 0 || a.K < 128 || a.K > (1 << 20)) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    if (a.N < 1 || a.N > ((int64_t)1 << 31)) return false;
    // scales: per row, or groups of 128 * 2^j columns
    sh.gshift = 30;
    if (a.ngroups != 1) {
        if (a.G % 128 != 0) return false;
        sh.gshift = 0;
        while ((int64_t)128 << sh.gshift < a.G) sh.gshift++;
        if ((int64_t)128 << sh.gshift != a.G) return false;
    }
    sh.sparse = 0;
    sh.swords = 0;
    if (a.has_ortho) {
        // the ortho term comes from the plan's slice records
        if (!plan || a.val_dtype != ORTH_DT_F16) return false;
        sh.swords = plan_srec_words(a.N, a.K, a.nnz);
        if (sh.swords != 256 && sh.swords != 512) return false;
        sh.sparse = sh.swords / 256;
    }
    return true;
}

static bool split_shape(const ForwardArgs *as, const void *const *plans, int count, SplitArgs *d, SplitShape &sh) {
    if (count < 1 || count > kSpMaxLayers) return false;
    if (!split_layer_shape(as[0], plans[0], sh)) return false;
    int64_t ngrp = 0;
    int gofs[kSpMaxLayers + 1] = {0, 0, 0, 0, 0};
    for (int l = 0; l < count; l++) {
        SplitShape s1;
        if (!split_layer_shape(as[l], plans[l], s1)) return false;
        if (l > 0 && (s1.sparse != sh.sparse || s1.swords != sh.swords || s1.gshift != sh.gshift || s1.xb != sh.xb ||
                      as[l].K != as[0].K || as[l].M != as[0].M || as[l].ngroups != as[0].ngroups ||
                      as[l].x != as[0].x))
            return false;
        ngrp += (as[l].N + kSpRows - 1) / kSpRows;
        if (ngrp > ((int64_t)1 << 30)) return false;
        gofs[l + 1] = (int)ngrp;
    }
    for (int l = count + 1; l <= kSpMaxLayers; l++) gofs[l] = (int)ngrp;
    const ForwardArgs &a = as[0];
    const int nchunks = (int)(a.K / 128);
    const int S = (nchunks + 7) / 8;
    // the row-major staging (prologue) at 0, the transposed one after it;
    // after the prologue the row-major space
    // holds the partials [4][64][RS], the sparse sums [64][RS] and the waves'
    // records
    auto al = [](int64_t v) { return (v + 15) & ~int64_t(15); };
    const int64_t xs_bytes = al((int64_t)kSpMT * kSpXS * 2);
    const int64_t lds_red = 0;
    const int64_t lds_sp = al(4 * kSpRows * kSpRS * 4);
    const int64_t lds_rec = lds_sp + (sh.sparse ? al(kSpRows * kSpRS * 4) : 0);
    if (lds_rec + (int64_t)kSpW * sh.swords * 4 > xs_bytes) return false;
    const int64_t lds_xt = xs_bytes;
    const int64_t total = lds_xt + (sh.sparse ? al((int64_t)kSpCols * kSpMT * 2 + (kSpCols / 8) * 16) : 0);
    if (total > kSpLdsMax) return false;
    sh.lds = (int)total;
    // one workgroup per CU: S slices x wps workgroups, each with >= 1 group
    const int wps = (int)std::max<int64_t>(1, std::min<int64_t>(ngrp, 256 / S));
    sh.grid = S * wps;
    if (d) {
        for (int l = 0; l < kSpMaxLayers; l++) {
            const int lc = l < count ? l : 0;
            const ForwardArgs &b = as[lc];
            SplitLayer &L = d->L[l];
            L.q = b.q;
            L.scales = static_cast<const f16 *>(b.scales);
            L.row_ptr = b.row_ptr;
            L.col = b.col;
            L.vals = static_cast<const f16 *>(b.vals);
            L.nnz = (int32_t)b.nnz;
            L.y = b.y;
            L.part = nullptr;
            L.bias = b.bias;
            L.bias_dtype = b.bias_dtype;
            L.N = b.N;
            L.nb16 = (int)((b.N + 15) / 16);
            L.alpha = b.alpha;
            L.srec = sh.sparse ? reinterpret_cast<const uint32_t *>(static_cast<const char *>(plans[lc]) +
                                                                    plan_srec_at(b.N, b.K, b.nnz))
                               : nullptr;
        }
        d->nlayers = count;
        for (int l = 0; l <= kSpMaxLayers; l++) d->gofs[l] = gofs[l];
        d->ngroups = (int)a.ngroups;
        d->gshift = sh.gshift;
        d->x = static_cast<const f16 *>(a.x);
        d->M = (int)a.M;
        d->K = (int)a.K;
        d->nchunks = nchunks;
        d->S = S;
        d->wps = wps;
        d->ngrp = (int)ngrp;
        d->lds_xt = (int)lds_xt;
        d->lds_red = (int)lds_red;
        d->lds_sp = (int)lds_sp;
        d->lds_rec = (int)lds_rec;
        d->swords = sh.swords;
    }
    return true;
}

// Whether the slice-split kernel takes this call (with this plan or none).
bool split_supported(const ForwardArgs &a, const void *plan) {
    SplitShape sh;
    return split_shape(&a, &plan, 1, nullptr, sh);
}

// Whether one launch takes these layers (same K, activations, token count,
// scale layout, ortho class and record size).
bool split_group_ok(const ForwardArgs *as, const void *const *plans, int count) {
    SplitShape sh;
    return count >= 2 && split_shape(as, plans, count, nullptr, sh);
}

// Workspace bytes of a call: the slices' FP32 partials (none for one slice).
int64_t split_workspace_bytes(const ForwardArgs &a) {
    const int64_t S = (a.K / 128 + 7) / 8;
    return S > 1 ? S * a.M * a.N * 4 : 0;
}

int64_t split_group_workspace_bytes(const ForwardArgs *as, int count) {
    int64_t b = 0;
    for (int l = 0; l < count; l++) b += split_workspace_bytes(as[l]);
    return b;
}

template <int SPARSE, bool XB>
static hipError_t split_launch_t(const SplitArgs &d, const SplitShape &sh, hipStream_t s) {
    // more than 64 KB of dynamic LDS must be allowed once per device (the
    // attribute call is idempotent, so two threads racing to set it is harmless)
    static std::atomic<int> allowed[64];
    int dev = 0;
    if (sh.lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 &&
        !allowed[dev].load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(split_kernel<SPARSE, XB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSpLdsMax);
        if (e != hipSuccess) return e;
        allowed[dev].store(1, std::memory_order_release);
    }
    hipLaunchKernelGGL((split_kernel<SPARSE, XB>), dim3((unsigned)sh.grid), dim3(kSpNT), (uint32_t)sh.lds, s, d);
    return hipGetLastError();
}

template <bool XB>
static hipError_t split_launch_x(const SplitArgs &d, const SplitShape &sh, hipStream_t s) {
    switch (sh.sparse) {
        case 1: return split_launch_t<1, XB>(d, sh, s);
        case 2: return split_launch_t<2, XB>(d, sh, s);
        default: return split_launch_t<0, XB>(d, sh, s);
    }
}

// Layers as[0 .. count) reading one input (plans[l]: layer l's ortho plan,
// required when its ortho term is on); part: a workspace of
// split_group_workspace_bytes bytes (unused with one slice).
hipError_t launch_split_group(const ForwardArgs *as, const void *const *plans, int count, float *part,
                              hipStream_t stream) {
    SplitArgs d;
    SplitShape sh;
    if (!split_shape(as, plans, count, &d, sh)) return hipErrorInvalidValue;
    if (d.S > 1 && !part) return hipErrorInvalidValue;
    SplitReduceArgs r;
    r.nlayers = count;
    r.M = d.M;
    r.S = d.S;
    r.xb = sh.xb ? 1 : 0;
    int64_t off = 0, blocks = 0;
    for (int l = 0; l < kSpMaxLayers; l++) {
        const ForwardArgs &b = as[l < count ? l : 0];
        if (l < count) {
            d.L[l].part = part ? part + off : nullptr;
            off += split_workspace_bytes(b) / 4;
        } else {
            d.L[l].part = d.L[0].part;
        }
        r.part[l] = d.L[l].part;
        r.y[l] = b.y;
        r.bias[l] = b.bias;
        r.bias_dtype[l] = b.bias_dtype;
        r.N[l] = b.N;
        r.vec4[l] = b.N % 4 == 0 ? 1 : 0;
        r.rb0[l] = (int)blocks;
        if (l < count) {
            const int64_t threads = r.vec4[l] ? b.M * b.N / 4 : b.M * b.N;
            blocks += (threads + 255) / 256;
        }
    }
    r.rb0[kSpMaxLayers] = (int)blocks;
    hipError_t e = sh.xb ? split_launch_x<true>(d, sh, stream) : split_launch_x<false>(d, sh, stream);
    if (e != hipSuccess || d.S == 1) return e;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, r);
    return hipGetLastError();
}

// y = part[0] + ... + part[S - 1] for one layer (the prefill kernel's K
// split), rounded (+ bias) as above
hipError_t launch_slice_reduce(const ForwardArgs &a, const float *part, int S, hipStream_t stream) {
    SplitReduceArgs r;
    r.nlayers = 1;
    r.M = (int)a.M;
    r.S = S;
    r.xb = a.io_dtype == ORTH_DT_BF16 ? 1 : 0;
    const int vec4 = a.N % 4 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 7) == 0 ? 1 : 0;
    const int64_t threads = vec4 ? a.M * a.N / 4 : a.M * a.N;
    const int64_t blocks = (threads + 255) / 256;
    for (int l = 0; l < kSpMaxLayers; l++) {
        r.part[l] = part;
        r.y[l] = a.y;
        r.bias[l] = a.bias;
        r.bias_dtype[l] = a.bias_dtype;
        r.N[l] = a.N;
        r.vec4[l] = vec4;
        r.rb0[l] = l == 0 ? 0 : (int)blocks;
    }
    r.rb0[kSpMaxLayers] = (int)blocks;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, r);
    return hipGetLastError();
}

hipError_t launch_split(const ForwardArgs &a, const void *plan, float *part, hipStream_t stream) {
    return launch_split_group(&a, &plan, 1, part, stream);
}

}  // namespace orth
