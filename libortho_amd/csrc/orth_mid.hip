// Mid-size batches (5 <= M <= 16 tokens) of the dual GEMM for gfx950, in
// one launch.
//
// Same formula as /root/reference/src/dual_gemm.cu:176-225.  The decode
// kernel stages the activations once per 16-row block, which costs M*K*2
// bytes of L2 reads per block and outgrows the weight stream from a few
// tokens on; the split-K mid-batch kernel shares them over 128 rows but
// needs a second launch to add its partials.  Here each workgroup (4 waves,
// one per SIMD) owns a contiguous range of 16-row blocks, about nblocks /
// CUs of them, and all of K:
//
//  * Wave w takes K quarter w (chunks [8w, 8w + 8) of 128 columns) of every
//    block and stages that quarter of the activations (M tokens, padded to
//    8 or 16 with zeros) in LDS once for the whole launch, in the
//    interleaved k order of the weight conversion, then reads its MFMA A
//    operands (16 tokens x 32 k per instruction, 32 of them) into registers
//    for the whole launch: per block the LDS serves only the ortho term.
//    No barrier precedes the work: a wave reads only the activations it
//    staged.
//  * Per block, lane (row r = lane % 16, g = lane / 16) loads 16 bytes of
//    row r per chunk (nontemporal), converts each word to 8 exact FP16
//    integers (five bit operations and four packed subtracts) and feeds
//    v_mfma_f32_16x16x32_f16 as the B operand; each chunk's FP32 partial is
//    multiplied by its group scale.  (The biased conversion of the decode
//    kernel needs per-chunk activation sums, whose staging costs more here
//    than the subtracts: the activations are staged for 8 or 16 tokens.)
//  * Loads run one block ahead: while a wave consumes chunk pair j of block
//    b it issues pair j of block b + 1, whose plan record and scales it
//    issued first, so a CU's vector-memory queue always holds one block of
//    weights per wave and the record of a block arrives before its weights.
//  * Ortho term (alpha > 0): once the A operands are in registers, the
//    activations are rewritten over the same LDS column by column (the MT
//    tokens of a column contiguous, so an entry's activations are two
//    16-byte reads instead of MT 2-byte ones, which queued on the LDS
//    banks).  Each wave reads the plan record of (block, quarter) --
//    packed column|value words at an address that needs no other load --
//    stages it in its own LDS region and sums v*x over its entries, 4 lanes
//    per row (a batch's activation reads all issued before its products),
//    reduced over the quad with DPP moves.  A quarter whose entries did not
//    fit its record reads the rows' CSR, filtered to the quarter's columns.
//  * The four quarters' partials (dense and sparse) are added in quarter
//    order after a workgroup barrier (deterministic, no atomics), then
//    y = fp16(dense + alpha * sparse) (+ bias) for the block's 16 rows.
//    Where the LDS holds two sets, the partial and sum regions alternate
//    between blocks, so one barrier per block orders both their writes and
//    their reads (else a second barrier ends the block).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "orth_common.h"

namespace orth {

int plan_qrec_words(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip
int64_t plan_rec_at(int64_t N, int64_t K, int64_t nnz);

constexpr int kMidW = 4;  // waves per workgroup (the K quarters)
constexpr int kMidNT = 64 * kMidW;
constexpr int kMidCPW = 8;  // chunks per wave: K = 4096
static const int64_t kMidLdsMax = 160 * 1024;

struct MidArgs {
    const uint8_t *q;
    const f16 *scales;
    int ngroups;
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int32_t nnz;
    const f16 *x;
    f16 *y;
    int M;
    int K;
    int64_t N;
    int nchunks;       // K / 128
    int nblk;          // 16-row blocks
    int lds_xs, lds_red, lds_sp, lds_e;  // byte offsets of the LDS regions
    float alpha;
    const uint32_t *rec;  // plan quarter records: qwords words per (block, wave)
    int qwords;
    const void *bias;     // [N] added after rounding (out_f16), or null
    int bias_dtype;
};

// MT: tokens padded to 8 or 16.  GMODE: 1 G = 128 (a row's 8 scales of a
// wave's quarter as one aligned 16-byte vector), 4 one scale per row.
// SPARSE: 0 no ortho term; 3 / 4 / 5 / 6 plan records of 256 / 512 / <= 1024
// / <= 2048 words.  DB: the partial and sum regions alternate between
// iterations (one barrier per iteration; else two).  XB: BF16 activations
// and output (v_mfma_f32_16x16x32_bf16, the weights as the exact BF16
// integers q + 136; each chunk's 136 * sum x is removed with the chunk sums
// of the activations, formed once per launch by MFMAs against a ones
// operand).
template <int MT, int GMODE, int SPARSE, bool DB, bool XB>
__global__ void __launch_bounds__(kMidNT) __attribute__((amdgpu_waves_per_eu(1, 1))) mid_kernel(MidArgs a) {
    constexpr int W = kMidW;
    constexpr int CPW = kMidCPW;
    constexpr int XIT = CPW * 16 / 64;  // 16-byte activation pieces per lane per token
    constexpr int XS = 512 * CPW + 8;   // LDS row stride of the activations, in halves (+16 bytes:
                                        // rows start in different banks)
    constexpr bool REC = SPARSE >= 3;
    constexpr int ER = REC ? 1 << (SPARSE - 3) : 1;  // record: 16-byte loads per lane
    constexpr int RS = W * 256;        // floats of the dense partials [W][16 tokens][16 rows]
    constexpr int SS = W * MT * 16;    // floats of the sparse sums [W][MT][16 rows]
    static_assert(MT == 8 || MT == 16, "tokens padded to 8 or 16");
    static_assert(GMODE == 1 || GMODE == 4, "G = 128 vectors or per-row scales");
    static_assert(SPARSE == 0 || REC, "the ortho term comes from plan records");

    extern __shared__ __align__(16) unsigned char smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem + a.lds_xs);         // [MT][XS] activations
    float *red0 = reinterpret_cast<float *>(smem + a.lds_red);  // [DB ? 2 : 1] partials
    float *sp0 = reinterpret_cast<float *>(smem + a.lds_sp);    // [DB ? 2 : 1] sums

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = wave;        // K quarter
    const int lane = tid & 63;
    const int nl = lane & 15;  // B column (weight row) and A row (token) of this lane
    const int g = lane >> 4;   // which 32-k quarter of a chunk
    const int qr = lane >> 2, tg = lane & 3;  // sparse term: row of the block, lane of its quad
    const int K = a.K;
    const int c_lo = q * CPW;
    const int32_t col0 = c_lo * 128, col1 = col0 + CPW * 128;
    const int bb0 = (int)(((int64_t)blockIdx.x * a.nblk) / gridDim.x);
    const int bb1 = (int)(((int64_t)(blockIdx.x + 1) * a.nblk) / gridDim.x);
    if (bb0 >= bb1) return;  // (uniform; the host keeps grid <= nblk)
    const int nit = bb1 - bb0;

    // ---- activations of quarter q, all tokens (L2-resident): piece (m, it)
    //      of this lane is token m, columns col0 + 8 (lane + 64 it) .. + 8
    u32x4 xreg[MT][XIT];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int it = 0; it < XIT; it++)
            xreg[m][it] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)min(m, a.M - 1) * K + col0 + (lane + 64 * it) * 8);

    // ---- per-block loads: record, scales, weights (in that order)
    auto last_row_of = [&](int b) -> int {
        const int64_t rows = a.N - (int64_t)b * 16;
        return rows < 16 ? (int)rows - 1 : 15;
    };
    u32x4 rv[ER];
    auto load_rec = [&](int b) {
        if (REC) {
            const uint32_t *rb = a.rec + ((int64_t)b * W + q) * a.qwords;
#pragma unroll
            for (int r = 0; r < ER; r++)
                rv[r] = *reinterpret_cast<const u32x4 *>(rb + min(4 * (lane + 64 * r), a.qwords - 4));
        }
    };
    auto load_scales = [&](int b) -> u32x4 {
        if (GMODE == 1) {
            const int64_t row = (int64_t)b * 16 + min(nl, last_row_of(b));
            return *reinterpret_cast<const u32x4 *>(a.scales + row * a.ngroups + c_lo);
        }
        return u32x4{0u, 0u, 0u, 0u};
    };
    auto qrow_of = [&](int b) -> const uint8_t * {
        const int64_t row = (int64_t)b * 16 + min(nl, last_row_of(b));
        return a.q + row * (int64_t)(K >> 1) + col0 / 2 + g * 16;
    };
    u32x4 wv[CPW];
    auto load_chunk = [&](const uint8_t *qrow, int p) {
        wv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + p * 64));
    };

    load_rec(bb0);
    u32x4 sv = load_scales(bb0);
    {
        const uint8_t *q0 = qrow_of(bb0);
#pragma unroll
        for (int p = 0; p < CPW; p++) load_chunk(q0, p);
    }

    // ---- stage the activations token by token (interleaved k order), then
    //      read this lane's MFMA A operands for the whole launch (16 tokens x
    //      32 k per instruction, token nl mod MT): the activations are read
    //      from LDS once, not once per block (a wave reads only what it
    //      staged: LDS keeps the wave's order, no barrier)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int it = 0; it < XIT; it++) {
            if (m >= a.M) xreg[m][it] = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4 *>(xs + (m * XS + col0 + (lane + 64 * it) * 8)) = permute_x8(xreg[m][it]);
        }
    u32x4 afr[CPW][4];
    {
        const f16 *xs_lane = xs + ((nl & (MT - 1)) * XS + g * 32 + col0);
#pragma unroll
        for (int p = 0; p < CPW; p++)
#pragma unroll
            for (int k = 0; k < 4; k++) afr[p][k] = *reinterpret_cast<const u32x4 *>(xs_lane + (p * 128 + 8 * k));
    }
    // XB: chunk p's activation sums, in the MFMA output layout (token
    // 4 g + i of this lane), against a ones B operand
    f32x4 xsum[XB ? CPW : 1];
    if constexpr (XB) {
        const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
#pragma unroll
        for (int p = 0; p < CPW; p++) {
            f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; k++)
                t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, afr[p][k]),
                                                            __builtin_bit_cast(bf16x8, ones), t, 0, 0, 0);
            xsum[p] = t;
        }
    }
    // ---- then, over the same LDS, column by column for the ortho term: the
    //      MT tokens of column c contiguous (two 16-byte reads per entry
    //      instead of MT 2-byte ones), 16 bytes of padding after every 8
    //      columns so that the lanes' writes (8 columns apart) spread over
    //      the banks.  Built from the staging registers (each lane holds all
    //      tokens of its 8-column pieces); the barrier first lets every wave
    //      finish reading its A operands.
    f16 *xt = xs;
    auto xt_col = [&](int c) -> f16 * { return xt + c * MT + (c >> 3) * 8; };
    if (REC) __syncthreads();
#pragma unroll
    for (int it = 0; it < (REC ? XIT : 0); it++) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t w[MT / 2];  // tokens 2t, 2t + 1 of column j of the piece
#pragma unroll
            for (int t = 0; t < MT / 2; t++)
                w[t] = __builtin_amdgcn_perm(xreg[2 * t + 1][it][j >> 1], xreg[2 * t][it][j >> 1],
                                             (j & 1) ? 0x07060302u : 0x05040100u);
            f16 *dst = xt_col(col0 + 8 * (lane + 64 * it) + j);
#pragma unroll
            for (int v = 0; v < MT / 8; v++)
                *reinterpret_cast<u32x4 *>(dst + 8 * v) = u32x4{w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]};
        }
    }
    uint32_t *er = reinterpret_cast<uint32_t *>(smem + a.lds_e) + wave * a.qwords;

    // iteration i: block bb0 + i; MORE: issue the next block's loads as this
    // one's are consumed
    auto iteration = [&](int i, auto more_c) {
        constexpr bool MORE = decltype(more_c)::value;
        const int b = bb0 + i;
        const int64_t n0 = (int64_t)b * 16;
        const int last_row = last_row_of(b);
        float *red = red0 + (DB ? (i & 1) : 0) * RS;
        float *sp = sp0 + (DB ? (i & 1) : 0) * SS;

        // ---- the record to this wave's LDS region; then the next block's
        //      record and scales are issued (ahead of its weights)
        if (REC) {
#pragma unroll
            for (int r = 0; r < ER; r++) {
                const int o = 4 * (lane + 64 * r);
                if (o < a.qwords) *reinterpret_cast<u32x4 *>(er + o) = rv[r];
            }
            __builtin_amdgcn_wave_barrier();  // (same wave: LDS keeps the order)
        }
        u32x4 sv_next = sv;
        const uint8_t *qnext = nullptr;
        if (MORE) {
            load_rec(b + 1);
            sv_next = load_scales(b + 1);
            qnext = qrow_of(b + 1);
        }

        // ---- dense term, one chunk pair (the two MFMA chains interleaved),
        //      issuing the next block's weights of the pair as it goes
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        auto dense_pair = [&](int j) {
            const u32x4 w0 = wv[2 * j], w1 = wv[2 * j + 1];
            if (MORE) {
                load_chunk(qnext, 2 * j);
                load_chunk(qnext, 2 * j + 1);
            }
            const uint32_t u0[4] = {w0.x, w0.y, w0.z, w0.w};
            const uint32_t u1[4] = {w1.x, w1.y, w1.z, w1.w};
            f32x4 pa = f32x4{0.f, 0.f, 0.f, 0.f}, pb = pa;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t b0[4], b1[4];
                if constexpr (XB) {
                    int4x8_to_bf16_biased(u0[k], b0);
                    int4x8_to_bf16_biased(u1[k], b1);
                    pa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, afr[2 * j][k]),
                                                                 __builtin_bit_cast(bf16x8, u32x4{b0[0], b0[1], b0[2], b0[3]}),
                                                                 pa, 0, 0, 0);
                    pb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, afr[2 * j + 1][k]),
                                                                 __builtin_bit_cast(bf16x8, u32x4{b1[0], b1[1], b1[2], b1[3]}),
                                                                 pb, 0, 0, 0);
                } else {
                    int4x8_to_f16_interleaved(u0[k], b0);
                    int4x8_to_f16_interleaved(u1[k], b1);
                    pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, afr[2 * j][k]),
                                                                __builtin_bit_cast(f16x8, u32x4{b0[0], b0[1], b0[2], b0[3]}),
                                                                pa, 0, 0, 0);
                    pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, afr[2 * j + 1][k]),
                                                                __builtin_bit_cast(f16x8, u32x4{b1[0], b1[1], b1[2], b1[3]}),
                                                                pb, 0, 0, 0);
                }
            }
            if constexpr (XB) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    pa[k] -= 136.0f * xsum[2 * j][k];
                    pb[k] -= 136.0f * xsum[2 * j + 1][k];
                }
            }
            float s0 = 1.0f, s1 = 1.0f;
            if (GMODE == 1) {
                const uint32_t s2 = sv[j];  // the scales of chunks 2j, 2j + 1 of row nl
                s0 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 & 0xffffu));
                s1 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 >> 16));
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc[k] += s0 * pa[k];
                acc[k] += s1 * pb[k];
            }
        };
        static_assert(CPW == 8, "four chunk pairs per block");
        if constexpr (!REC) {
#pragma unroll
            for (int j = 0; j < CPW / 2; j++) dense_pair(j);
        } else {
            // ---- ortho sums of this quarter, 4 lanes per row (entries
            //      start + tg + 4u in order), reduced over the quad.  The
            //      first two batches of 4 entries per lane are interleaved
            //      with the dense pairs, so that their LDS round trips (the
            //      record words, then the activations they address) overlap
            //      the matrix work: the wave is alone on its SIMD and would
            //      otherwise wait for each round trip.  The dense pairs stay
            //      outside any branch (their weight loads too); a record that
            //      does not hold all the block's entries (ok false) leaves
            //      the batches empty and the rows are read from the CSR after.
            float sacc[MT];
#pragma unroll
            for (int m = 0; m < MT; m++) sacc[m] = 0.f;
            const bool ok = (er[0] == plan_cell_tag(kCellQuarter, a.N, K, a.nnz, a.qwords, b, q)) &
                            (er[1] == 0u);  // (uniform)
            const uint32_t hw = er[2 + qr];
            const int32_t lo = ok ? (int32_t)(hw & 0xffffu) : 0;
            const int32_t hi = ok && qr <= last_row ? (int32_t)(hw >> 16) : lo;
            const uint32_t *ee = er + kCellHdrWords;
            constexpr int U = 4;
            uint32_t w[2][U];
            f16x8 xh[U][MT / 8];
            float ve[U];
            auto rec_reads = [&](int k) {
#pragma unroll
                for (int u = 0; u < U; u++) w[k][u] = ee[max(min(lo + tg + 16 * k + 4 * u, hi - 1), 0)];
            };
            auto x_reads = [&](int k) {
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const bool ok_e = lo + tg + 16 * k + 4 * u < hi;
                    const int cc = ok_e ? (int)(w[k][u] & 0xffffu) + col0 : col0;
                    ve[u] = ok_e ? (float)__builtin_bit_cast(f16, (uint16_t)(w[k][u] >> 16)) : 0.f;
                    const f16 *xc = xt_col(cc);
#pragma unroll
                    for (int v = 0; v < MT / 8; v++) xh[u][v] = *reinterpret_cast<const f16x8 *>(xc + 8 * v);
                }
            };
            auto fmas = [&]() {
#pragma unroll
                for (int u = 0; u < U; u++)
#pragma unroll
                    for (int m = 0; m < MT; m++)
                        sacc[m] = __builtin_fmaf(ve[u], x16_to_f32<XB>(xh[u][m >> 3][m & 7]), sacc[m]);
            };
            rec_reads(0);
            rec_reads(1);
            __builtin_amdgcn_sched_barrier(0);
            dense_pair(0);
            __builtin_amdgcn_sched_barrier(0);
            x_reads(0);
            __builtin_amdgcn_sched_barrier(0);
            dense_pair(1);
            __builtin_amdgcn_sched_barrier(0);
            fmas();
            x_reads(1);
            __builtin_amdgcn_sched_barrier(0);
            dense_pair(2);
            __builtin_amdgcn_sched_barrier(0);
            fmas();
            __builtin_amdgcn_sched_barrier(0);
            dense_pair(3);
            if (ok) {
                // entries past the first two batches (rows with more than 8
                // entries in the quarter per lane of the quad)
                for (int32_t j0 = lo + tg + 32; j0 < hi; j0 += 4 * U) {
                    uint32_t wr[U];
#pragma unroll
                    for (int u = 0; u < U; u++) wr[u] = ee[min(j0 + 4 * u, hi - 1)];
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const bool ok_e = j0 + 4 * u < hi;
                        const int cc = ok_e ? (int)(wr[u] & 0xffffu) + col0 : col0;
                        ve[u] = ok_e ? (float)__builtin_bit_cast(f16, (uint16_t)(wr[u] >> 16)) : 0.f;
                        const f16 *xc = xt_col(cc);
#pragma unroll
                        for (int v = 0; v < MT / 8; v++) xh[u][v] = *reinterpret_cast<const f16x8 *>(xc + 8 * v);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    fmas();
                }
            } else {
                int32_t fs = 0, fe = 0;
                csr_row_range(a.row_ptr, n0 + min(qr, last_row), a.nnz, fs, fe);
                if (qr > last_row) fe = fs;
                for (int32_t j = fs + tg; j < fe; j += 4) {
                    const int32_t c = a.col[j];
                    const bool ok_e = c >= col0 && c < col1;
                    const f16 *xc = xt_col(ok_e ? c : col0);
                    const float vv = ok_e ? (float)a.vals[j] : 0.f;
#pragma unroll
                    for (int m = 0; m < MT; m++) sacc[m] = __builtin_fmaf(vv, x16_to_f32<XB>(xc[m]), sacc[m]);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; m++) {
                float v = sacc[m];
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
                sacc[m] = v;
            }
            if (tg == 0) {
#pragma unroll
                for (int m = 0; m < MT; m++) sp[(q * MT + m) * 16 + qr] = sacc[m];
            }
        }

        sv = sv_next;

        // ---- the four quarters in order, scaled (GMODE 4), plus alpha * sparse
#pragma unroll
        for (int k = 0; k < 4; k++) red[(q * 16 + 4 * g + k) * 16 + nl] = acc[k];
        __syncthreads();
        if (tid < MT * 16) {
            const int m = tid >> 4, r = tid & 15;
            const int64_t n = n0 + r;
            if (m < a.M && r <= last_row) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < W; w++) v += red[(w * 16 + m) * 16 + r];
                if (GMODE == 4) v *= (float)a.scales[n];
                if (REC) {
                    float s = 0.f;
#pragma unroll
                    for (int w = 0; w < W; w++) s += sp[(w * MT + m) * 16 + r];
                    v += a.alpha * s;
                }
                if constexpr (XB)
                    reinterpret_cast<uint16_t *>(a.y)[(int64_t)m * a.N + n] = out_bf16(v, a.bias, a.bias_dtype, n);
                else
                    a.y[(int64_t)m * a.N + n] = out_f16(v, a.bias, a.bias_dtype, n);
            }
        }
        if (!DB) __syncthreads();  // the regions are rewritten in the next iteration
    };
    for (int i = 0; i < nit - 1; i++) iteration(i, std::integral_constant<bool, true>{});
    iteration(nit - 1, std::integral_constant<bool, false>{});
}

// ------------------------------------------------------------------ host

struct MidShape {
    int mt, gmode, sparse, lds, grid;
    bool db;  // alternating partial and sum regions
    bool xb;  // BF16 activations and output
};

static bool mid_shape(const ForwardArgs &a, const void *plan, int cus, MidArgs *d, MidShape &sh) {
    // FP16: 5..16 tokens (the decode kernel takes fewer); BF16: 1..16 (the
    // decode kernel is FP16 only)
    sh.xb = a.io_dtype == ORTH_DT_BF16;
    if (a.M > 16 || a.M < (sh.xb ? 1 : 5)) return false;
    if ((a.io_dtype != ORTH_DT_F16 && !sh.xb) || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.K != 512 * kMidCPW) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    if (a.N > ((int64_t)1 << 31) || a.N < 1) return false;
    if (a.ngroups == 1) sh.gmode = 4;
    else if (a.G == 128 && (reinterpret_cast<uintptr_t>(a.scales) & 15) == 0) sh.gmode = 1;
    else return false;
    sh.sparse = 0;
    int qwords = 0;
    if (a.has_ortho) {
        // the ortho term comes from the plan's quarter records
        if (!plan || a.val_dtype != ORTH_DT_F16) return false;
        qwords = plan_qrec_words(a.N, a.K, a.nnz);
        if (qwords <= 0 || decode_chunks_per_wave(a.K) != kMidCPW) return false;
        sh.sparse = qwords == 256 ? 3 : qwords == 512 ? 4 : qwords <= 1024 ? 5 : 6;
    }
    sh.mt = a.M <= 8 ? 8 : 16;
    const int nchunks = (int)(a.K / 128);
    const int xstride = (int)(a.K + 8);  // the kernel's XS
    auto al = [](int64_t v) { return (v + 15) & ~int64_t(15); };
    // activations, then per (buffer, group) the quarters' partials and
    // sums, then one record region per wave; alternating buffers when the
    // LDS holds them
    int64_t lds_xs = 0, lds_red = 0, lds_sp = 0, lds_e = 0, off = 0;
    for (int nbuf = 2; nbuf >= 1; nbuf--) {
        off = 0;
        lds_xs = off;
        // row-major activations, then the column-major copy over them
        const int64_t xt_bytes = (int64_t)a.K * sh.mt * 2 + (a.K / 8) * 16;
        off = al(off + std::max<int64_t>((int64_t)sh.mt * xstride * 2, xt_bytes));
        lds_red = off;
        off += (int64_t)nbuf * kMidW * 256 * 4;
        lds_sp = off;
        off += (int64_t)nbuf * kMidW * sh.mt * 16 * 4;
        lds_e = off;
        off += (int64_t)kMidW * qwords * 4;
        sh.db = nbuf == 2;
        if (off <= kMidLdsMax) break;
    }
    if (off > kMidLdsMax) return false;
    sh.lds = (int)off;
    const int64_t nblk = (a.N + 15) / 16;
    // one workgroup per CU, blocks dealt evenly
    sh.grid = (int)std::min<int64_t>(nblk, (int64_t)cus);
    if (d) {
        d->q = a.q;
        d->scales = static_cast<const f16 *>(a.scales);
        d->ngroups = (int)a.ngroups;
        d->row_ptr = a.row_ptr;
        d->col = a.col;
        d->vals = static_cast<const f16 *>(a.vals);
        d->nnz = (int32_t)a.nnz;
        d->x = static_cast<const f16 *>(a.x);
        d->y = static_cast<f16 *>(a.y);
        d->M = (int)a.M;
        d->K = (int)a.K;
        d->N = a.N;
        d->nchunks = nchunks;
        d->nblk = (int)nblk;
        d->lds_xs = (int)lds_xs;
        d->lds_red = (int)lds_red;
        d->lds_sp = (int)lds_sp;
        d->lds_e = (int)lds_e;
        d->alpha = a.alpha;
        d->rec = sh.sparse ? reinterpret_cast<const uint32_t *>(static_cast<const char *>(plan) +
                                                                plan_rec_at(a.N, a.K, a.nnz))
                           : nullptr;
        d->qwords = qwords;
        d->bias = a.bias;
        d->bias_dtype = a.bias_dtype;
    }
    return true;
}

// Whether the mid-batch kernel takes this call (with this plan or none).
bool mid_supported(const ForwardArgs &a, const void *plan) {
    MidShape sh;
    return mid_shape(a, plan, 256, nullptr, sh);
}

template <int MT, int GMODE, int SPARSE, bool DB, bool XB>
static hipError_t mid_launch_t(const MidArgs &d, const MidShape &sh, hipStream_t s) {
    // more than 64 KB of dynamic LDS must be allowed once per device (the
    // attribute call is idempotent, so two threads racing to set it is harmless)
    static std::atomic<int> allowed[64];
    int dev = 0;
    if (sh.lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 &&
        !allowed[dev].load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(mid_kernel<MT, GMODE, SPARSE, DB, XB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMidLdsMax);
        if (e != hipSuccess) return e;
        allowed[dev].store(1, std::memory_order_release);
    }
    hipLaunchKernelGGL((mid_kernel<MT, GMODE, SPARSE, DB, XB>), dim3((unsigned)sh.grid), dim3(kMidNT), (uint32_t)sh.lds,
                       s, d);
    return hipGetLastError();
}

template <int MT, int GMODE, bool DB, bool XB>
static hipError_t mid_launch_s(const MidArgs &d, const MidShape &sh, hipStream_t s) {
    switch (sh.sparse) {
        case 3: return mid_launch_t<MT, GMODE, 3, DB, XB>(d, sh, s);
        case 4: return mid_launch_t<MT, GMODE, 4, DB, XB>(d, sh, s);
        case 5: return mid_launch_t<MT, GMODE, 5, DB, XB>(d, sh, s);
        case 6:
            // 16 tokens: the activations leave no LDS for records of 2048
            // words (mid_shape refuses them)
            if constexpr (MT == 8) return mid_launch_t<MT, GMODE, 6, DB, XB>(d, sh, s);
            return hipErrorInvalidValue;
        default: return mid_launch_t<MT, GMODE, 0, DB, XB>(d, sh, s);
    }
}

template <int MT, int GMODE, bool XB>
static hipError_t mid_launch_b(const MidArgs &d, const MidShape &sh, hipStream_t s) {
    return sh.db ? mid_launch_s<MT, GMODE, true, XB>(d, sh, s) : mid_launch_s<MT, GMODE, false, XB>(d, sh, s);
}

template <bool XB>
static hipError_t mid_launch_x(const MidArgs &d, const MidShape &sh, hipStream_t s) {
    if (sh.mt == 8) return sh.gmode == 1 ? mid_launch_b<8, 1, XB>(d, sh, s) : mid_launch_b<8, 4, XB>(d, sh, s);
    return sh.gmode == 1 ? mid_launch_b<16, 1, XB>(d, sh, s) : mid_launch_b<16, 4, XB>(d, sh, s);
}

// plan: the layer's ortho plan (required when the ortho term is on).
hipError_t launch_mid(const ForwardArgs &a, const void *plan, int cus, hipStream_t stream) {
    MidArgs d;
    MidShape sh;
    if (!mid_shape(a, plan, cus, &d, sh)) return hipErrorInvalidValue;
    return sh.xb ? mid_launch_x<true>(d, sh, stream) : mid_launch_x<false>(d, sh, stream);
}

}  // namespace orth
