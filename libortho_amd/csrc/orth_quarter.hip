// 17..32 tokens of the dual GEMM for gfx950, K = 4096: K split in quarters
// over the grid, partials added by a second launch.
//
// Same formula as /root/reference/src/dual_gemm.cu:176-225.  With 32 tokens
// the activations of all of K are 256 KB, more than one workgroup can stage
// per CU cheaply, so each workgroup takes one K quarter (1024 columns, the
// decode kernel's quarter and the ortho plan's record cell) of a range of
// 16-row blocks:
//
//  * The workgroup (4 waves, one per SIMD) stages its quarter of the
//    activations once, 64 KB for 32 tokens (padded with zeros past M), twice
//    over: row-major in the interleaved k order of the weight conversion,
//    from which every wave reads its MFMA A operands (two 16-token tiles x 8
//    chunks x 4 k steps) into registers for the whole launch, and column by
//    column (a column's 32 tokens contiguous) for the ortho gather.
//  * Wave w takes the workgroup's blocks w, w + 4, ...; per block, lane (row
//    r = lane % 16, g = lane / 16) loads 16 bytes of row r per chunk
//    (nontemporal), converts each word to 8 exact FP16 integers and feeds
//    v_mfma_f32_16x16x32_f16 for both token tiles; each chunk's FP32 partial
//    is multiplied by its group scale.  (BF16 activations: the exact BF16
//    integers q + 136 into v_mfma_f32_16x16x32_bf16, less 136 times the
//    chunk's activation sum per token, formed once at staging.)  Loads run one block ahead (record,
//    scales, then weights, issued as the previous block's are consumed).
//  * Ortho term (alpha > 0): the plan record of (block, quarter) is staged in
//    the wave's own LDS region and v*x summed over its entries, 4 lanes per
//    row (an entry's 32 activations are four 16-byte reads), reduced over
//    the quad with DPP moves and handed to the MFMA lanes through a
//    wave-private LDS region.  A quarter whose entries did not fit its
//    record reads the rows' CSR, filtered to the quarter's columns.
//  * Each wave stores its blocks' FP32 partials dense + alpha * sparse (per
//    row scale applied) to part[quarter][m][n]; no workgroup barrier after
//    the staging.  quarter_reduce_kernel adds the four quarters in order
//    (deterministic) and rounds to FP16 (+ bias).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "orth_common.h"

namespace orth {

int plan_qrec_words(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip
int64_t plan_rec_at(int64_t N, int64_t K, int64_t nnz);

constexpr int kQuW = 4;           // waves per workgroup
constexpr int kQuNT = 64 * kQuW;
constexpr int kQuCPW = 8;         // chunks per quarter: K = 4096
constexpr int kQuMT = 32;         // tokens (two MFMA tiles)
constexpr int kQuWGs = 64;        // workgroups per quarter (4 * 64 = 256 = CUs)
static const int64_t kQuLdsMax = 160 * 1024;

struct QuarterArgs {
    const uint8_t *q;
    const f16 *scales;
    int ngroups;
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int32_t nnz;
    const f16 *x;
    float *part;       // [4][M][N]
    int M;
    int K;
    int64_t N;
    int nblk;          // 16-row blocks
    int gq;            // workgroups per quarter
    int lds_xt, lds_e, lds_ex;  // byte offsets of the LDS regions (activations at 0)
    int lds_xsum;               // BF16: [CPW chunks][MT tokens] 136 * sum of the chunk's activations
    float alpha;
    const uint32_t *rec;  // plan quarter records: qwords words per (block, quarter)
    int qwords;
};

// GMODE: 1 G = 128 (a row's 8 scales of the quarter as one aligned 16-byte
// vector), 4 one scale per row.  SPARSE: 0 no ortho term; 3 / 4 / 5 plan
// records of 256 / 512 / <= 1024 words.  XB: BF16 activations and output:
// the weights become the exact BF16 integers q + 136, and each chunk's
// partial loses 136 * (the chunk's activation sum), formed once at staging.
template <int GMODE, int SPARSE, bool XB>
__global__ void __launch_bounds__(kQuNT) __attribute__((amdgpu_waves_per_eu(1, 1))) quarter_kernel(QuarterArgs a) {
    constexpr int MT = kQuMT;
    constexpr int CPW = kQuCPW;
    constexpr int XS = 128 * CPW + 8;  // LDS row stride of the row-major activations, in halves
    constexpr bool REC = SPARSE >= 3;
    constexpr int ER = REC ? 1 << (SPARSE - 3) : 1;  // record: 16-byte loads per lane
    static_assert(GMODE == 1 || GMODE == 4, "G = 128 vectors or per-row scales");
    static_assert(SPARSE == 0 || REC, "the ortho term comes from plan records");

    extern __shared__ __align__(16) unsigned char smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem);                 // [MT][XS] row-major, interleaved k order
    f16 *xt = reinterpret_cast<f16 *>(smem + a.lds_xt);      // column-major, see xt_col

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int nl = lane & 15;  // B column (weight row) and A row (token within a tile) of this lane
    const int g = lane >> 4;   // which 32-k quarter of a chunk
    const int qr = lane >> 2, tg = lane & 3;  // sparse term: row of the block, lane of its quad
    const int K = a.K;
    const int qq = (int)(blockIdx.x & 3);     // K quarter
    const int wg = (int)(blockIdx.x >> 2);    // workgroup within the quarter
    const int c_lo = qq * CPW;
    const int32_t col0 = c_lo * 128;
    const int bb0 = (int)(((int64_t)wg * a.nblk) / a.gq);
    const int bb1 = (int)(((int64_t)(wg + 1) * a.nblk) / a.gq);
    // this wave's blocks: bb0 + wave + 4 i; a wave with none repeats the
    // workgroup's last block's loads and stores nothing
    const int nit = bb1 - bb0 > wave ? (bb1 - bb0 - wave + 3) / 4 : 0;
    auto block_of = [&](int i) { return min(bb0 + wave + 4 * i, bb1 - 1); };

    // ---- activations: wave w stages columns [256 w, 256 w + 256) of the
    //      quarter; lane l takes the 8 columns 8 (l % 32) .. and the 16
    //      tokens 16 (l / 32) ..
    const int cg = lane & 31, th = (lane >> 5) * 16;
    const int cl0 = 256 * wave + 8 * cg;  // first column of the lane's group, quarter-local
    u32x4 xreg[16];
#pragma unroll
    for (int t = 0; t < 16; t++)
        xreg[t] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)min(th + t, a.M - 1) * K + col0 + cl0);

    // ---- per-block loads: record, scales, weights (in that order)
    auto last_row_of = [&](int b) -> int {
        const int64_t rows = a.N - (int64_t)b * 16;
        return rows < 16 ? (int)rows - 1 : 15;
    };
    u32x4 rv[ER];
    auto load_rec = [&](int b) {
        if (REC) {
            const uint32_t *rb = a.rec + ((int64_t)b * 4 + qq) * a.qwords;
#pragma unroll
            for (int r = 0; r < ER; r++)
                rv[r] = *reinterpret_cast<const u32x4 *>(rb + min(4 * (lane + 64 * r), a.qwords - 4));
        }
    };
    auto load_scales = [&](int b) -> u32x4 {
        const int64_t row = (int64_t)b * 16 + min(nl, last_row_of(b));
        if (GMODE == 1) return *reinterpret_cast<const u32x4 *>(a.scales + row * a.ngroups + c_lo);
        const f16 s = a.scales[row];
        return u32x4{(uint32_t)__builtin_bit_cast(uint16_t, s), 0u, 0u, 0u};
    };
    auto qrow_of = [&](int b) -> const uint8_t * {
        const int64_t row = (int64_t)b * 16 + min(nl, last_row_of(b));
        return a.q + row * (int64_t)(K >> 1) + col0 / 2 + g * 16;
    };
    u32x4 wv[CPW];
    auto load_chunk = [&](const uint8_t *qrow, int p) {
        wv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + p * 64));
    };
    load_rec(block_of(0));
    u32x4 sv = load_scales(block_of(0));
    {
        const uint8_t *q0 = qrow_of(block_of(0));
#pragma unroll
        for (int p = 0; p < CPW; p++) load_chunk(q0, p);
    }

    // ---- stage: row-major (interleaved k order) and column-major (the MT
    //      tokens of column c contiguous, 16 bytes of padding after every 8
    //      columns so that the lanes' writes spread over the banks)
    auto xt_col = [&](int c) -> f16 * { return xt + c * MT + (c >> 3) * 8; };
#pragma unroll
    for (int t = 0; t < 16; t++) {
        if (th + t >= a.M) xreg[t] = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4 *>(xs + ((th + t) * XS + cl0)) = permute_x8(xreg[t]);
    }
    if constexpr (XB) {
        // 136 * sum over the 128 columns of chunk cl0 / 128 (16 lanes of 8),
        // per token: the bias the q + 136 weights add to every output row
        float *xsum = reinterpret_cast<float *>(smem + a.lds_xsum);
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const uint32_t w[4] = {xreg[t].x, xreg[t].y, xreg[t].z, xreg[t].w};
            float v = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++)
                v += bf16_bits_to_f32((uint16_t)(w[e] & 0xffffu)) + bf16_bits_to_f32((uint16_t)(w[e] >> 16));
            v = group_sum<16>(v);
            if ((cg & 15) == 0) xsum[(cl0 >> 7) * MT + th + t] = 136.0f * v;
        }
    }
    if (REC) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t w[8];  // tokens th + 2u, th + 2u + 1 of column cl0 + j
#pragma unroll
            for (int u = 0; u < 8; u++)
                w[u] = __builtin_amdgcn_perm(xreg[2 * u + 1][j >> 1], xreg[2 * u][j >> 1],
                                             (j & 1) ? 0x07060302u : 0x05040100u);
            f16 *dst = xt_col(cl0 + j) + th;
            *reinterpret_cast<u32x4 *>(dst) = u32x4{w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u32x4 *>(dst + 8) = u32x4{w[4], w[5], w[6], w[7]};
        }
    }
    __syncthreads();  // every wave's columns are in LDS

    // ---- this lane's MFMA A operands for the whole launch: tile t, token
    //      16 t + nl, chunk p, k step kk
    u32x4 afr[2][CPW][4];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const f16 *xl = xs + ((16 * t + nl) * XS + g * 32);
#pragma unroll
        for (int p = 0; p < CPW; p++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) afr[t][p][kk] = *reinterpret_cast<const u32x4 *>(xl + (p * 128 + 8 * kk));
    }
    uint32_t *er = reinterpret_cast<uint32_t *>(smem + a.lds_e) + wave * a.qwords;
    float *ex = reinterpret_cast<float *>(smem + a.lds_ex) + wave * (16 * MT);  // [16 rows][MT] sparse sums

    // iteration i: block block_of(i); MORE: issue the next block's loads as
    // this one's are consumed
    auto iteration = [&](int i, auto more_c) {
        constexpr bool MORE = decltype(more_c)::value;
        const int b = block_of(i);
        const int64_t n0 = (int64_t)b * 16;
        const int last_row = last_row_of(b);

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
            load_rec(block_of(i + 1));
            sv_next = load_scales(block_of(i + 1));
            qnext = qrow_of(block_of(i + 1));
        }

        // ---- sparse sums of this quarter: 4 lanes per row, entries
        //      start + tg + 4u in order, reduced over the quad
        if (REC) {
            float sacc[MT];
#pragma unroll
            for (int m = 0; m < MT; m++) sacc[m] = 0.f;
            const bool ok = (er[0] == plan_cell_tag(kCellQuarter, a.N, K, a.nnz, a.qwords, b, qq)) &
                            (er[1] == 0u);  // (uniform)
            if (ok) {
                const uint32_t hw = er[2 + qr];
                const int32_t lo = (int32_t)(hw & 0xffffu);
                const int32_t hi = qr <= last_row ? (int32_t)(hw >> 16) : lo;
                const uint32_t *ee = er + kCellHdrWords;
                constexpr int U = 2;
                for (int32_t j0 = lo + tg; j0 < hi; j0 += 4 * U) {
                    uint32_t w[U];
#pragma unroll
                    for (int u = 0; u < U; u++) w[u] = ee[min(j0 + 4 * u, hi - 1)];
                    // all activation reads of the batch, then the products
                    f16x8 xh[U][MT / 8];
                    float ve[U];
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const bool ok_e = j0 + 4 * u < hi;
                        const int cc = ok_e ? (int)(w[u] & 0xffffu) : 0;
                        ve[u] = ok_e ? (float)__builtin_bit_cast(f16, (uint16_t)(w[u] >> 16)) : 0.f;
                        const f16 *xc = xt_col(cc);
#pragma unroll
                        for (int v = 0; v < MT / 8; v++) xh[u][v] = *reinterpret_cast<const f16x8 *>(xc + 8 * v);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int u = 0; u < U; u++)
#pragma unroll
                        for (int m = 0; m < MT; m++)
                            sacc[m] = __builtin_fmaf(ve[u], x16_to_f32<XB>(xh[u][m >> 3][m & 7]), sacc[m]);
                }
            } else {
                int32_t fs = 0, fe = 0;
                csr_row_range(a.row_ptr, n0 + min(qr, last_row), a.nnz, fs, fe);
                if (qr > last_row) fe = fs;
                for (int32_t j = fs + tg; j < fe; j += 4) {
                    const int32_t c = a.col[j] - col0;
                    const bool ok_e = c >= 0 && c < CPW * 128;
                    const f16 *xc = xt_col(ok_e ? c : 0);
                    const float ve = ok_e ? (float)a.vals[j] : 0.f;
#pragma unroll
                    for (int m = 0; m < MT; m++) sacc[m] = __builtin_fmaf(ve, x16_to_f32<XB>(xc[m]), sacc[m]);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; m++) {
                float v = sacc[m];
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
                sacc[m] = v;
            }
            __builtin_amdgcn_wave_barrier();  // the previous block's sums were read
            if (tg == 0) {
#pragma unroll
                for (int m = 0; m < MT; m += 4)
                    *reinterpret_cast<f32x4 *>(ex + qr * MT + m) = f32x4{sacc[m], sacc[m + 1], sacc[m + 2], sacc[m + 3]};
            }
            __builtin_amdgcn_wave_barrier();  // (same wave: LDS keeps the order)
        }

        // ---- dense term: chunk pairs, both token tiles
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int j = 0; j < CPW / 2; j++) {
            const u32x4 w0 = wv[2 * j], w1 = wv[2 * j + 1];
            if (MORE) {
                load_chunk(qnext, 2 * j);
                load_chunk(qnext, 2 * j + 1);
            }
            const uint32_t u0[4] = {w0.x, w0.y, w0.z, w0.w};
            const uint32_t u1[4] = {w1.x, w1.y, w1.z, w1.w};
            f32x4 pa[2], pb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) pa[t] = pb[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                uint32_t b0[4], b1[4];
                if constexpr (XB) {
                    int4x8_to_bf16_biased(u0[kk], b0);
                    int4x8_to_bf16_biased(u1[kk], b1);
                    const bf16x8 bf0 = __builtin_bit_cast(bf16x8, u32x4{b0[0], b0[1], b0[2], b0[3]});
                    const bf16x8 bf1 = __builtin_bit_cast(bf16x8, u32x4{b1[0], b1[1], b1[2], b1[3]});
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        pa[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, afr[t][2 * j][kk]),
                                                                        bf0, pa[t], 0, 0, 0);
                        pb[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, afr[t][2 * j + 1][kk]),
                                                                        bf1, pb[t], 0, 0, 0);
                    }
                } else {
                    int4x8_to_f16_interleaved(u0[kk], b0);
                    int4x8_to_f16_interleaved(u1[kk], b1);
                    const f16x8 bf0 = __builtin_bit_cast(f16x8, u32x4{b0[0], b0[1], b0[2], b0[3]});
                    const f16x8 bf1 = __builtin_bit_cast(f16x8, u32x4{b1[0], b1[1], b1[2], b1[3]});
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        pa[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, afr[t][2 * j][kk]),
                                                                       bf0, pa[t], 0, 0, 0);
                        pb[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, afr[t][2 * j + 1][kk]),
                                                                       bf1, pb[t], 0, 0, 0);
                    }
                }
            }
            float s0 = 1.0f, s1 = 1.0f;
            if (GMODE == 1) {
                const uint32_t s2 = sv[j];  // the scales of chunks 2j, 2j + 1 of row nl
                s0 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 & 0xffffu));
                s1 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 >> 16));
            }
            if constexpr (XB) {
                // D[token 16 t + 4 g + k]: remove 136 * (the chunk's activation sum)
                const float *xsum = reinterpret_cast<const float *>(smem + a.lds_xsum);
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const f32x4 ca = *reinterpret_cast<const f32x4 *>(xsum + (2 * j) * MT + 16 * t + 4 * g);
                    const f32x4 cb = *reinterpret_cast<const f32x4 *>(xsum + (2 * j + 1) * MT + 16 * t + 4 * g);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        pa[t][k] -= ca[k];
                        pb[t][k] -= cb[k];
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    acc[t][k] += s0 * pa[t][k];
                    acc[t][k] += s1 * pb[t][k];
                }
        }
        const float srow = GMODE == 4 ? (float)__builtin_bit_cast(f16, (uint16_t)(sv.x & 0xffffu)) : 1.0f;
        sv = sv_next;

        // ---- this quarter's partials: lane (row nl, tokens 16 t + 4 g + k)
        const int64_t n = n0 + nl;
        if (i < nit && nl <= last_row) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                // FP16: the tile's 4 sparse sums as one vector read ahead of
                // its stores (read inside each store's token test, they took
                // one LDS round trip per store); BF16 reads them per store
                // (the vector spills registers there)
                f32x4 es = f32x4{0.f, 0.f, 0.f, 0.f};
                if (REC && !XB) es = *reinterpret_cast<const f32x4 *>(ex + nl * MT + 16 * t + 4 * g);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int m = 16 * t + 4 * g + k;
                    float v = acc[t][k] * srow;
                    if (REC) v += a.alpha * (XB ? ex[nl * MT + m] : es[k]);
                    if (m < a.M) a.part[((int64_t)qq * a.M + m) * a.N + n] = v;
                }
            }
        }
    };
    const int its = nit > 0 ? nit : 1;
    for (int i = 0; i < its - 1; i++) iteration(i, std::integral_constant<bool, true>{});
    iteration(its - 1, std::integral_constant<bool, false>{});
}

// y = part[0] + part[1] + part[2] + part[3] (in that order), rounded to
// FP16 (+ bias): thread t takes 4 consecutive outputs of one token (N % 4
// == 0; else one output), all four quarters' loads issued together.
__global__ void __launch_bounds__(256) quarter_reduce_kernel(const float *part, f16 *y, int M, int64_t N, int vec4,
                                                             const void *bias, int bias_dtype, int xb) {
    const int64_t MN = (int64_t)M * N;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (vec4) {
        const int64_t o = 4 * t;
        if (o >= MN) return;
        f32x4 v[4];
#pragma unroll
        for (int s = 0; s < 4; s++) v[s] = *reinterpret_cast<const f32x4 *>(part + s * MN + o);
        const f32x4 r = ((v[0] + v[1]) + v[2]) + v[3];
        const int64_t n = o % N;
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            h[e] = xb ? (uint32_t)out_bf16(r[e], bias, bias_dtype, n + e)
                      : (uint32_t)__builtin_bit_cast(uint16_t, out_f16(r[e], bias, bias_dtype, n + e));
        *reinterpret_cast<uint2 *>(y + o) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
        if (t >= MN) return;
        float v[4];
#pragma unroll
        for (int s = 0; s < 4; s++) v[s] = part[s * MN + t];
        const float r = ((v[0] + v[1]) + v[2]) + v[3];
        if (xb) reinterpret_cast<uint16_t *>(y)[t] = out_bf16(r, bias, bias_dtype, t % N);
        else y[t] = out_f16(r, bias, bias_dtype, t % N);
    }
}

// ------------------------------------------------------------------ host

struct QuarterShape {
    int gmode, sparse, lds, grid;
    bool xb;
};

static bool quarter_shape(const ForwardArgs &a, const void *plan, QuarterArgs *d, QuarterShape &sh) {
    if (a.M < 17 || a.M > kQuMT) return false;
    if ((a.io_dtype != ORTH_DT_F16 && a.io_dtype != ORTH_DT_BF16) || a.scale_dtype != ORTH_DT_F16) return false;
    sh.xb = a.io_dtype == ORTH_DT_BF16;
    if (a.K != 512 * kQuCPW) return false;
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
        if (qwords <= 0 || qwords > 1024 || decode_chunks_per_wave(a.K) != kQuCPW) return false;
        sh.sparse = qwords == 256 ? 3 : qwords == 512 ? 4 : 5;
        // BF16: 256-word records only (with 512 or more the registers of the
        // chunk-sum correction spill; those calls take the split-K kernel)
        if (sh.xb && sh.sparse > 3) return false;
    }
    auto al = [](int64_t v) { return (v + 15) & ~int64_t(15); };
    const int64_t cols = 128 * kQuCPW;
    int64_t off = al((int64_t)kQuMT * (cols + 8) * 2);  // row-major activations
    const int64_t lds_xt = off;
    if (sh.sparse) off = al(off + cols * kQuMT * 2 + (cols / 8) * 16);
    const int64_t lds_e = off;
    off += (int64_t)kQuW * qwords * 4;
    const int64_t lds_ex = off;
    if (sh.sparse) off += (int64_t)kQuW * 16 * kQuMT * 4;
    const int64_t lds_xsum = off;
    if (sh.xb) off += (int64_t)kQuCPW * kQuMT * 4;
    if (off > kQuLdsMax) return false;
    sh.lds = (int)off;
    const int64_t nblk = (a.N + 15) / 16;
    const int gq = (int)std::min<int64_t>(nblk, kQuWGs);
    sh.grid = 4 * gq;
    if (d) {
        d->q = a.q;
        d->scales = static_cast<const f16 *>(a.scales);
        d->ngroups = (int)a.ngroups;
        d->row_ptr = a.row_ptr;
        d->col = a.col;
        d->vals = static_cast<const f16 *>(a.vals);
        d->nnz = (int32_t)a.nnz;
        d->x = static_cast<const f16 *>(a.x);
        d->part = nullptr;
        d->M = (int)a.M;
        d->K = (int)a.K;
        d->N = a.N;
        d->nblk = (int)nblk;
        d->gq = gq;
        d->lds_xt = (int)lds_xt;
        d->lds_e = (int)lds_e;
        d->lds_ex = (int)lds_ex;
        d->lds_xsum = (int)lds_xsum;
        d->alpha = a.alpha;
        d->rec = sh.sparse ? reinterpret_cast<const uint32_t *>(static_cast<const char *>(plan) +
                                                                plan_rec_at(a.N, a.K, a.nnz))
                           : nullptr;
        d->qwords = qwords;
    }
    return true;
}

// Whether the quarter-split kernel takes this call (with this plan or none).
bool quarter_supported(const ForwardArgs &a, const void *plan) {
    QuarterShape sh;
    return quarter_shape(a, plan, nullptr, sh);
}

// Workspace bytes of a call: the four quarters' FP32 partials.
int64_t quarter_workspace_bytes(const ForwardArgs &a) { return 4 * a.M * a.N * 4; }

template <int GMODE, int SPARSE, bool XB>
static hipError_t quarter_launch_t(const QuarterArgs &d, const QuarterShape &sh, hipStream_t s) {
    // more than 64 KB of dynamic LDS must be allowed once per device (the
    // attribute call is idempotent, so two threads racing to set it is harmless)
    static std::atomic<int> allowed[64];
    int dev = 0;
    if (sh.lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 &&
        !allowed[dev].load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(quarter_kernel<GMODE, SPARSE, XB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQuLdsMax);
        if (e != hipSuccess) return e;
        allowed[dev].store(1, std::memory_order_release);
    }
    hipLaunchKernelGGL((quarter_kernel<GMODE, SPARSE, XB>), dim3((unsigned)sh.grid), dim3(kQuNT), (uint32_t)sh.lds, s, d);
    return hipGetLastError();
}

template <int GMODE, bool XB>
static hipError_t quarter_launch_s(const QuarterArgs &d, const QuarterShape &sh, hipStream_t s) {
    switch (sh.sparse) {
        case 3: return quarter_launch_t<GMODE, 3, XB>(d, sh, s);
        case 4:
        case 5:
            if constexpr (XB) return hipErrorInvalidValue;  // excluded by quarter_shape
            else return sh.sparse == 4 ? quarter_launch_t<GMODE, 4, XB>(d, sh, s) : quarter_launch_t<GMODE, 5, XB>(d, sh, s);
        default: return quarter_launch_t<GMODE, 0, XB>(d, sh, s);
    }
}

// plan: the layer's ortho plan (required when the ortho term is on); part:
// a workspace of quarter_workspace_bytes(a) bytes.
hipError_t launch_quarter(const ForwardArgs &a, const void *plan, float *part, hipStream_t stream) {
    QuarterArgs d;
    QuarterShape sh;
    if (!quarter_shape(a, plan, &d, sh) || !part) return hipErrorInvalidValue;
    d.part = part;
    hipError_t e = sh.xb ? (sh.gmode == 1 ? quarter_launch_s<1, true>(d, sh, stream) : quarter_launch_s<4, true>(d, sh, stream))
                         : (sh.gmode == 1 ? quarter_launch_s<1, false>(d, sh, stream) : quarter_launch_s<4, false>(d, sh, stream));
    if (e != hipSuccess) return e;
    const int vec4 = a.N % 4 == 0 ? 1 : 0;
    const int64_t threads = vec4 ? a.M * a.N / 4 : a.M * a.N;
    hipLaunchKernelGGL(quarter_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, part,
                       static_cast<f16 *>(a.y), (int)a.M, a.N, vec4, a.bias, a.bias_dtype, sh.xb ? 1 : 0);
    return hipGetLastError();
}

}  // namespace orth
