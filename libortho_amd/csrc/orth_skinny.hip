// Mid-size batches (5 <= M <= 64) of the dual GEMM for gfx950.
//
// Same formula as /root/reference/src/dual_gemm.cu:176-225.  The decode
// kernel gives each 16-row workgroup its own copy of the activations, which
// is cheap at M <= 4 but makes the activation traffic grow as M * K per 16
// rows; here a workgroup of 8 waves owns 128 output rows (one ortho-plan row
// block) and one K slice, and the activation slice is staged once in LDS and
// shared by the 8 waves:
//
//  * Wave w takes rows 16 w .. 16 w + 15; every lane issues one 16-byte
//    nontemporal load per 128-wide chunk of its row at entry (all loads
//    straight-line, addresses clamped).  The weights become biased exact FP16
//    integers (five bit operations per 8 nibbles) and feed
//    v_mfma_f32_16x16x32_f16 as the B operand (BF16 activations: exact BF16
//    integers q + 136 into v_mfma_f32_16x16x32_bf16); the activations of each
//    16-token tile are the A operand, read from LDS (interleaved k order).
//    The bias is removed per chunk with the activation sums computed while
//    staging; group scales multiply each chunk's FP32 partial.
//  * The sparse ortho term reads the CSR itself.  The ortho plan's chunk
//    table (per row, the count of entries below each 128-column boundary)
//    gives each row's entries inside the slice as one contiguous CSR range
//    when the rows' columns ascend; otherwise (or without a plan) each row's
//    whole range is read and filtered by column, in batches of eight
//    entries.  Up to 16 tokens, four consecutive lanes share a row: each
//    loads two of every eight entries, DPP quad broadcasts hand all eight to
//    the four, each multiplies them with four tokens' staged activations
//    (two up to 8 tokens: tokens past M are padding of the tile), and the
//    sums reach the MFMA lanes through LDS.  From 17 tokens (more
//    registers, and an LDS exchange would cost the second workgroup per CU)
//    each lane takes the row and tokens of its own MFMA output and reads the
//    row's entries itself.  Sums are formed in CSR order: the result does not
//    depend on scheduling.
//  * With the plan's slice records (one token tile, 8-chunk slices,
//    K % 1024 == 0) each wave instead loads its 16 rows' record of the slice
//    at entry (packed column | value words at an address that needs no other
//    load), stages it in its own LDS region, and forms the sums before the
//    dense term, after issuing the rest of its weight loads.
//  * When the row blocks alone cannot fill the GPU, K is split over S
//    workgroups.  Each writes its FP32 partial (ortho term included) to a
//    workspace and a second kernel adds the S partials in slice order and
//    writes y.  (The kernel boundary makes the partials visible across the
//    XCDs; an in-kernel hand-off would need device-scope fences, which on
//    this part write back and invalidate the L2 of every XCD.)
#include <algorithm>

#include <atomic>

#include "orth_common.h"

namespace orth {

int64_t plan_chunks_at(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip
int64_t plan_chunks_bytes(int64_t N, int64_t K);
int plan_srec_words(int64_t N, int64_t K, int64_t nnz);
int64_t plan_srec_at(int64_t N, int64_t K, int64_t nnz);

constexpr int kSkNT = 512;            // 8 waves
constexpr int kSkRows = 128;          // rows per workgroup (= ortho plan block)
constexpr int kSkMaxCPS = 8;          // chunks per slice (compile-time bound)
constexpr int kSkEB = 8;              // CSR entries of a row per batch

// x from lane s of each group of four lanes (DPP quad_perm)
template <int S>
__device__ __forceinline__ int quad_bcast(int x) {
    return __builtin_amdgcn_update_dpp(0, x, S | (S << 2) | (S << 4) | (S << 6), 0xf, 0xf, false);
}
constexpr uint32_t kSkPlanMagic = 0x504f5254u;
constexpr uint32_t kSkPlanVersion = 5;
constexpr uint32_t kSkPlanUnsorted = 4u;  // plan flag: the chunk table does not locate ranges

// Chunks per slice the kernel of ntt token tiles is built for: even (group
// scales are read in pairs) and with at most 8 activation pieces per thread.
constexpr int sk_cps_bound(int ntt) { return ntt * kSkMaxCPS > 16 ? ((16 / ntt) & ~1) : kSkMaxCPS; }

struct SkinnyArgs {
    const uint8_t *q;
    const f16 *scales;
    int ngroups;
    int gshift;          // group of chunk c is c >> gshift (G = 128 << gshift)
    const int32_t *row_ptr;   // CSR of the ortho term
    const int32_t *col;
    const f16 *vals;
    const uint16_t *chunks;   // plan chunk table [N][nchunks + 1], or null
    const uint32_t *phdr;     // plan header (magic, version, bn, bk, nblocks, nsteps, n, k, nnz, flags), or null
    int32_t nnz;
    const f16 *x;
    f16 *y;
    int M;
    int K;
    int64_t N;
    int nchunks;         // K / 128
    int cps;             // chunks per slice (even)
    int S;               // slices
    int nblocks;         // 128-row blocks
    int xstride;         // LDS row stride of the staged activations, in halves
    int lds_cr, lds_xs, lds_sp;  // byte offsets of the LDS regions
    float alpha;
    float *part;         // [S][M][N] partials (S > 1)
    const uint32_t *srec;  // plan slice records (SPK >= 3), swords words each
    int swords;
    int nslices;         // K / 1024
    int lds_sr;          // SPK >= 3: per-wave record regions
    const void *bias;  // [N] added after rounding (out_f16), or null
    int bias_dtype;
};

// GMODE: 0 per-row scale (G == K); 1 G = 128, scales read as aligned pairs;
// 2 any G = 128 * 2^j; 3 (one token tile) G = 128 with every slice exactly CPS = 8 chunks
// (K = 1024 S) and its scales one aligned 16-byte vector per row: the dense
// term is straight-line code over chunk pairs (two MFMA chains interleaved)
// and the weight loads run four chunks ahead instead of all at entry.
// NTT: 16-token tiles.  CPS: chunk bound per slice.  SPK: 0 no ortho term,
// 1 ortho term, 2 ortho term for at most 8 tokens (one tile: the four lanes
// of a row gather two tokens each, not four); 3 .. 6 (one tile, GMODE 3) the
// same from the plan's slice records instead of the CSR: 3 / 4 records of
// 256 words (4: at most 8 tokens), 5 / 6 of 512 words.
// (4 waves per SIMD up to two token tiles; BF16 with two tiles needs the
// registers of 2: at 4 one instantiation spilled 8 bytes)
template <int NTT, int GMODE, int CPS, int SPK, bool XB>
__global__ void __launch_bounds__(kSkNT) __attribute__((amdgpu_waves_per_eu(NTT == 1 || (NTT == 2 && !XB) ? 4 : 2)))
skinny_kernel(SkinnyArgs a) {
    constexpr bool SPARSE = SPK != 0;
    constexpr bool SREC = SPK >= 3;                  // slice records: each wave reads its 16 rows' record
    constexpr bool HALF = SPK == 2 || SPK == 4 || SPK == 6;
    constexpr int RQ = SPK >= 5 ? 2 : 1;             // record loads per lane (256 words each per wave)
    constexpr int MP = NTT * 16;                     // padded tokens
    constexpr int XP = (MP * CPS * 16 + kSkNT - 1) / kSkNT;  // 16-byte pieces per thread
    constexpr int SW = (CPS + 7) / 8;
    constexpr bool GROUPED = GMODE != 0;
    constexpr bool FULL = GMODE == 3;  // every slice holds exactly CPS chunks
    static_assert(!SREC || (FULL && NTT == 1), "slice records: one token tile, 8-chunk slices");
    static_assert(!FULL || CPS == 8, "full slices are one scale vector");
    constexpr int PDC = FULL ? 4 : CPS;  // weight loads issued at entry
    // QUAD: four consecutive lanes per row in the sparse term (one token tile)
    constexpr bool QUAD = NTT == 1;
    // XB: BF16 activations and output.  The weights become the exact BF16
    // integers q + 136 (every k weighs 136 in the chunk's bias sum) and feed
    // v_mfma_f32_16x16x32_bf16; FP16: q + 1032 (even k) / q + 72 (odd k).
    auto wconv = [](uint32_t w, uint32_t out[4]) {
        if constexpr (XB) int4x8_to_bf16_biased(w, out);
        else int4x8_to_f16_biased(w, out);
    };
    auto mfma = [](const f16x8 &av, const uint32_t b[4], f32x4 c) -> f32x4 {
        if constexpr (XB)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                           __builtin_bit_cast(bf16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(f16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                          c, 0, 0, 0);
    };
    constexpr int EL = QUAD ? kSkEB / 4 : kSkEB;  // entries a lane loads per batch

    extern __shared__ __align__(16) unsigned char smem[];
    float *cr = reinterpret_cast<float *>(smem + a.lds_cr);     // [cps][MP] bias sums
    f16 *xs = reinterpret_cast<f16 *>(smem + a.lds_xs);         // [MP][xstride] activations
    float *sp = reinterpret_cast<float *>(smem + a.lds_sp);     // QUAD: [128][MP] sparse sums

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int nl = lane & 15, g = lane >> 4;
    // Workgroup ids are dealt round-robin to the 8 XCDs: all K slices of row
    // block blk run on XCD blk % 8, as does the reduction workgroup of blk,
    // so a block's partials are written and read through one L2.  The grid
    // is padded to 8 * ceil(nblocks / 8) * S.
    const int q = (int)(blockIdx.x >> 3);
    const int blk = (int)(blockIdx.x & 7) + 8 * (q / a.S), slice = q - (q / a.S) * a.S;
    if (blk >= a.nblocks) return;
    const int64_t n0 = (int64_t)blk * kSkRows;
    const int kc0 = slice * a.cps;                               // first chunk of the slice
    const int nci = max(0, min(a.cps, a.nchunks - kc0));         // uniform
    const int clast = a.nchunks - 1;
    const int64_t wrow0 = n0 + wave * 16;
    const int64_t my_n = min(wrow0 + nl, a.N - 1);               // clamped weight row
    const int K = a.K;

    // ---- activations of the slice: piece p = (m, c, j) covers 8 halves
    u32x4 xreg[XP];
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + kSkNT * i;
        const int m = min(p / (CPS * 16), a.M - 1);
        const int c = min(kc0 + (p / 16) % CPS, clast);
        xreg[i] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)m * K + c * 128 + (p & 15) * 8);
    }

    // ---- sparse term inputs of this lane's row, issued after the
    //      activations and before the weights (loads complete in order: the
    //      staging does not wait for them, nor they for the weights): the
    //      row's CSR bounds, its chunk-table counts at the slice's ends, and
    //      (lanes 0 .. 12) the plan header.  Without a plan the addresses fall
    //      back to the row pointers (read, not used).
    // (QUAD: row tid / 4 of the block, tokens tid % 4 + 4 i; else the MFMA
    //  output's row 16 w + nl)
    const int sr = QUAD ? tid >> 2 : wave * 16 + nl, tg = tid & 3;
    const int64_t sn = min(n0 + sr, a.N - 1);
    int32_t rp0 = 0, rp1 = 0, hw = 0;
    uint32_t ck0 = 0, ck1 = 0;
    // SREC: this wave's record (rows 16 w .. 16 w + 15 of the block, the
    // slice's columns), at an address that needs no other load
    const int64_t g16 = min((int64_t)blk * 8 + wave, (a.N + 15) / 16 - 1);
    const int sl = kc0 >> 3;
    u32x4 rq[RQ];
    if (SREC) {
        const uint32_t *rb = a.srec + (g16 * a.nslices + sl) * (int64_t)a.swords;
#pragma unroll
        for (int i = 0; i < RQ; i++)
            rq[i] = *reinterpret_cast<const u32x4 *>(rb + min(4 * (lane + 64 * i), a.swords - 4));
    }
    if (SPARSE && !SREC) {
        rp0 = a.row_ptr[sn];
        rp1 = a.row_ptr[sn + 1];
        const bool tab = a.chunks != nullptr;
        const uint16_t *ct = tab ? a.chunks + sn * (int64_t)(a.nchunks + 1) : reinterpret_cast<const uint16_t *>(a.row_ptr);
        ck0 = ct[tab ? kc0 : 0];
        ck1 = ct[tab ? kc0 + nci : 0];
        const uint32_t *hp = a.phdr ? a.phdr : reinterpret_cast<const uint32_t *>(a.row_ptr);
        hw = (int32_t)hp[a.phdr ? min(lane, 12) : 0];
    }

    // ---- scales
    const f16 *sbase = a.scales + my_n * (int64_t)a.ngroups;
    uint32_t sw[SW];
    f16 sh[GMODE == 2 ? CPS : 1];
    u32x4 sv = u32x4{0u, 0u, 0u, 0u};  // GMODE 3: this row's 8 scales of the slice
    float srow = 0.f;  // GMODE 0: the scale of row 16 w + nl (tid & 15 == nl)
    if (GMODE == 0) srow = (float)a.scales[min(wrow0 + (tid & 15), a.N - 1)];
    if (GMODE == 3) {
        sv = *reinterpret_cast<const u32x4 *>(sbase + kc0);
    } else if (GMODE == 1) {
#pragma unroll
        for (int i = 0; i < SW; i++)
            sw[i] = *reinterpret_cast<const uint32_t *>(sbase + (min(kc0 + 8 * i + 2 * g, clast) & ~1));
    } else if (GMODE == 2) {
#pragma unroll
        for (int p = 0; p < CPS; p++) sh[p] = sbase[min(kc0 + p, clast) >> a.gshift];
    }

    // ---- weights (nontemporal), one 16-byte load per chunk
    const uint8_t *qrow = a.q + my_n * (int64_t)(K >> 1) + g * 16;
    u32x4 wv[CPS];
    auto load_chunk = [&](int p) {
        wv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + min(kc0 + p, clast) * 64));
    };
#pragma unroll
    for (int p = 0; p < PDC; p++) load_chunk(p);

    // ---- stage the activations (interleaved k order) and their bias sums
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + kSkNT * i;
        const int m = p / (CPS * 16), c = (p / 16) % CPS;
        u32x4 v = xreg[i];
        if (m >= a.M) v = u32x4{0, 0, 0, 0};
        const f16x8 h = __builtin_bit_cast(f16x8, v);
        // even k weigh 1032, odd k weigh 72 (see int4x8_to_f16_biased); BF16:
        // every k weighs 136 (int4x8_to_bf16_biased)
        const float e = (x16_to_f32<XB>(h[0]) + x16_to_f32<XB>(h[2])) + (x16_to_f32<XB>(h[4]) + x16_to_f32<XB>(h[6]));
        const float o = (x16_to_f32<XB>(h[1]) + x16_to_f32<XB>(h[3])) + (x16_to_f32<XB>(h[5]) + x16_to_f32<XB>(h[7]));
        const float b = group_sum<16>(XB ? 136.0f * (e + o) : 1032.0f * e + 72.0f * o);  // the 16 pieces of (m, c)
        if (m < MP && c < a.cps) {  // the LDS tile holds the host's cps chunks
            *reinterpret_cast<u32x4 *>(xs + (m * a.xstride + c * 128 + (p & 15) * 8)) = permute_x8(v);
            if ((p & 15) == 0) cr[c * MP + m] = b;
        }
    }
    if (SREC) {
        uint32_t *wr = reinterpret_cast<uint32_t *>(smem + a.lds_sr) + wave * a.swords;
#pragma unroll
        for (int i = 0; i < RQ; i++) {
            const int o = 4 * (lane + 64 * i);
            if (o < a.swords) *reinterpret_cast<u32x4 *>(wr + o) = rq[i];
        }
    }
    __syncthreads();

    // ---- the row's CSR range in the slice.  With a matching plan whose
    //      rows ascend, the chunk table gives it; otherwise the whole row is
    //      read and filtered by column.  (Read after the staging and its
    //      barrier, kept there by the scheduling barrier.)
    __builtin_amdgcn_sched_barrier(0);
    int32_t lo = 0, hi = 0;
    constexpr int EB = kSkEB;
    int32_t ecol[EL], ecol2[EL];  // the first two batches, loaded before the dense term
    uint32_t eval[EL], eval2[EL];
    // entry u of this lane in the batch at j0: j0 + tg + 4 u (QUAD) or j0 + u
    auto load_batch = [&](int32_t j0, int32_t (&c)[EL], uint32_t (&v)[EL]) {
        const int32_t jl = min(max(hi - 1, lo), a.nnz - 1);
#pragma unroll
        for (int u = 0; u < EL; u++) {
            const int32_t j = min(j0 + (QUAD ? tg + 4 * u : u), jl);
            c[u] = a.col[j];
            v[u] = __builtin_bit_cast(uint16_t, a.vals[j]);
        }
    };
    if (SPARSE && !SREC) {
        auto word = [&](int l) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane(hw, l); };
        auto dword = [&](int l) -> int64_t { return (int64_t)(word(l) | ((uint64_t)word(l + 1) << 32)); };
        const bool fast = (a.phdr != nullptr) & (a.chunks != nullptr) & (word(0) == kSkPlanMagic) &
                          (word(1) == kSkPlanVersion) & (dword(6) == a.N) & (dword(8) == (int64_t)K) &
                          (dword(10) == (int64_t)a.nnz) & ((word(12) & kSkPlanUnsorted) == 0);
        const int32_t rs = min(max(rp0, 0), a.nnz), re = min(max(rp1, rs), a.nnz);
        lo = fast ? rs + min((int32_t)ck0, re - rs) : rs;
        hi = fast ? rs + min(max((int32_t)ck1, (int32_t)ck0), re - rs) : re;
        if (n0 + sr >= a.N) hi = lo;  // rows past N
        load_batch(lo, ecol, eval);
        load_batch(lo + EB, ecol2, eval2);
    }

    // ---- SREC: the sparse sums from the record, before the dense term:
    //      the remaining weight loads are issued first, so the stream does
    //      not pause while the sums are formed
    constexpr int TQ = QUAD ? (HALF ? 2 : MP / 4) : NTT * 4;  // tokens per lane
    float sacc_e[SREC ? TQ : 1];
    if constexpr (SREC) {
#pragma unroll
        for (int p = PDC; p < CPS; p++) load_chunk(p);
    }
    if constexpr (SREC) {
#pragma unroll
        for (int t = 0; t < TQ; t++) sacc_e[t] = 0.f;
        const int32_t c0 = kc0 * 128, cw = nci * 128;
        const int xstride = a.xstride;
        auto fma_batch = [&](int32_t j0, const int32_t (&c)[EL], const uint32_t (&v)[EL]) {
#pragma unroll
            for (int e = 0; e < kSkEB; e++) {
                int32_t ce;
                uint32_t ve;
                if (QUAD) {  // entry j0 + e sits in lane e % 4 of the quad, slot e / 4
                    const int slot = e >> 2;
                    switch (e & 3) {
                        case 0: ce = quad_bcast<0>(c[slot]); ve = (uint32_t)quad_bcast<0>((int)v[slot]); break;
                        case 1: ce = quad_bcast<1>(c[slot]); ve = (uint32_t)quad_bcast<1>((int)v[slot]); break;
                        case 2: ce = quad_bcast<2>(c[slot]); ve = (uint32_t)quad_bcast<2>((int)v[slot]); break;
                        default: ce = quad_bcast<3>(c[slot]); ve = (uint32_t)quad_bcast<3>((int)v[slot]); break;
                    }
                } else {
                    ce = c[e % EL];
                    ve = v[e % EL];
                }
                const int32_t cl = ce - c0;
                const bool ok = (j0 + e < hi) & (cl >= 0) & (cl < cw);
                const int cc = ok ? cl : 0;
                const float val = (float)__builtin_bit_cast(f16, (uint16_t)(ve & 0xffffu));
                const int xi = (cc & ~7) | interleaved_pos(cc & 7);
#pragma unroll
                for (int t = 0; t < TQ; t++) {
                    const int m = QUAD ? tg + 4 * t : 16 * (t >> 2) + 4 * g + (t & 3);
                    const float pr = val * x16_to_f32<XB>(xs[m * xstride + xi]);
                    sacc_e[t] += ok ? pr : 0.f;
                }
            }
        };
        const uint32_t *wr = reinterpret_cast<const uint32_t *>(smem + a.lds_sr) + wave * a.swords;
        // (uniform per wave) the record of this group and slice, all its
        // entries inside: else the row's CSR range, filtered by column
        const bool ok = (wr[0] == plan_cell_tag(kCellSlice, a.N, K, a.nnz, a.swords, g16, sl)) & (wr[1] == 0u);
        if (ok) {
            const uint32_t h = wr[2 + ((tid >> 2) & 15)];
            lo = (int32_t)(h & 0xffffu);
            hi = (int32_t)(h >> 16);
            if (n0 + sr >= a.N) hi = lo;
            const uint32_t *ent = wr + kCellHdrWords;
            for (int32_t j0 = lo; j0 < hi; j0 += kSkEB) {
                int32_t c2[EL];
                uint32_t v2[EL];
#pragma unroll
                for (int u = 0; u < EL; u++) {
                    const uint32_t w = ent[min(j0 + tg + 4 * u, hi - 1)];
                    c2[u] = (int32_t)(w & 0xffffu) + c0;
                    v2[u] = w >> 16;
                }
                fma_batch(j0, c2, v2);
            }
        } else {
            int32_t rs, re;
            csr_row_range(a.row_ptr, sn, a.nnz, rs, re);
            lo = rs;
            hi = (n0 + sr < a.N) ? re : rs;
            for (int32_t j0 = lo; j0 < hi; j0 += kSkEB) {
                int32_t c2[EL];
                uint32_t v2[EL];
                load_batch(j0, c2, v2);
                fma_batch(j0, c2, v2);
            }
        }
        if (QUAD) {
#pragma unroll
            for (int t = 0; t < TQ; t++) sp[sr * MP + tg + 4 * t] = sacc_e[t];
        }
    }
    // ---- dense term: wave w, rows 16 w + nl, token tiles tt
    f32x4 acc[NTT];
    float bias_acc[NTT][4];
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) bias_acc[tt][i] = 0.f;
    }
    if constexpr (FULL) {
#pragma unroll
        for (int p = 0; p < CPS; p += 2) {
            uint32_t bq0[4][4], bq1[4][4];
            {
                const uint32_t w0[4] = {wv[p].x, wv[p].y, wv[p].z, wv[p].w};
                const uint32_t w1[4] = {wv[p + 1].x, wv[p + 1].y, wv[p + 1].z, wv[p + 1].w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    wconv(w0[j], bq0[j]);
                    wconv(w1[j], bq1[j]);
                }
            }
            if (!SREC && p + PDC < CPS) load_chunk(p + PDC);
            if (!SREC && p + 1 + PDC < CPS) load_chunk(p + 1 + PDC);
            const uint32_t s2 = sv[p >> 1];  // the scales of chunks p, p + 1
            const float s0 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 & 0xffffu));
            const float s1 = (float)__builtin_bit_cast(f16, (uint16_t)(s2 >> 16));
#pragma unroll
            for (int tt = 0; tt < NTT; tt++) {
                const f16 *xl = xs + ((tt * 16 + nl) * a.xstride + p * 128 + g * 32);
                f32x4 pa = f32x4{0.f, 0.f, 0.f, 0.f}, pb = pa;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f16x8 a0 = *reinterpret_cast<const f16x8 *>(xl + 8 * j);
                    const f16x8 a1 = *reinterpret_cast<const f16x8 *>(xl + 128 + 8 * j);
                    pa = mfma(a0, bq0[j], pa);
                    pb = mfma(a1, bq1[j], pb);
                }
                // D[token 4g + i][row nl]
                const f32x4 cra = *reinterpret_cast<const f32x4 *>(cr + p * MP + tt * 16 + 4 * g);
                const f32x4 crb = *reinterpret_cast<const f32x4 *>(cr + (p + 1) * MP + tt * 16 + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc[tt][i] += s0 * (pa[i] - cra[i]);
                    acc[tt][i] += s1 * (pb[i] - crb[i]);
                }
            }
        }
    } else {
    #pragma unroll
        for (int p = 0; p < CPS; p++) {
            if (p < nci) {  // uniform
                const uint32_t words[4] = {wv[p].x, wv[p].y, wv[p].z, wv[p].w};
                uint32_t bq[4][4];
    #pragma unroll
                for (int j = 0; j < 4; j++) wconv(words[j], bq[j]);
                float s = 1.0f;
                if (GMODE == 1) {
                    // scales of chunks kc0 + 8i + 2g', +1 sit in lane 16g' + nl
                    const uint32_t w2 = (uint32_t)__shfl((int)sw[p >> 3], 16 * ((p & 7) >> 1) + nl, 64);
                    s = (float)__builtin_bit_cast(f16, (uint16_t)((p & 1) ? (w2 >> 16) : (w2 & 0xffffu)));
                } else if (GMODE == 2) {
                    s = (float)sh[p];
                }
    #pragma unroll
                for (int tt = 0; tt < NTT; tt++) {
                    const f16 *xl = xs + ((tt * 16 + nl) * a.xstride + p * 128 + g * 32);
                    f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
    #pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const f16x8 afr = *reinterpret_cast<const f16x8 *>(xl + 8 * j);
                        part = mfma(afr, bq[j], part);
                    }
                    // D[token 4g + i][row nl]
                    const f32x4 crv = *reinterpret_cast<const f32x4 *>(cr + p * MP + tt * 16 + 4 * g);
    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if (GROUPED) {
                            acc[tt][i] += s * (part[i] - crv[i]);
                        } else {
                            acc[tt][i] += part[i];
                            bias_acc[tt][i] += crv[i];
                        }
                    }
                }
            }
        }
    }

    // ---- sparse term, in batches of eight entries; columns outside the
    //      slice are skipped.  Token t of the lane: QUAD tg + 4 t, else
    //      16 (t / 4) + 4 g + t % 4 (the MFMA output's tokens).
    float sacc[SPARSE && !SREC ? TQ : 1];
    if constexpr (SPARSE && !SREC) {
#pragma unroll
        for (int t = 0; t < TQ; t++) sacc[t] = 0.f;
        const int32_t c0 = kc0 * 128, cw = nci * 128;
        const int xstride = a.xstride;
        auto fma_batch = [&](int32_t j0, const int32_t (&c)[EL], const uint32_t (&v)[EL]) {
#pragma unroll
            for (int e = 0; e < kSkEB; e++) {
                int32_t ce;
                uint32_t ve;
                if (QUAD) {  // entry j0 + e sits in lane e % 4 of the quad, slot e / 4
                    const int slot = e >> 2;
                    switch (e & 3) {
                        case 0: ce = quad_bcast<0>(c[slot]); ve = (uint32_t)quad_bcast<0>((int)v[slot]); break;
                        case 1: ce = quad_bcast<1>(c[slot]); ve = (uint32_t)quad_bcast<1>((int)v[slot]); break;
                        case 2: ce = quad_bcast<2>(c[slot]); ve = (uint32_t)quad_bcast<2>((int)v[slot]); break;
                        default: ce = quad_bcast<3>(c[slot]); ve = (uint32_t)quad_bcast<3>((int)v[slot]); break;
                    }
                } else {
                    ce = c[e % EL];
                    ve = v[e % EL];
                }
                const int32_t cl = ce - c0;
                const bool ok = (j0 + e < hi) & (cl >= 0) & (cl < cw);
                const int cc = ok ? cl : 0;
                const float val = (float)__builtin_bit_cast(f16, (uint16_t)(ve & 0xffffu));
                const int xi = (cc & ~7) | interleaved_pos(cc & 7);
#pragma unroll
                for (int t = 0; t < TQ; t++) {
                    const int m = QUAD ? tg + 4 * t : 16 * (t >> 2) + 4 * g + (t & 3);
                    const float pr = val * x16_to_f32<XB>(xs[m * xstride + xi]);
                    sacc[t] += ok ? pr : 0.f;
                }
            }
        };
        fma_batch(lo, ecol, eval);
        // the lanes of a row take the same branches and trip counts
        if (lo + kSkEB < hi) fma_batch(lo + kSkEB, ecol2, eval2);
        // more entries (dense rows, or a whole row without the chunk table)
        for (int32_t j0 = lo + 2 * kSkEB; j0 < hi; j0 += kSkEB) {
            int32_t c2[EL];
            uint32_t v2[EL];
            load_batch(j0, c2, v2);
            fma_batch(j0, c2, v2);
        }
        if (QUAD) {
#pragma unroll
            for (int t = 0; t < TQ; t++) sp[sr * MP + tg + 4 * t] = sacc[t];
        }
    }
    if (SPARSE && QUAD) __syncthreads();  // the sums reach the MFMA lanes

    // ---- this slice's values: lane (row nl, tokens tt*16 + 4g + i)
    float val[NTT][4];
    const int64_t n = wrow0 + nl;
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = acc[tt][i];
            if (!GROUPED) v = (v - bias_acc[tt][i]) * srow;
            if (SPARSE) v += a.alpha * (QUAD ? sp[(wave * 16 + nl) * MP + tt * 16 + 4 * g + i] : sacc[tt * 4 + i]);
            val[tt][i] = v;
        }
    }
    if (a.S == 1) {
#pragma unroll
        for (int tt = 0; tt < NTT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = tt * 16 + 4 * g + i;
                if (m < a.M && n < a.N) {
                    if constexpr (XB)
                        reinterpret_cast<uint16_t *>(a.y)[(int64_t)m * a.N + n] = out_bf16(val[tt][i], a.bias, a.bias_dtype, n);
                    else
                        a.y[(int64_t)m * a.N + n] = out_f16(val[tt][i], a.bias, a.bias_dtype, n);
                }
            }
        return;
    }

    // ---- split K: this slice's partial to the workspace
    float *pw = a.part + (int64_t)slice * a.M * a.N;
#pragma unroll
    for (int tt = 0; tt < NTT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = tt * 16 + 4 * g + i;
            if (m < a.M && n < a.N) pw[(int64_t)m * a.N + n] = val[tt][i];
        }
}

// y = sum of the S partials, in slice order.  Thread t takes 4 consecutive
// outputs of one token (N % 4 == 0) or one output (otherwise).
// Row block blk's outputs (its 128 rows x M tokens) are dealt to R
// workgroups, one output group per thread; workgroup id b takes block
// (b & 7) + 8 ((b >> 3) / R), part (b >> 3) % R, so every workgroup of
// block blk runs on XCD blk % 8 like the slices that wrote its partials.
// The loads of all S slices (up to 16 per round) are issued before the
// first add (addresses clamped to the last slice, the extra ones not
// added); sums in slice order.
constexpr int kSkRedU = 16;

static int skinny_reduce_parts(int M, int vec4) {
    const int items = M * (vec4 ? kSkRows / 4 : kSkRows);
    return (items + 255) / 256;
}

__global__ void __launch_bounds__(256) skinny_reduce_kernel(const float *part, f16 *y, int M, int64_t N, int S,
                                                            int vec4, int nblocks, int R, const void *bias,
                                                            int bias_dtype, int xb) {
    constexpr int U = kSkRedU;
    const int q = (int)(blockIdx.x >> 3);
    const int blk = (int)(blockIdx.x & 7) + 8 * (q / R);
    const int r = q - (q / R) * R;
    if (blk >= nblocks) return;
    const int64_t n0 = (int64_t)blk * kSkRows;
    const int64_t MN = (int64_t)M * N;
    const int idx = r * 256 + (int)threadIdx.x;
    if (vec4) {
        if (idx >= M * (kSkRows / 4)) return;
        const int m = idx / (kSkRows / 4);
        const int64_t n = n0 + 4 * (idx - m * (kSkRows / 4));
        if (n >= N) return;
        const int64_t o = (int64_t)m * N + n;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += U) {
            f32x4 w[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                w[u] = *reinterpret_cast<const f32x4 *>(part + (int64_t)min(s0 + u, S - 1) * MN + o);
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u == 0) v = w[u];
                else if (s0 + u < S) v += w[u];
            }
        }
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            h[e] = xb ? (uint32_t)out_bf16(v[e], bias, bias_dtype, n + e)
                      : (uint32_t)__builtin_bit_cast(uint16_t, out_f16(v[e], bias, bias_dtype, n + e));
        *reinterpret_cast<uint2 *>(y + o) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
        if (idx >= M * kSkRows) return;
        const int m = idx / kSkRows;
        const int64_t n = n0 + (idx - m * kSkRows);
        if (n >= N) return;
        const int64_t o = (int64_t)m * N + n;
        float v = 0.f;
        for (int s0 = 0; s0 < S; s0 += U) {
            float w[U];
#pragma unroll
            for (int u = 0; u < U; u++) w[u] = part[(int64_t)min(s0 + u, S - 1) * MN + o];
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u == 0) v = w[u];
                else if (s0 + u < S) v += w[u];
            }
        }
        if (xb) reinterpret_cast<uint16_t *>(y)[o] = out_bf16(v, bias, bias_dtype, n);
        else y[o] = out_f16(v, bias, bias_dtype, n);
    }
}

// ------------------------------------------------------------------ host

struct SkinnyShape {
    int ntt, cps, S, nblocks, xstride;
    int lds_cr, lds_xs, lds_sp, lds_bytes;
};

static bool skinny_shape(const ForwardArgs &a, int cus, SkinnyShape &sh) {
    const int ntt = (int)((a.M + 15) / 16);
    const int nchunks = (int)(a.K / 128);
    sh.ntt = ntt;
    sh.nblocks = (int)((a.N + kSkRows - 1) / kSkRows);
    const int mp = ntt * 16;
    const int cps_max = sk_cps_bound(ntt);
    // enough workgroups to keep every CU streaming: about 1.3 per CU
    int S = (int)std::min<int64_t>(nchunks, std::max<int64_t>(1, (cus * 13 / 10 + sh.nblocks - 1) / sh.nblocks));
    int cps = (nchunks + S - 1) / S;
    cps = std::min(cps + (cps & 1), cps_max);              // even: group scales read as pairs
    S = (nchunks + cps - 1) / cps;
    sh.cps = cps;
    sh.S = S;
    sh.xstride = cps * 128 + 8;
    int off = 0;
    sh.lds_cr = off;
    off += cps * mp * 4;
    sh.lds_xs = off;
    off += ((mp * sh.xstride * 2) + 15) & ~15;
    sh.lds_sp = off;
    off += a.has_ortho && ntt == 1 ? kSkRows * mp * 4 : 0;  // the kernel's QUAD exchange
    sh.lds_bytes = off;
    return off <= 150 * 1024;
}

bool skinny_supported(const ForwardArgs &a) {
    if (a.M < 1 || a.M > 64) return false;
    if ((a.io_dtype != ORTH_DT_F16 && a.io_dtype != ORTH_DT_BF16) || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.has_ortho && a.val_dtype != ORTH_DT_F16) return false;  // values read from the CSR as FP16
    if (a.K % 128 != 0) return false;
    if (a.ngroups != 1) {
        if (a.G % 128 != 0) return false;
        const int64_t r = a.G / 128;
        if (r & (r - 1)) return false;
    }
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    if (a.N > ((int64_t)1 << 31)) return false;
    SkinnyShape sh;
    return skinny_shape(a, 256, sh);
}

template <int NTT, int GMODE, int CPS, int SPARSE, bool XB>
static hipError_t skinny_launch_t(const SkinnyArgs &d, int blocks, int lds, hipStream_t s) {
    // more than 64 KB of dynamic LDS must be allowed once per device (the
    // attribute call is idempotent, so two threads racing to set it is harmless)
    static std::atomic<int> allowed[64];
    int dev = 0;
    if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 &&
        !allowed[dev].load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(skinny_kernel<NTT, GMODE, CPS, SPARSE, XB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        if (e != hipSuccess) return e;
        allowed[dev].store(1, std::memory_order_release);
    }
    hipLaunchKernelGGL((skinny_kernel<NTT, GMODE, CPS, SPARSE, XB>), dim3(blocks), dim3(kSkNT), (uint32_t)lds, s, d);
    return hipGetLastError();
}

template <int NTT, int GMODE, bool XB>
static hipError_t skinny_launch_g(const SkinnyArgs &d, bool sparse, int blocks, int lds, hipStream_t s) {
    constexpr int C = sk_cps_bound(NTT);
    if (d.cps > C) return hipErrorInvalidValue;  // the kernel handles at most C chunks per slice
    if (sparse) {
        if constexpr (NTT == 1 && GMODE == 3) {
            if (d.swords > 0) {  // slice records (launch_skinny checked the shape)
                const bool half = d.M <= 8;
                if (d.swords == 256) return half ? skinny_launch_t<NTT, GMODE, C, 4, XB>(d, blocks, lds, s)
                                                 : skinny_launch_t<NTT, GMODE, C, 3, XB>(d, blocks, lds, s);
                return half ? skinny_launch_t<NTT, GMODE, C, 6, XB>(d, blocks, lds, s)
                            : skinny_launch_t<NTT, GMODE, C, 5, XB>(d, blocks, lds, s);
            }
        }
        if (NTT == 1 && d.M <= 8) return skinny_launch_t<NTT, GMODE, C, (NTT == 1 ? 2 : 1), XB>(d, blocks, lds, s);
        return skinny_launch_t<NTT, GMODE, C, 1, XB>(d, blocks, lds, s);
    }
    return skinny_launch_t<NTT, GMODE, C, 0, XB>(d, blocks, lds, s);
}

template <int NTT, bool XB>
static hipError_t skinny_launch_n(const SkinnyArgs &d, int gmode, bool sparse, int blocks, int lds, hipStream_t s) {
    switch (gmode) {
        case 0: return skinny_launch_g<NTT, 0, XB>(d, sparse, blocks, lds, s);
        case 1: return skinny_launch_g<NTT, 1, XB>(d, sparse, blocks, lds, s);
        case 3:
            if constexpr (NTT == 1) return skinny_launch_g<NTT, 3, XB>(d, sparse, blocks, lds, s);
            return hipErrorInvalidValue;
        default: return skinny_launch_g<NTT, 2, XB>(d, sparse, blocks, lds, s);
    }
}

template <bool XB>
static hipError_t skinny_launch_x(const SkinnyArgs &d, int ntt, int gmode, bool sparse, int blocks, int lds,
                                  hipStream_t s) {
    switch (ntt) {
        case 1: return skinny_launch_n<1, XB>(d, gmode, sparse, blocks, lds, s);
        case 2: return skinny_launch_n<2, XB>(d, gmode, sparse, blocks, lds, s);
        case 3: return skinny_launch_n<3, XB>(d, gmode, sparse, blocks, lds, s);
        default: return skinny_launch_n<4, XB>(d, gmode, sparse, blocks, lds, s);
    }
}

// Workspace bytes of a call (0 when K is not split).
int64_t skinny_workspace_bytes(const ForwardArgs &a, int cus) {
    SkinnyShape sh;
    skinny_shape(a, cus, sh);
    return sh.S > 1 ? (int64_t)sh.S * a.M * a.N * 4 : 0;
}

// plan: the ortho plan (optional: its chunk table locates the slice's CSR
// ranges; without it rows are filtered by column); part: the workspace.
hipError_t launch_skinny(const ForwardArgs &a, const void *plan, int cus, float *part, hipStream_t stream) {
    SkinnyShape sh;
    if (!skinny_shape(a, cus, sh)) return hipErrorInvalidValue;
    if (sh.S > 1 && !part) return hipErrorInvalidValue;
    SkinnyArgs d;
    d.q = a.q;
    d.scales = static_cast<const f16 *>(a.scales);
    d.ngroups = (int)a.ngroups;
    d.gshift = 0;
    if (a.ngroups != 1)
        for (int64_t r = a.G / 128; r > 1; r >>= 1) d.gshift++;
    const bool sparse = a.has_ortho;
    d.row_ptr = a.row_ptr;
    d.col = a.col;
    d.vals = static_cast<const f16 *>(a.vals);
    d.phdr = sparse && plan ? static_cast<const uint32_t *>(plan) : nullptr;
    d.chunks = sparse && plan && plan_chunks_bytes(a.N, a.K)
                   ? reinterpret_cast<const uint16_t *>(static_cast<const char *>(plan) + plan_chunks_at(a.N, a.K, a.nnz))
                   : nullptr;
    d.nnz = (int32_t)a.nnz;
    d.x = static_cast<const f16 *>(a.x);
    d.y = static_cast<f16 *>(a.y);
    d.bias = a.bias;
    d.bias_dtype = a.bias_dtype;
    d.M = (int)a.M;
    d.K = (int)a.K;
    d.N = a.N;
    d.nchunks = (int)(a.K / 128);
    d.cps = sh.cps;
    d.S = sh.S;
    d.nblocks = sh.nblocks;
    d.xstride = sh.xstride;
    d.lds_cr = sh.lds_cr;
    d.lds_xs = sh.lds_xs;
    d.lds_sp = sh.lds_sp;
    d.alpha = a.alpha;
    d.part = part;
    // pairs of group-128 scales are read as aligned 32-bit words when every
    // row starts on a pair (even group count, 4-byte aligned scales)
    const bool pairs = (a.ngroups & 1) == 0 && (reinterpret_cast<uintptr_t>(a.scales) & 3) == 0;
    // full slices of 8 chunks with 16-byte scale vectors (GMODE 3)
    // (one token tile: with two the pair loop would not fit the registers)
    const bool full = sh.ntt == 1 && sh.cps == 8 && (int64_t)sh.S * 8 == a.K / 128 &&
                      a.ngroups % 8 == 0 && (reinterpret_cast<uintptr_t>(a.scales) & 15) == 0;
    const int gmode = a.ngroups == 1 ? 0 : (d.gshift != 0 ? 2 : (full ? 3 : (pairs ? 1 : 2)));
    // the plan's slice records (one token tile, full 8-chunk slices): each
    // wave stages its record in its own LDS region
    d.srec = nullptr;
    d.swords = 0;
    d.nslices = (int)(a.K / 1024);
    d.lds_sr = sh.lds_bytes;
    int lds = sh.lds_bytes;
    const int sw = plan ? plan_srec_words(a.N, a.K, a.nnz) : 0;
    if (sparse && gmode == 3 && sh.ntt == 1 && sh.cps == 8 && sw > 0 && lds + 8 * sw * 4 <= 150 * 1024) {
        d.srec = reinterpret_cast<const uint32_t *>(static_cast<const char *>(plan) + plan_srec_at(a.N, a.K, a.nnz));
        d.swords = sw;
        lds += 8 * sw * 4;
    }
    const int blocks = ((sh.nblocks + 7) / 8) * 8 * sh.S;  // padded: see skinny_kernel
    const bool xb = a.io_dtype == ORTH_DT_BF16;
    const hipError_t e = xb ? skinny_launch_x<true>(d, sh.ntt, gmode, sparse, blocks, lds, stream)
                            : skinny_launch_x<false>(d, sh.ntt, gmode, sparse, blocks, lds, stream);
    if (e != hipSuccess || sh.S == 1) return e;
    const int vec4 = (a.N % 4 == 0) ? 1 : 0;
    const int R = skinny_reduce_parts((int)a.M, vec4);
    const unsigned rblocks = (unsigned)(((sh.nblocks + 7) / 8) * 8 * R);
    hipLaunchKernelGGL(skinny_reduce_kernel, dim3(rblocks), dim3(256), 0, stream, part, static_cast<f16 *>(a.y),
                       (int)a.M, a.N, sh.S, vec4, sh.nblocks, R, a.bias, a.bias_dtype, xb ? 1 : 0);
    return hipGetLastError();
}

}  // namespace orth
