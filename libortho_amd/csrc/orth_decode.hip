// Decode dual GEMM for gfx950: up to 16 tokens; the dispatcher gives it 1..4
// (and up to 8 where no mid-batch kernel applies).
//
// Computes what /root/reference/src/dual_gemm.cu:176-225 computes (the
// reference launches one 32-thread block per 32 output rows and walks K
// serially per thread, one byte load per nibble); the work here is laid out
// for CDNA4 instead:
//
//  * A workgroup of 4 waves owns 16 consecutive output rows (one contiguous
//    16*K/2-byte block of the packed weights).  K is cut into 128-wide
//    chunks; wave w takes the contiguous run [w*cpw, (w+1)*cpw) (split-K
//    inside the workgroup, reduced through LDS: deterministic, no atomics).
//  * Per chunk every lane issues ONE 16-byte nontemporal load: lane (row
//    r = lane%16, quarter g = lane/16) takes bytes [64c + 16g, +16) of row r.
//    The first chunk pairs are issued at entry and the rest a fixed number
//    of pairs ahead of the main loop; none is scattered: measured on MI355X,
//    per-lane 2- and 4-byte loads touching 16 rows per instruction cost more
//    than the weight stream.
//  * Each 32-bit word (8 nibbles) becomes 8 FP16 values in registers and
//    feeds v_mfma_f32_16x16x32_f16 as the B operand; the activations (tokens
//    padded to 16) are the A operand.  The tensor core does the K reduction.
//  * Activations staged in LDS (small M*K), each wave staging only its own
//    chunks (so no barrier precedes the main loop): the weights are
//    converted with five bit operations into exact FP16 integers q+1032
//    (even k) / q+72 (odd k), and the FP32 partial of each chunk is corrected
//    by 1032*sum(x even) + 72*sum(x odd) of that chunk, computed while
//    staging.  Activations read from global memory (larger M*K): the bias is
//    subtracted in FP16, exactly.  Either way q is never rounded and q*s is
//    never formed in FP16.
//  * Group scales: G = 128 (one 32-bit load per lane per 8 chunks, broadcast
//    by lane shuffles) or G = 128 * 2^j; per-row scales (G = K) are applied
//    once at the end.
//  * Sparse ortho term: the CSR entries of the workgroup's 16 rows are
//    contiguous; they are loaded with 16-byte loads into LDS (bounds first,
//    then the block), then 16 lanes per row sum v*x with x from LDS, reduce
//    with DPP moves, and lane 0 of the row adds alpha*sum after the base term
//    and stores, as /root/reference/src/dual_gemm.cu:212-221 does.  alpha <=
//    0 takes a kernel without the term, which never touches the CSR arrays.
//  * With an ortho plan, each wave reads the entries of its K quarter from
//    the plan's record of (block, quarter) instead: packed column|value words
//    at an address that needs no row pointer, loaded with the activations and
//    summed (4 lanes per row) before the main loop, while the weights are in
//    flight; no workgroup barrier is needed since a wave's entries use only
//    the activations it staged.  A quarter whose entries did not fit its
//    record reads the rows' CSR, filtered to the quarter's columns.
#include <atomic>
#include <type_traits>

#include "orth_common.h"

namespace orth {

constexpr int kDecodeW = 4;       // waves per workgroup
constexpr int kDecodeNT = 64 * kDecodeW;
constexpr int kDecodeESlots = 2;  // CSR entries staged per thread: 4 * slots
constexpr int kDecodeEStaged = kDecodeESlots * 4 * kDecodeNT;

constexpr int kDecodeMaxGroup = 4;  // layers one decode launch may take

// The per-layer part of a decode launch (weights, ortho, output).
struct DecodeLayerArgs {
    const uint8_t *q;
    const f16 *scales;
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int32_t nnz;
    int csr_vec;
    f16 *y;
    int64_t N;
    float alpha;
    const uint32_t *rec;
    const void *bias;
    int bias_dtype;
};

struct DecodeArgs {
    const uint8_t *q;
    const f16 *scales;
    int ngroups;
    int gshift;        // group of chunk c is c >> gshift (G = 128 << gshift)
    int scale_pairs;   // group-128 scales readable as aligned 32-bit pairs
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int32_t nnz;
    int csr_vec;       // col 16-byte and vals 8-byte aligned: vector staging
    const f16 *x;
    f16 *y;
    int M;
    int nchunks;       // K / 128
    int K;
    int64_t N;
    int cpw;           // chunks per wave, even, <= the CPW template bound
    int xstride;       // LDS row stride of the staged activations, in halves
    int lds_red;       // byte offsets of the LDS regions
    int lds_cr;
    int lds_xs;
    int lds_e;
    float alpha;
    int has_ortho;
    const uint32_t *rec;   // plan quarter records: qwords words per (16-row block, wave)
    int qwords;            // a multiple of 256, at most 2048; 0 without a plan
    int deep;              // (host) fewer than two workgroups per CU: deeper weight prefetch
    const void *bias;      // [N] added after rounding (out_f16), or null
    int bias_dtype;
    // A group launch: layers 1 .. nextra of the same shape class (K, scale
    // layout, token count, ortho mode, record size) reading the same
    // activations; layer 0 is the fields above.  Workgroups [blk0[l],
    // blk0[l + 1]) take layer l.
    int nextra;
    DecodeLayerArgs extra[kDecodeMaxGroup - 1];
    int blk0[kDecodeMaxGroup + 1];
};

// Weights pass through LDS (whole-line loads, transposed on the way) for
// one or two tokens with staged activations: there the weight stream is all
// the kernel does, and the LDS holds a wave's weights beside the activations
// with three workgroups per CU.
constexpr bool decode_wt(int mt, bool xlds) { return xlds && mt <= 2; }

// GMODE: 0 per-row scale (G == K); 4 the same with every wave taking
// exactly CPW chunks (K == 512 * CPW); 1 G = 128 with the scales of 8 chunks
// readable as one aligned 16-byte vector (K % 4096 == 0, so every wave takes
// exactly CPW chunks); 3 G = 128 with scales readable as aligned 32-bit
// pairs; 2 any G = 128 * 2^j (one 16-bit load per chunk).
// CPW: compile-time bound of the chunks per wave.  The weight loads of the
// first PDP = min(PD, CPW / 2) chunk pairs are issued at entry; with all CPW
// chunks valid the main loop issues pair j + PDP as it takes pair j, so a
// wave never has more than PDP + 1 pairs in flight and its vector-memory
// instructions do not queue behind the weight streams of the whole CU
// before it can compute.  PD 1 when a CU holds two or more workgroups (c2:
// 688 workgroups), 3 when it holds one (4096-row layers), 2 otherwise.
// SPARSE: 0 no ortho term; 1 ortho term with the workgroup's CSR block
// staged through LDS (16-byte aligned columns, nnz >= 4); 2 ortho term read
// entry by entry in the epilogue; 3 / 4 / 5 / 6 the plan's records of the
// block's four K quarters (256 / 512 / <= 1024 / <= 2048 words), one per
// wave, staged through LDS and summed before the main loop (XLDS only).
//
// XB: BF16 activations and output (staged activations only): the weights
// become the exact BF16 integers q + 136 (every half biased alike, the
// chunk's bias 136 * sum x) and feed v_mfma_f32_16x16x32_bf16.
//
// Every global load below is unconditional with a clamped, always valid
// address: a load under a branch makes the compiler's wait-count insertion
// fall back to waiting for all outstanding loads, which serialises the
// kernel behind its own weight stream.
template <int MT, int GMODE, bool XLDS, int CPW, int SPARSE, int PD, bool XB>
__global__ void __launch_bounds__(kDecodeNT) decode_kernel(DecodeArgs a) {
    // a group launch: this workgroup's layer and its block within the layer.
    // Constant indices only: an index computed at run time into the
    // argument struct would move the whole struct to scratch memory.
    static_assert(kDecodeMaxGroup == 4, "the layer pick below takes up to four layers");
    int bid = blockIdx.x;
    if (a.nextra > 0) {
        const int b1 = a.blk0[1], b2 = a.blk0[2], b3 = a.blk0[3];
        const int l = (bid >= b1 ? 1 : 0) + (a.nextra >= 2 && bid >= b2 ? 1 : 0) + (a.nextra >= 3 && bid >= b3 ? 1 : 0);
        if (l > 0) {
            bid -= l == 1 ? b1 : (l == 2 ? b2 : b3);
#define ORTH_PICK(f) a.f = l == 1 ? a.extra[0].f : (l == 2 ? a.extra[1].f : a.extra[2].f)
            ORTH_PICK(q);
            ORTH_PICK(scales);
            ORTH_PICK(row_ptr);
            ORTH_PICK(col);
            ORTH_PICK(vals);
            ORTH_PICK(nnz);
            ORTH_PICK(csr_vec);
            ORTH_PICK(y);
            ORTH_PICK(N);
            ORTH_PICK(alpha);
            ORTH_PICK(rec);
            ORTH_PICK(bias);
            ORTH_PICK(bias_dtype);
#undef ORTH_PICK
        }
    }
    constexpr int W = kDecodeW;
    constexpr int NT = kDecodeNT;
    constexpr int RT = 16;
    constexpr int MI = MT < 4 ? MT : 4;        // live D rows per lane group (tokens 4g + i)
    constexpr bool GROUPED = GMODE != 0 && GMODE != 4;
    constexpr bool FULL = GMODE == 1 || GMODE == 4;  // every wave has CPW chunks
    constexpr int PDP = CPW / 2 < PD ? CPW / 2 : PD;  // weight pairs in flight ahead of the main loop
    constexpr int PDC = 2 * PDP;                     // the same in chunks (direct loads)
    // record kernels issue PDP more pairs after the record barrier, before
    // the sparse sums, so the stream does not pause while those are formed;
    // the main loop then runs PDM pairs ahead
    constexpr int PDM = (SPARSE >= 3 && FULL) ? (2 * PDP < CPW / 2 ? 2 * PDP : CPW / 2) : PDP;
    constexpr int PDMC = 2 * PDM;
    constexpr int XIT = (CPW * 16 + 63) / 64;  // 16-byte activation pieces per lane per token
    constexpr int ES = kDecodeESlots;
    // WT: the weights pass through LDS (see decode_wt)
    constexpr bool WT = decode_wt(MT, XLDS);
    constexpr int WREG = CPW * 1024;  // WT: LDS bytes of a wave's weight region
    constexpr bool REC = SPARSE >= 3;
    constexpr int ER = 1 << (SPARSE >= 3 ? SPARSE - 3 : 0);  // record: 16-byte loads per lane
    static_assert(!REC || XLDS, "the record kernels gather staged activations");
    static_assert(!XB || XLDS, "BF16 activations are staged");
    // one chunk-word of weights as MFMA B operand halves, and the MFMA
    auto wconv = [](uint32_t w, uint32_t out[4]) {
        if constexpr (XB) int4x8_to_bf16_biased(w, out);
        else int4x8_to_f16_biased(w, out);
    };
    auto mfma = [](u32x4 av, const uint32_t b[4], f32x4 c) -> f32x4 {
        if constexpr (XB)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                           __builtin_bit_cast(bf16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                          __builtin_bit_cast(f16x8, u32x4{b[0], b[1], b[2], b[3]}),
                                                          c, 0, 0, 0);
    };
    auto store_y = [&](int64_t i, float v, int64_t n) {
        if constexpr (XB) reinterpret_cast<uint16_t *>(a.y)[i] = out_bf16(v, a.bias, a.bias_dtype, n);
        else a.y[i] = out_f16(v, a.bias, a.bias_dtype, n);
    };

    extern __shared__ __align__(16) unsigned char smem[];
    // WT: wave w's region holds its weights during the main loop, then its
    // split-K partials (1 KB), CSR columns (2 KB) and values (1 KB)
    float *cr = reinterpret_cast<float *>(smem + a.lds_cr);     // [MT][nchunks] bias sums (XLDS)
    f16 *xs = reinterpret_cast<f16 *>(smem + a.lds_xs);         // [MT][xstride] activations
    // split-K partials of wave w: [16 tokens][16 rows]
    auto red = [&](int w) -> float * {
        return reinterpret_cast<float *>(smem + (WT ? w * WREG : a.lds_red + w * 1024));
    };
    // staged CSR entry li: WT keeps entries [512 w, 512 w + 512) in wave w's region
    auto ec_at = [&](int32_t li) -> int32_t * {
        return WT ? reinterpret_cast<int32_t *>(smem + (li >> 9) * WREG + 1024) + (li & 511)
                  : reinterpret_cast<int32_t *>(smem + a.lds_e) + li;
    };
    auto ev_at = [&](int32_t li) -> f16 * {
        return WT ? reinterpret_cast<f16 *>(smem + (li >> 9) * WREG + 3072) + (li & 511)
                  : reinterpret_cast<f16 *>(smem + a.lds_e + kDecodeEStaged * 4) + li;
    };

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int nl = lane & 15;  // B column (weight row) and A row (token) of this lane
    const int g = lane >> 4;   // which 32-k quarter of a chunk
    const int64_t n0 = (int64_t)bid * RT;
    const int K = a.K;
    const int c_lo = wave * a.cpw;
    const int nci = max(0, min(a.cpw, a.nchunks - c_lo));  // uniform
    const int clast = a.nchunks - 1;                        // last valid chunk of a row
    const int64_t rows_here = a.N - n0;
    const int last_row = (int)(rows_here < 16 ? rows_here - 1 : 15);
    const int my_row = min(nl, last_row);

    // ---- activations of this wave's chunks (L2-resident), contiguous;
    //      pieces past the wave's range re-read the last valid piece
    u32x4 xreg[XLDS ? MT * XIT : 1];
    const int xlast = a.nchunks * 16 - 1;  // last 16-byte piece of a token row
    if (XLDS) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const f16 *xr = a.x + (int64_t)min(m, a.M - 1) * K;
#pragma unroll
            for (int it = 0; it < XIT; it++) {
                const int pc = min(c_lo * 16 + lane + 64 * it, xlast);
                xreg[m * XIT + it] = *reinterpret_cast<const u32x4 *>(xr + pc * 8);
            }
        }
    }

    // ---- REC: this wave's plan record (the block's 16 rows, the wave's K
    //      quarter): its address needs no other load, so it is issued before
    //      the weights and returns with the activations
    u32x4 rv[ER];
    if (REC) {
        const uint32_t *rb = a.rec + ((int64_t)bid * 4 + wave) * a.qwords;
#pragma unroll
        for (int r = 0; r < ER; r++)
            rv[r] = *reinterpret_cast<const u32x4 *>(rb + min(4 * (lane + 64 * r), a.qwords - 4));
    }

    // ---- CSR bounds: this thread's epilogue row, and the workgroup block
    //      (loaded here, used after the staging).  The block bounds come
    //      from one vector load (lane i: row_ptr[n0 + i]) read with
    //      readlane: as a scalar load it would be issued late and waited for
    //      before the CSR block loads.
    const int rl = tid >> 4, sub = tid & 15;
    int32_t r_lo = 0, r_hi = 0, pv = 0;
    if (SPARSE && !REC) {
        r_lo = a.row_ptr[n0 + min(rl, last_row)];
        r_hi = a.row_ptr[n0 + min(rl, last_row) + 1];
        pv = a.row_ptr[n0 + min(lane, last_row + 1)];
    }

    // ---- per-row scale of the row this thread combines at the end
    f16 srow = (f16)0.0f;
    if (!GROUPED) srow = a.scales[n0 + min((SPARSE && !REC) ? tid >> 4 : tid & 15, last_row)];

    // ---- group scales of this lane's row nl: chunks c_lo + 8i .. + 8i + 7
    //      as one 16-byte vector (GMODE 1), chunks c_lo + 2i, + 2i + 1 as one
    //      32-bit pair (GMODE 3), or one scale per chunk (GMODE 2)
    const f16 *sbase = a.scales + (n0 + my_row) * (int64_t)a.ngroups;
    u32x4 sv[GMODE == 1 ? (CPW + 7) / 8 : 1];
    uint32_t sw[GMODE == 3 ? CPW / 2 : 1];
    f16 sh[GMODE == 2 ? CPW : 1];
    if (GMODE == 1) {
#pragma unroll
        for (int i = 0; i < (CPW + 7) / 8; i++)
            sv[i] = *reinterpret_cast<const u32x4 *>(sbase + min(c_lo + 8 * i, clast & ~7));
    } else if (GMODE == 3) {
#pragma unroll
        for (int i = 0; i < CPW / 2; i++)
            sw[i] = *reinterpret_cast<const uint32_t *>(sbase + (min(c_lo + 2 * i, clast) & ~1));
    } else if (GMODE == 2) {
#pragma unroll
        for (int p = 0; p < CPW; p++) sh[p] = sbase[min(c_lo + p, clast) >> a.gshift];
    }

    // ---- weights (nontemporal).  Direct: lane (row nl, g) loads the 16
    //      bytes of chunk p it feeds to the MFMA (half a 128-byte line per
    //      row per instruction).  WT: chunk pair j (128 bytes of each row),
    //      rows 8h .. 8h + 7 per instruction, so that every instruction reads
    //      whole lines: lane l takes row 8h + l/8, 16-byte slot l%8 of the
    //      row's line, which holds logical slot s = (l%8) ^ ((row/2) & 7)
    //      (the XOR spreads the MFMA-layout reads below over all LDS banks).
    u32x4 wv[WT ? 1 : CPW];
    u32x4 wq[WT ? CPW / 2 : 1][2];
    const uint8_t *qrow = a.q + (n0 + my_row) * (int64_t)(K >> 1) + g * 16;
    const uint8_t *qh[2];
    int sh2[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int r = 8 * h + (lane >> 3);
        const int sl = (lane & 7) ^ ((r >> 1) & 7);
        qh[h] = a.q + (n0 + min(r, last_row)) * (int64_t)(K >> 1) + (sl & 3) * 16;
        sh2[h] = sl >> 2;  // which chunk of the pair
    }
    auto load_chunk = [&](int p) {
        wv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + min(c_lo + p, clast) * 64));
    };
    auto load_pair = [&](int j) {
#pragma unroll
        for (int h = 0; h < 2; h++)
            wq[j][h] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(qh[h] + min(c_lo + 2 * j + sh2[h], clast) * 64));
    };
    if (!WT) {
#pragma unroll
        for (int p = 0; p < PDC; p++) load_chunk(p);
    } else {
#pragma unroll
        for (int j = 0; j < PDP; j++) load_pair(j);
    }

    // ---- activations from global memory (no LDS staging): 64 bytes per
    //      lane per chunk; A rows beyond M repeat row 0 (outputs unused)
    u32x4 ag[XLDS ? 1 : CPW][4];
    if (!XLDS) {
        const f16 *xrow = a.x + (int64_t)(nl < a.M ? nl : 0) * K + g * 32;
#pragma unroll
        for (int p = 0; p < CPW; p++) {
            const int c = min(c_lo + p, clast);
#pragma unroll
            for (int j = 0; j < 4; j++) ag[p][j] = *reinterpret_cast<const u32x4 *>(xrow + (c * 128 + 8 * j));
        }
    }

    // ---- stage this wave's activations (interleaved k order) and their
    //      per-chunk bias sums; only this wave reads them before the end
    const int wpieces = nci * 16;
    // SGB: the bias sums of token i < MI and chunk p are the same in every
    // lane (tokens (4 g + i) & (MT - 1) = i): read from the staging registers
    // into scalar registers instead of LDS
    constexpr bool SGB = XLDS && MT <= 4 && MT * CPW <= 32;
    float bsum[SGB ? MT : 1][SGB ? XIT : 1];
    if (XLDS) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
#pragma unroll
            for (int it = 0; it < XIT; it++) {
                {
                    const int pc = lane + 64 * it;
                    u32x4 v = xreg[m * XIT + it];
                    if (m >= a.M) v = u32x4{0, 0, 0, 0};
                    const f16x8 h = __builtin_bit_cast(f16x8, v);
                    // even k weigh 1032, odd k weigh 72 (see int4x8_to_f16_biased);
                    // BF16: every k weighs 136 (int4x8_to_bf16_biased)
                    const float e = (x16_to_f32<XB>(h[0]) + x16_to_f32<XB>(h[2])) +
                                    (x16_to_f32<XB>(h[4]) + x16_to_f32<XB>(h[6]));
                    const float o = (x16_to_f32<XB>(h[1]) + x16_to_f32<XB>(h[3])) +
                                    (x16_to_f32<XB>(h[5]) + x16_to_f32<XB>(h[7]));
                    const float b = group_sum<16>(XB ? 136.0f * (e + o) : 1032.0f * e + 72.0f * o);  // 16 pieces of a chunk
                    if (SGB) bsum[m][it] = b;
                    if (pc < wpieces) {
                        *reinterpret_cast<u32x4 *>(xs + (m * a.xstride + c_lo * 128 + pc * 8)) = permute_x8(v);
                        if ((pc & 15) == 0) cr[m * a.nchunks + c_lo + (pc >> 4)] = b;
                    }
                }
            }
        }
    }

    // ---- CSR block of the workgroup: 4 entries per thread per slot, from the
    //      aligned start eb.  Addresses are clamped to the workgroup's last
    //      aligned group (threads past the block re-read one cached line) and
    //      to the last aligned group of the arrays (in bounds).  Issued after
    //      the staging (held there by the scheduling barrier): the addresses
    //      wait for the row pointers, and the staging need not.
    __builtin_amdgcn_sched_barrier(0);
    int32_t rs = 0, re = 0, e0 = 0, e1 = 0;
    if (SPARSE && !REC) {
        rs = min(max(r_lo, 0), a.nnz);
        re = min(max(r_hi, rs), a.nnz);
        if (rl > last_row) re = rs;  // rows past N have no entries
        e0 = min(max(__builtin_amdgcn_readlane(pv, 0), 0), a.nnz);
        e1 = min(max(__builtin_amdgcn_readlane(pv, last_row + 1), e0), a.nnz);
    }
    // ---- REC: the wave stages its record in its own LDS region and sums
    //      v * x over the entries of its quarter, 4 lanes per row (entries
    //      start + tg + 4 u, in order), reduced over the quad; the sums wait in
    //      the region (over the record) for the epilogue, which adds
    //      alpha * (sum over the 4 quarters) after the dense term.  No
    //      workgroup barrier: the wave reads only activations it staged.
    //      The remaining weight pairs are issued first.  Without a matching
    //      record (another layer's plan, or entries that did not fit) the
    //      rows are read from the CSR, filtered to the quarter's columns.
    float sacc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) sacc[m] = 0.f;
    if (REC) {
        uint32_t *er = reinterpret_cast<uint32_t *>(smem + a.lds_e) + wave * a.qwords;
#pragma unroll
        for (int r = 0; r < ER; r++) {
            const int o = 4 * (lane + 64 * r);
            if (o < a.qwords) *reinterpret_cast<u32x4 *>(er + o) = rv[r];
        }
        __builtin_amdgcn_wave_barrier();  // (same wave: LDS keeps the order)
        if (FULL) {
            if (WT) {
#pragma unroll
                for (int j = PDP; j < PDM; j++) load_pair(j);
            } else {
#pragma unroll
                for (int p = PDC; p < PDMC; p++) load_chunk(p);
            }
        }
        const int qr = lane >> 2, tg = lane & 3;  // row of the block, lane of its quad
        const int32_t col0 = c_lo * 128, col1 = (c_lo + nci) * 128;
        auto add_entry = [&](bool ok_e, int c, float vv) {
            const int cc = ok_e ? c : 0;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const float xv = x16_to_f32<XB>(xs[m * a.xstride + ((cc & ~7) | interleaved_pos(cc & 7))]);
                sacc[m] = __builtin_fmaf(ok_e ? vv : 0.f, ok_e ? xv : 0.f, sacc[m]);
            }
        };
        const bool ok = (er[0] == plan_cell_tag(kCellQuarter, a.N, K, a.nnz, a.qwords, bid, wave)) &
                        (er[1] == 0u);  // (uniform)
        if (ok) {
            const uint32_t h = er[2 + qr];
            const int32_t lo = (int32_t)(h & 0xffffu);
            const int32_t hi = qr <= last_row ? (int32_t)(h >> 16) : lo;
            const uint32_t *ee = er + kCellHdrWords;
            constexpr int U = 4;
            for (int32_t j0 = lo + tg; j0 < hi; j0 += 4 * U) {
                uint32_t w[U];
#pragma unroll
                for (int u = 0; u < U; u++) w[u] = ee[min(j0 + 4 * u, hi - 1)];
#pragma unroll
                for (int u = 0; u < U; u++)
                    add_entry(j0 + 4 * u < hi, (int)(w[u] & 0xffffu) + col0,
                              (float)__builtin_bit_cast(f16, (uint16_t)(w[u] >> 16)));
            }
        } else {
            int32_t fs = 0, fe = 0;
            csr_row_range(a.row_ptr, n0 + min(qr, last_row), a.nnz, fs, fe);
            if (qr > last_row) fe = fs;
            for (int32_t j = fs + tg; j < fe; j += 4) {
                const int32_t c = a.col[j];
                add_entry(c >= col0 && c < col1, c, (float)a.vals[j]);
            }
        }
        // quad sums (fixed order), kept for the epilogue in the record region
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float v = sacc[m];
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
            sacc[m] = v;
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read the record
        if (tg == 0) {
#pragma unroll
            for (int m = 0; m < MT; m++) reinterpret_cast<float *>(er)[m * 16 + qr] = sacc[m];
        }
    }
    const int32_t eb = e0 & ~3;
    const int32_t last4 = (a.nnz - 4) & ~3;
    const int32_t wlast4 = min(max((e1 - 1) & ~3, eb), last4);
    u32x4 ecv[ES];
    uint2 evv[ES];
    // staged slot of thread (wave, lane), group s: entries eb + 4 * slot ..
    auto e_slot = [&](int s) -> int {
        return WT ? wave * (kDecodeEStaged / W) + 4 * (lane + 64 * s) : 4 * (tid + NT * s);
    };
    if (SPARSE == 1) {
#pragma unroll
        for (int s = 0; s < ES; s++) {
            const int32_t ic = min(eb + e_slot(s), wlast4);
            ecv[s] = *reinterpret_cast<const u32x4 *>(a.col + ic);
            evv[s] = *reinterpret_cast<const uint2 *>(a.vals + ic);
        }
    }

    // ---- main loop over this wave's chunks: straight-line code when the
    //      wave has all CPW chunks (FULL), so that the reads and conversions
    //      of later chunks overlap the matrix ops of earlier ones
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    float bias_acc[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) bias_acc[i] = 0.f;
    const f16 *xs_lane = xs + ((nl & (MT - 1)) * a.xstride + g * 32 + c_lo * 128);
    const float *cr_lane[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) cr_lane[i] = cr + ((4 * g + i) & (MT - 1)) * a.nchunks + c_lo;
    // bias sum of token i, chunk p of this wave
    auto bias_of = [&](int i, int p) -> float {
        if constexpr (SGB)
            return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bsum[i][p >> 2]), 16 * (p & 3)));
        else
            return cr_lane[i][p];
    };
    // WT: this wave's weight region as 16-byte slots
    u32x4 *wl = reinterpret_cast<u32x4 *>(smem + wave * WREG);
    // one chunk: weights wp (4 words), activations of chunk p; FP32 partial
    auto chunk_mfma = [&](const u32x4 &wp, int p, f32x4 part) -> f32x4 {
        const uint32_t words[4] = {wp.x, wp.y, wp.z, wp.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t b[4];
            u32x4 av;
            if (XLDS) {
                wconv(words[j], b);
                av = *reinterpret_cast<const u32x4 *>(xs_lane + (p * 128 + 8 * j));
            } else {
                int4x8_to_f16_interleaved(words[j], b);
                av = permute_x8(ag[p][j]);
            }
            part = mfma(av, b, part);
        }
        return part;
    };
    // chunk p's partial into acc: scaled (GROUPED) after its bias sum is removed
    auto chunk_done = [&](const f32x4 &part, int p) {
        float s;
        if (GMODE == 1 || GMODE == 3) {
            const uint32_t w2 = GMODE == 1 ? sv[p >> 3][(p >> 1) & 3] : sw[p >> 1];
            s = (float)__builtin_bit_cast(f16, (uint16_t)((p & 1) ? (w2 >> 16) : (w2 & 0xffffu)));
        } else {
            s = (float)sh[p];
        }
#pragma unroll
        for (int i = 0; i < MI; i++) {
            float v = part[i];
            if (XLDS) v -= bias_of(i, p);
            acc[i] += s * v;
        }
    };
    // WT: pair j (chunks 2j, 2j + 1) to LDS as loaded, then lane (row nl, g)
    // reads logical slot 4 h + g of row nl for chunk 2j + h
    auto pair_to_lds = [&](int j) {
        wl[(2 * j) * 64 + lane] = wq[j][0];
        wl[(2 * j + 1) * 64 + lane] = wq[j][1];
        __builtin_amdgcn_wave_barrier();  // (same wave: LDS keeps the order)
    };
    auto wt_read = [&](int j, int h) -> u32x4 {
        const int phys = (4 * h + g) ^ ((nl >> 1) & 7);
        return wl[(2 * j + (nl >> 3)) * 64 + (nl & 7) * 8 + phys];
    };
    auto main_loop = [&](auto full) {
        constexpr bool FULL = decltype(full)::value;
        if constexpr (FULL && GROUPED && CPW % 2 == 0) {
            // chunks in pairs, the two MFMA chains interleaved
#pragma unroll
            for (int j = 0; j < CPW / 2; j++) {
                u32x4 w0, w1;
                if (WT) {
                    pair_to_lds(j);
                    w0 = wt_read(j, 0);
                    w1 = wt_read(j, 1);
                } else {
                    w0 = wv[2 * j];
                    w1 = wv[2 * j + 1];
                    if (2 * j + PDMC < CPW) load_chunk(2 * j + PDMC);
                    if (2 * j + 1 + PDMC < CPW) load_chunk(2 * j + 1 + PDMC);
                }
                const uint32_t u0[4] = {w0.x, w0.y, w0.z, w0.w};
                const uint32_t u1[4] = {w1.x, w1.y, w1.z, w1.w};
                f32x4 pa = f32x4{0.f, 0.f, 0.f, 0.f}, pb = pa;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t b0[4], b1[4];
                    u32x4 a0, a1;
                    if (XLDS) {
                        wconv(u0[k], b0);
                        wconv(u1[k], b1);
                        a0 = *reinterpret_cast<const u32x4 *>(xs_lane + ((2 * j) * 128 + 8 * k));
                        a1 = *reinterpret_cast<const u32x4 *>(xs_lane + ((2 * j + 1) * 128 + 8 * k));
                    } else {
                        int4x8_to_f16_interleaved(u0[k], b0);
                        int4x8_to_f16_interleaved(u1[k], b1);
                        a0 = permute_x8(ag[2 * j][k]);
                        a1 = permute_x8(ag[2 * j + 1][k]);
                    }
                    pa = mfma(a0, b0, pa);
                    pb = mfma(a1, b1, pb);
                }
                if (WT && j + PDM < CPW / 2) load_pair(j + PDM);
                chunk_done(pa, 2 * j);
                chunk_done(pb, 2 * j + 1);
            }
        } else {
            if constexpr (!FULL) {
                // the rest of the weights at once (addresses clamped, branch-free)
                if (WT) {
#pragma unroll
                    for (int j = PDP; j < CPW / 2; j++) load_pair(j);
                } else {
#pragma unroll
                    for (int p = PDC; p < CPW; p++) load_chunk(p);
                }
            }
#pragma unroll
            for (int p = 0; p < CPW; p++) {
                if (FULL || p < nci) {  // uniform
                    u32x4 wp;
                    if (WT) {
                        if ((p & 1) == 0) {
                            pair_to_lds(p >> 1);
                            if (FULL && (p >> 1) + PDM < CPW / 2) load_pair((p >> 1) + PDM);
                        }
                        wp = wt_read(p >> 1, p & 1);
                    } else {
                        wp = wv[p];
                        if (FULL && p + PDMC < CPW) load_chunk(p + PDMC);
                    }
                    if (GROUPED) {
                        chunk_done(chunk_mfma(wp, p, f32x4{0.f, 0.f, 0.f, 0.f}), p);
                    } else {
                        acc = chunk_mfma(wp, p, acc);
                        if (XLDS) {
#pragma unroll
                            for (int i = 0; i < MI; i++) bias_acc[i] += bias_of(i, p);
                        }
                    }
                }
            }
        }
    };
    main_loop(std::integral_constant<bool, FULL>{});
    if (!GROUPED && XLDS) {
#pragma unroll
        for (int i = 0; i < MI; i++) acc[i] -= bias_acc[i];
    }

    // ---- split-K partials and the staged CSR block to LDS
#pragma unroll
    for (int i = 0; i < 4; i++) red(wave)[(4 * g + i) * 16 + nl] = acc[i];
    if (SPARSE == 1) {
#pragma unroll
        for (int s = 0; s < ES; s++) {
            const int slot = e_slot(s);
            *reinterpret_cast<u32x4 *>(ec_at(slot)) = ecv[s];
            *reinterpret_cast<uint2 *>(ev_at(slot)) = evv[s];
        }
    }
    __syncthreads();  // every wave's activation chunks and the CSR block are in LDS

    // ---- sparse ortho term: 16 lanes per output row.  Entries staged in
    //      LDS are taken four per lane per pass: their column/value reads,
    //      then their activation reads, are issued together (one LDS or L2
    //      round trip each instead of one per entry); entries past the
    //      staged block (very dense rows) are read from memory one by one.
    if (SPARSE && !REC) {
        constexpr int U = 4;
        const int32_t staged_hi = SPARSE == 1 ? min(min(eb + kDecodeEStaged, last4 + 4), e1) : eb;
        const int32_t fast_hi = min(re, staged_hi);
        for (int32_t j0 = rs + sub; j0 < fast_hi; j0 += 16 * U) {
            int32_t c[U];
            float v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int32_t j = j0 + 16 * u;
                const int32_t li = min(j, fast_hi - 1) - eb;  // in [0, kDecodeEStaged)
                c[u] = *ec_at(li);
                v[u] = (float)*ev_at(li);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                // entries past the row, or with a column outside [0, K), add nothing
                const bool ok = (j0 + 16 * u < fast_hi) & (c[u] >= 0) & (c[u] < K);
                const int cc = ok ? c[u] : 0;
                const float vv = ok ? v[u] : 0.f;
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    float xv;
                    if (XLDS) xv = x16_to_f32<XB>(xs[m * a.xstride + ((cc & ~7) | interleaved_pos(cc & 7))]);
                    else xv = x16_to_f32<XB>(a.x[(int64_t)min(m, a.M - 1) * K + cc]);
                    sacc[m] = __builtin_fmaf(vv, ok ? xv : 0.f, sacc[m]);
                }
            }
        }
        // first entry of this lane's residue class (mod 16) at or past fast_hi
        const int32_t d = fast_hi - (rs + sub);
        for (int32_t j = rs + sub + (d > 0 ? (d + 15) / 16 * 16 : 0); j < re; j += 16) {
            const int32_t c = a.col[j];
            const float v = (float)a.vals[j];
            if (c >= 0 && c < K) {
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    float xv;
                    if (XLDS) xv = x16_to_f32<XB>(xs[m * a.xstride + ((c & ~7) | interleaved_pos(c & 7))]);
                    else xv = x16_to_f32<XB>(a.x[(int64_t)min(m, a.M - 1) * K + c]);
                    sacc[m] = __builtin_fmaf(v, xv, sacc[m]);
                }
            }
        }
        // lane 0 of each row combines the split-K partials (visible since the
        // barrier above), scales, adds alpha * sparse and stores
        const int64_t n = n0 + rl;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float s = group_sum<16>(sacc[m]);
            if (sub == 0 && m < a.M && n < a.N) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < W; w++) v += red(w)[m * 16 + rl];
                if (!GROUPED) v *= (float)srow;
                v += a.alpha * s;
                store_y((int64_t)m * a.N + n, v, n);
            }
        }
        return;
    }

    // ---- combine split-K partials (visible since the barrier above), scale,
    //      add alpha * (the quarters' sparse sums, REC), store
    if (tid < MT * RT) {
        const int m = tid >> 4, r = tid & 15;
        const int64_t n = n0 + r;
        if (m < a.M && n < a.N) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < W; w++) v += red(w)[m * 16 + r];
            if (!GROUPED) v *= (float)srow;
            if (REC) {
                float sp = 0.f;
#pragma unroll
                for (int w = 0; w < W; w++) sp += (reinterpret_cast<const float *>(smem + a.lds_e) + w * a.qwords)[m * 16 + r];
                v += a.alpha * sp;
            }
            store_y((int64_t)m * a.N + n, v, n);
        }
    }
}

// ------------------------------------------------------------------ host

static const int64_t kDecodeLdsMax = 160 * 1024;

// LDS layout of decode_kernel<MT, *, XLDS, CPW, *>: weight regions (WT) or
// split-K partials, bias sums, activations, staged CSR block (outside the
// weight regions when not WT) or plan record (rec_words > 0).  Returns the
// bytes.
static int64_t decode_lds_layout(DecodeArgs &d, int mt, bool xlds, int cpw_bound, int rec_words) {
    auto al = [](int64_t v) { return (v + 15) & ~int64_t(15); };
    const bool wt = decode_wt(mt, xlds);
    int64_t off = wt ? (int64_t)kDecodeW * cpw_bound * 1024 : (int64_t)kDecodeW * 1024;
    d.lds_red = 0;
    d.lds_cr = (int)off;
    if (xlds) off = al(off + (int64_t)mt * d.nchunks * 4);
    d.lds_xs = (int)off;
    if (xlds) off = al(off + (int64_t)mt * d.xstride * 2);
    d.lds_e = (int)off;
    if (rec_words > 0) off += (int64_t)rec_words * 4;
    else if (!wt && d.has_ortho && d.csr_vec) off += (int64_t)kDecodeEStaged * (4 + 2);
    return off;
}

template <int MT, int GMODE, bool XLDS, int CPW, int SPARSE, int PD, bool XB>
static hipError_t launch_decode_kp(const DecodeArgs &d, int64_t lds, hipStream_t stream) {
    // more than 64 KB of dynamic LDS must be allowed once per device (the
    // attribute call is idempotent, so two threads racing to set it is harmless)
    static std::atomic<int> allowed[64];
    int dev = 0;
    if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 &&
        !allowed[dev].load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(decode_kernel<MT, GMODE, XLDS, CPW, SPARSE, PD, XB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDecodeLdsMax);
        if (e != hipSuccess) return e;
        allowed[dev].store(1, std::memory_order_release);
    }
    const unsigned blocks = d.nextra > 0 ? (unsigned)d.blk0[d.nextra + 1] : (unsigned)((d.N + 15) / 16);
    hipLaunchKernelGGL((decode_kernel<MT, GMODE, XLDS, CPW, SPARSE, PD, XB>), dim3(blocks), dim3(kDecodeNT),
                       (uint32_t)lds, stream, d);
    return hipGetLastError();
}

// Prefetch depth: full-width kernels (GMODE 1 and 4) by CU occupancy, the
// others issue everything at entry past the first pairs anyway.
template <int MT, int GMODE, bool XLDS, int CPW, int SPARSE, bool XB>
static hipError_t launch_decode_k(const DecodeArgs &d, int64_t lds, hipStream_t stream) {
    if constexpr (GMODE == 1 || GMODE == 4)
        return d.deep ? launch_decode_kp<MT, GMODE, XLDS, CPW, SPARSE, 3, XB>(d, lds, stream)
                      : launch_decode_kp<MT, GMODE, XLDS, CPW, SPARSE, 1, XB>(d, lds, stream);
    else
        return launch_decode_kp<MT, GMODE, XLDS, CPW, SPARSE, 2, XB>(d, lds, stream);
}

// XB: the BF16 instantiations take the plan records or no ortho term only
// (decode_bf16_supported).
template <int MT, int GMODE, bool XLDS, int CPW, bool XB = false>
static hipError_t launch_decode_t(const DecodeArgs &d0, hipStream_t stream) {
    DecodeArgs d = d0;
    // GMODE 1 and 4 kernels take exactly CPW chunks in every wave
    if ((GMODE == 1 || GMODE == 4) && !(d.cpw == CPW && d.nchunks == 4 * CPW)) return hipErrorInvalidValue;
    if constexpr (XLDS && MT <= 4) {
        // plan records when the LDS takes them (else the CSR block below)
        if (d.has_ortho && d.qwords > 0) {
            const int64_t lds = decode_lds_layout(d, MT, XLDS, CPW, kDecodeW * d.qwords);
            if (lds <= kDecodeLdsMax) {
                if (d.qwords == 256) return launch_decode_k<MT, GMODE, XLDS, CPW, 3, XB>(d, lds, stream);
                if (d.qwords == 512) return launch_decode_k<MT, GMODE, XLDS, CPW, 4, XB>(d, lds, stream);
                if (d.qwords <= 1024) return launch_decode_k<MT, GMODE, XLDS, CPW, 5, XB>(d, lds, stream);
                return launch_decode_k<MT, GMODE, XLDS, CPW, 6, XB>(d, lds, stream);
            }
        }
    }
    const int64_t lds = decode_lds_layout(d, MT, XLDS, CPW, 0);
    if (lds > kDecodeLdsMax) return hipErrorInvalidValue;
    if constexpr (XB) {
        if (d.has_ortho) return hipErrorInvalidValue;
    } else {
        if (d.has_ortho && d.csr_vec) return launch_decode_k<MT, GMODE, XLDS, CPW, 1, XB>(d, lds, stream);
        if (d.has_ortho) return launch_decode_k<MT, GMODE, XLDS, CPW, 2, XB>(d, lds, stream);
    }
    return launch_decode_k<MT, GMODE, XLDS, CPW, 0, XB>(d, lds, stream);
}

// Chunk-count bounds that can occur: the staged activation block is at most
// 40 KB (so MT * K is bounded) and the global-memory A path takes CPW <= 8.
template <int MT, int GMODE, bool XLDS>
static hipError_t launch_decode_cpw(const DecodeArgs &d, hipStream_t s) {
    constexpr bool c16 = XLDS && MT <= 4;
    constexpr bool c24 = XLDS && MT <= 2;
    if (d.cpw <= 8) return launch_decode_t<MT, GMODE, XLDS, 8>(d, s);
    if (d.cpw <= 16 && c16) return launch_decode_t<MT, GMODE, XLDS, (c16 ? 16 : 8)>(d, s);
    if (c24) return launch_decode_t<MT, GMODE, XLDS, (c24 ? 24 : 8)>(d, s);
    return hipErrorInvalidValue;  // excluded by decode_supported()
}

template <int GMODE, bool XLDS>
static hipError_t launch_decode_mt(int mt, const DecodeArgs &d, hipStream_t s) {
    switch (mt) {
        case 1: return launch_decode_cpw<1, GMODE, XLDS>(d, s);
        case 2: return launch_decode_cpw<2, GMODE, XLDS>(d, s);
        case 4: return launch_decode_cpw<4, GMODE, XLDS>(d, s);
        case 8: return launch_decode_cpw<8, GMODE, XLDS>(d, s);
        default: return launch_decode_cpw<16, GMODE, XLDS>(d, s);
    }
}

// Largest activation block staged in LDS; above it the A operand is read
// straight from global memory (L2-resident), 64 bytes per lane per chunk.
static const int64_t kDecodeXLdsMax = 40 * 1024;
static const int kDecodeMaxCPW = 24;

// Chunks per wave: an even count (group-128 scales come in pairs).
// chunks per wave; the plan's decode records cover the same K quarters
static int decode_cpw(int64_t K) { return decode_chunks_per_wave(K); }

static bool decode_xlds(int64_t M, int64_t K) {
    int64_t mt = 1;
    while (mt < M) mt <<= 1;
    return mt * (K + 8) * 2 <= kDecodeXLdsMax;
}

int plan_qrec_words(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip

bool decode_supported(const ForwardArgs &a) {
    if (a.M < 1 || a.M > 16) return false;
    if (a.io_dtype != ORTH_DT_F16 || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.has_ortho && a.val_dtype != ORTH_DT_F16) return false;
    if (a.K % 128 != 0 || decode_cpw(a.K) > kDecodeMaxCPW || a.N > ((int64_t)1 << 31)) return false;
    // group size 128 * 2^j (the group of a 128-wide chunk is a shift)
    if (a.ngroups != 1 && (a.G % 128 != 0 || ((a.G / 128) & (a.G / 128 - 1)) != 0)) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    // the global-memory A operand keeps 64 bytes per lane per chunk in
    // registers: at most 8 chunks per wave
    if (!decode_xlds(a.M, a.K) && decode_cpw(a.K) > 8) return false;
    return true;
}

int64_t plan_rec_at(int64_t N, int64_t K, int64_t nnz);  // orth_prefill.hip

// The per-layer fields of a decode launch for layer a (with its plan or null).
static DecodeLayerArgs decode_layer_args(const ForwardArgs &a, const void *plan) {
    DecodeLayerArgs e;
    e.q = a.q;
    e.scales = static_cast<const f16 *>(a.scales);
    e.row_ptr = a.row_ptr;
    e.col = a.col;
    e.vals = static_cast<const f16 *>(a.vals);
    e.nnz = (int32_t)a.nnz;
    e.csr_vec = a.nnz >= 4 && ((reinterpret_cast<uintptr_t>(a.col) & 15) == 0) &&
                ((reinterpret_cast<uintptr_t>(a.vals) & 7) == 0);
    e.y = static_cast<f16 *>(a.y);
    e.N = a.N;
    e.alpha = a.alpha;
    const bool rec = plan && a.has_ortho;
    e.rec = rec ? reinterpret_cast<const uint32_t *>(static_cast<const char *>(plan) + plan_rec_at(a.N, a.K, a.nnz))
                : nullptr;
    e.bias = a.bias;
    e.bias_dtype = a.bias_dtype;
    return e;
}

// Everything that selects the kernel instantiation and its shared fields:
// layers of one group launch must agree on all of it.
struct DecodeClass {
    int mt, gmode;
    bool xlds, xb;
    int qwords, has_ortho, csr_vec;
    int64_t M, K, ngroups;
    bool operator==(const DecodeClass &o) const {
        return mt == o.mt && gmode == o.gmode && xlds == o.xlds && xb == o.xb && qwords == o.qwords &&
               has_ortho == o.has_ortho && csr_vec == o.csr_vec && M == o.M && K == o.K && ngroups == o.ngroups;
    }
};

static DecodeClass decode_class(const ForwardArgs &a, const void *plan, DecodeArgs &d) {
    const DecodeLayerArgs e = decode_layer_args(a, plan);
    d.q = e.q;
    d.scales = e.scales;
    d.ngroups = (int)a.ngroups;
    d.row_ptr = e.row_ptr;
    d.col = e.col;
    d.vals = e.vals;
    d.nnz = e.nnz;
    d.csr_vec = e.csr_vec;
    d.x = static_cast<const f16 *>(a.x);
    d.y = e.y;
    d.bias = e.bias;
    d.bias_dtype = e.bias_dtype;
    d.M = (int)a.M;
    d.nchunks = (int)(a.K / 128);
    d.K = (int)a.K;
    d.N = a.N;
    d.cpw = decode_cpw(a.K);
    d.xstride = (int)(a.K + 8);  // +16 bytes: rows start in different LDS banks
    d.alpha = a.alpha;
    d.has_ortho = a.has_ortho;
    d.rec = e.rec;
    d.qwords = e.rec ? plan_qrec_words(a.N, a.K, a.nnz) : 0;
    d.nextra = 0;

    DecodeClass c;
    c.mt = 1;
    while (c.mt < a.M) c.mt <<= 1;
    const bool grouped = a.ngroups != 1;
    d.gshift = 0;
    if (grouped)
        while ((128LL << d.gshift) < a.G) d.gshift++;
    d.scale_pairs = (a.ngroups % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.scales) & 3) == 0);
    c.xlds = decode_xlds(a.M, a.K);
    // 16-byte scale vectors: 8 chunks per vector, each wave's chunks start
    // on a vector boundary
    const bool scale_vec = d.gshift == 0 && a.ngroups % 8 == 0 && d.cpw % 8 == 0 &&
                           (reinterpret_cast<uintptr_t>(a.scales) & 15) == 0;
    // every wave takes exactly the chunk bound (8, 16 or 24 chunks)
    const bool full = d.nchunks == 4 * d.cpw && (d.cpw == 8 || d.cpw == 16 || d.cpw == 24);
    c.gmode = !grouped ? (full ? 4 : 0) : (d.gshift != 0 ? 2 : (scale_vec && full ? 1 : (d.scale_pairs ? 3 : 2)));
    c.xb = a.io_dtype == ORTH_DT_BF16;
    c.qwords = d.qwords;
    c.has_ortho = d.has_ortho;
    c.csr_vec = d.csr_vec;
    c.M = a.M;
    c.K = a.K;
    c.ngroups = a.ngroups;
    return c;
}

// The BF16 instantiations: staged activations and 1..4 tokens with K = 4096
// (group-128 scale vectors or per-row scales), or 1..2 tokens with 17..24
// chunks per wave and paired group-128 scales (K = 11008).
static bool decode_bf16_class_ok(const DecodeClass &c, const DecodeArgs &d) {
    if (!c.xlds || c.mt > 4) return false;
    if (d.cpw == 8) return c.gmode == 1 || c.gmode == 4;
    if (d.cpw > 16 && d.cpw <= 24) return c.gmode == 3 && c.mt <= 2;
    return false;
}

static hipError_t decode_dispatch_bf16(const DecodeClass &c, const DecodeArgs &d, hipStream_t stream) {
    if (!decode_bf16_class_ok(c, d)) return hipErrorInvalidValue;
    if (d.cpw > 8) return c.mt == 1 ? launch_decode_t<1, 3, true, 24, true>(d, stream)
                                     : launch_decode_t<2, 3, true, 24, true>(d, stream);
    if (c.gmode == 1) {
        if (c.mt == 1) return launch_decode_t<1, 1, true, 8, true>(d, stream);
        if (c.mt == 2) return launch_decode_t<2, 1, true, 8, true>(d, stream);
        return launch_decode_t<4, 1, true, 8, true>(d, stream);
    }
    if (c.gmode == 4) {
        if (c.mt == 1) return launch_decode_t<1, 4, true, 8, true>(d, stream);
        if (c.mt == 2) return launch_decode_t<2, 4, true, 8, true>(d, stream);
        return launch_decode_t<4, 4, true, 8, true>(d, stream);
    }
    return hipErrorInvalidValue;
}

static hipError_t decode_dispatch(const DecodeClass &c, const DecodeArgs &d, hipStream_t stream) {
    if (c.xb) return decode_dispatch_bf16(c, d, stream);
    const int mt = c.mt;
    if (c.gmode == 1) return c.xlds ? launch_decode_mt<1, true>(mt, d, stream) : launch_decode_mt<1, false>(mt, d, stream);
    if (c.gmode == 3) return c.xlds ? launch_decode_mt<3, true>(mt, d, stream) : launch_decode_mt<3, false>(mt, d, stream);
    if (c.gmode == 4) return c.xlds ? launch_decode_mt<4, true>(mt, d, stream) : launch_decode_mt<4, false>(mt, d, stream);
    if (c.gmode == 2) return c.xlds ? launch_decode_mt<2, true>(mt, d, stream) : launch_decode_mt<2, false>(mt, d, stream);
    return c.xlds ? launch_decode_mt<0, true>(mt, d, stream) : launch_decode_mt<0, false>(mt, d, stream);
}

// plan: an ortho plan of at least plan_bytes_for(N, K, nnz) bytes, or null;
// cus: the device's compute units.
hipError_t launch_decode(const ForwardArgs &a, const void *plan, int cus, hipStream_t stream) {
    DecodeArgs d;
    const DecodeClass c = decode_class(a, plan, d);
    d.deep = (a.N + 15) / 16 < 2 * (int64_t)cus;
    return decode_dispatch(c, d, stream);
}

// Whether layers as[0 .. n) (each decode_supported, the same activations)
// can share one decode launch: at most kDecodeMaxGroup layers of one
// instantiation class.
bool decode_group_ok(const ForwardArgs *as, const void *const *plans, int n) {
    if (n < 1 || n > kDecodeMaxGroup) return false;
    DecodeArgs d;
    const DecodeClass c0 = decode_class(as[0], plans ? plans[0] : nullptr, d);
    for (int l = 1; l < n; l++) {
        if (as[l].x != as[0].x) return false;
        DecodeArgs dl;
        if (!(decode_class(as[l], plans ? plans[l] : nullptr, dl) == c0)) return false;
    }
    int64_t blocks = 0;
    for (int l = 0; l < n; l++) blocks += (as[l].N + 15) / 16;
    return blocks <= INT32_MAX;
}

// One decode launch for the layers as[0 .. n) (decode_group_ok): workgroups
// are dealt to the layers in order, each layer's blocks contiguous.
hipError_t launch_decode_group(const ForwardArgs *as, const void *const *plans, int n, int cus, hipStream_t stream) {
    DecodeArgs d;
    const DecodeClass c = decode_class(as[0], plans ? plans[0] : nullptr, d);
    d.nextra = n - 1;
    int64_t blk = 0;
    for (int l = 0; l < n; l++) {
        d.blk0[l] = (int)blk;
        blk += (as[l].N + 15) / 16;
        if (l > 0) d.extra[l - 1] = decode_layer_args(as[l], plans ? plans[l] : nullptr);
    }
    for (int l = n; l <= kDecodeMaxGroup; l++) d.blk0[l] = (int)blk;
    d.deep = blk < 2 * (int64_t)cus;
    return decode_dispatch(c, d, stream);
}

// BF16 activations (this plan or none): a shape class with a BF16
// instantiation (decode_bf16_class_ok), and the ortho term (if on) from
// plan records that the LDS takes beside the staged activations.
bool decode_bf16_supported(const ForwardArgs &a, const void *plan) {
    if (a.io_dtype != ORTH_DT_BF16 || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.M < 1 || a.M > 4 || a.K % 128 != 0 || decode_cpw(a.K) > kDecodeMaxCPW || a.N > ((int64_t)1 << 31))
        return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    if (a.ngroups != 1 && a.G != 128) return false;
    if (a.has_ortho && a.val_dtype != ORTH_DT_F16) return false;
    DecodeArgs d;
    const DecodeClass c = decode_class(a, a.has_ortho ? plan : nullptr, d);
    if (!decode_bf16_class_ok(c, d)) return false;
    if (a.has_ortho) {
        if (d.qwords <= 0 || d.qwords > 2048) return false;  // (no plan: no records)
        const int cpw_bound = d.cpw <= 8 ? 8 : 24;
        if (decode_lds_layout(d, c.mt, true, cpw_bound, kDecodeW * d.qwords) > kDecodeLdsMax) return false;
    }
    return true;
}

}  // namespace orth
