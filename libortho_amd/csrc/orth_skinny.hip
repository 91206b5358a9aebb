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
//    v_mfma_f32_16x16x32_f16 as the B operand; the activations of each
//    16-token tile are the A operand, read from LDS (interleaved k order).
//    The bias is removed per chunk with the activation sums computed while
//    staging; group scales multiply each chunk's FP32 partial.
//  * The sparse ortho term of the slice comes from the ortho plan: its
//    (128-row block, 64-column step) buckets are sorted by row.  The slice's
//    entries are staged in LDS, counted per (bucket, row) with LDS atomics
//    and turned into row starts by a DPP prefix sum per bucket; four threads
//    per row then multiply the row's entries with the staged activations,
//    first the leading entry of every bucket (LDS reads issued in batches),
//    then the rest.  Sums are formed in a fixed order: the result does not
//    depend on scheduling.
//  * When the row blocks alone cannot fill the GPU, K is split over S
//    workgroups.  Each writes its FP32 partial (ortho term included) to a
//    workspace and a second kernel adds the S partials in slice order and
//    writes y.  (The kernel boundary makes the partials visible across the
//    XCDs; an in-kernel hand-off would need device-scope fences, which on
//    this part write back and invalidate the L2 of every XCD.)
#include <algorithm>

#include "orth_common.h"

namespace orth {

constexpr int kSkNT = 512;            // 8 waves
constexpr int kSkRows = 128;          // rows per workgroup (= ortho plan block)
constexpr int kSkMaxCPS = 8;          // chunks per slice (compile-time bound)
constexpr int kSkESlots = 8;          // plan entries per thread loaded at entry
constexpr int kSkEStaged = kSkESlots * 512;  // plan entries staged in LDS per workgroup
constexpr int kSkPlanBK = 64;         // plan column step
constexpr uint32_t kSkPlanMagic = 0x504f5254u;

// Chunks per slice the kernel of ntt token tiles is built for: even (group
// scales are read in pairs) and with at most 8 activation pieces per thread.
constexpr int sk_cps_bound(int ntt) { return ntt * kSkMaxCPS > 16 ? ((16 / ntt) & ~1) : kSkMaxCPS; }

struct SkinnyArgs {
    const uint8_t *q;
    const f16 *scales;
    int ngroups;
    int gshift;          // group of chunk c is c >> gshift (G = 128 << gshift)
    const int32_t *poffs;     // plan offsets [nblocks][nsteps + 1]
    const uint32_t *pents;    // plan entries
    const uint32_t *phdr;     // plan header: magic, version, bn, bk, nblocks, nsteps, n, k, nnz
    int32_t nnz;
    const f16 *x;
    f16 *y;
    int M;
    int K;
    int64_t N;
    int nchunks;         // K / 128
    int nsteps;          // K / 64
    int cps;             // chunks per slice (even)
    int S;               // slices
    int nblocks;         // 128-row blocks
    int xstride;         // LDS row stride of the staged activations, in halves
    int lds_cr, lds_xs, lds_sp, lds_e, lds_idx;  // byte offsets of the LDS regions
    float alpha;
    float *part;         // [S][M][N] partials (S > 1)
};

// v[i] for wave-uniform v and a runtime i in [0, L): a chain of selects, so
// that v stays in registers (a runtime subscript moves the array to per-lane
// scratch memory, which is written back through the L2 to HBM).  The
// readfirstlane keeps the compiler from folding the chain back into a
// subscripted load.
template <int L>
__device__ __forceinline__ int32_t pick(const int32_t (&v)[L], int i) {
    int32_t r = __builtin_amdgcn_readfirstlane(v[0]);
#pragma unroll
    for (int k = 1; k < L; k++) r = i == k ? __builtin_amdgcn_readfirstlane(v[k]) : r;
    return r;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves: shifts
// by 1, 2, 4, 8 within each row of 16 lanes, then row 0's total into row 1
// and row 2's into row 3 (row_bcast:15), then the total of rows 0-1 into
// rows 2-3 (row_bcast:31).  Lanes without a source take 0.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// GMODE: 0 per-row scale (G == K); 1 G = 128, scales read as aligned pairs;
// 2 any G = 128 * 2^j.  NTT: 16-token tiles.  CPS: chunk bound per slice.
template <int NTT, int GMODE, int CPS, bool SPARSE>
__global__ void __launch_bounds__(kSkNT) skinny_kernel(SkinnyArgs a) {
    constexpr int MP = NTT * 16;                     // padded tokens
    constexpr int XP = (MP * CPS * 16 + kSkNT - 1) / kSkNT;  // 16-byte pieces per thread
    constexpr int SW = (CPS + 7) / 8;
    constexpr bool GROUPED = GMODE != 0;

    extern __shared__ __align__(16) unsigned char smem[];
    float *cr = reinterpret_cast<float *>(smem + a.lds_cr);     // [cps][MP] bias sums
    f16 *xs = reinterpret_cast<f16 *>(smem + a.lds_xs);         // [MP][xstride] activations
    float *sp = reinterpret_cast<float *>(smem + a.lds_sp);     // [128][MP] sparse sums
    uint32_t *es = reinterpret_cast<uint32_t *>(smem + a.lds_e);  // staged plan entries
    int32_t *ridx = reinterpret_cast<int32_t *>(smem + a.lds_idx);  // [2 cps][129] row starts per bucket

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

    // ---- plan words, one vector load per wave issued after the activations
    //      and before the weights (loads complete in order: the staging does
    //      not wait for it, and it does not wait for the weights): lanes
    //      0 .. 2 CPS read the slice's bucket offsets, lanes 32 .. 43 the plan
    //      header words 0 .. 11
    int32_t pword = 0;
    if (SPARSE) {
        const int64_t ob = (int64_t)blk * (a.nsteps + 1);
        const int32_t *src = lane < 32 ? a.poffs + (ob + min(2 * kc0 + min(lane, 2 * nci), a.nsteps))
                                       : reinterpret_cast<const int32_t *>(a.phdr) + min(lane - 32, 11);
        pword = *src;
    }

    // ---- scales
    const f16 *sbase = a.scales + my_n * (int64_t)a.ngroups;
    uint32_t sw[SW];
    f16 sh[GMODE == 2 ? CPS : 1];
    float srow = 0.f;  // GMODE 0: the scale of row 16 w + nl (tid & 15 == nl)
    if (GMODE == 0) srow = (float)a.scales[min(wrow0 + (tid & 15), a.N - 1)];
    if (GMODE == 1) {
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
#pragma unroll
    for (int p = 0; p < CPS; p++)
        wv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + min(kc0 + p, clast) * 64));

    // ---- stage the activations (interleaved k order) and their bias sums
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + kSkNT * i;
        const int m = p / (CPS * 16), c = (p / 16) % CPS;
        u32x4 v = xreg[i];
        if (m >= a.M) v = u32x4{0, 0, 0, 0};
        const f16x8 h = __builtin_bit_cast(f16x8, v);
        // even k weigh 1032, odd k weigh 72 (see int4x8_to_f16_biased)
        const float e = ((float)h[0] + (float)h[2]) + ((float)h[4] + (float)h[6]);
        const float o = ((float)h[1] + (float)h[3]) + ((float)h[5] + (float)h[7]);
        const float b = group_sum<16>(1032.0f * e + 72.0f * o);  // the 16 pieces of (m, c)
        if (m < MP && c < a.cps) {  // the LDS tile holds the host's cps chunks
            *reinterpret_cast<u32x4 *>(xs + (m * a.xstride + c * 128 + (p & 15) * 8)) = permute_x8(v);
            if ((p & 15) == 0) cr[c * MP + m] = b;
        }
    }
    if (SPARSE)
        for (int i = tid; i < 2 * CPS * 129; i += kSkNT) ridx[i] = 0;
    __syncthreads();

    // ---- bucket offsets of the slice (uniform), checked against the header.
    //      Read after the staging and its barrier (kept there by the
    //      scheduling barrier): the offsets miss the caches more often than
    //      the activations, and neither need wait for them.
    __builtin_amdgcn_sched_barrier(0);
    int32_t soff[2 * CPS + 1];
    int32_t e_lo = 0, e_hi = 0;
    if (SPARSE) {
        auto word = [&](int l) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane(pword, l); };
        auto dword = [&](int l) -> int64_t { return (int64_t)(word(l) | ((uint64_t)word(l + 1) << 32)); };
        const bool plan_ok = (word(32) == kSkPlanMagic) & (word(33) == 1u) & (dword(38) == a.N) &
                             (dword(40) == (int64_t)K) & (dword(42) == (int64_t)a.nnz);
#pragma unroll
        for (int i = 0; i <= 2 * CPS; i++) soff[i] = min(max(__builtin_amdgcn_readlane(pword, i), 0), a.nnz);
        e_lo = soff[0];
        e_hi = plan_ok ? max(min(max(__builtin_amdgcn_readlane(pword, 2 * nci), 0), a.nnz), e_lo) : e_lo;
        // monotone within [e_lo, e_hi] whatever the plan holds
#pragma unroll
        for (int i = 0; i <= 2 * CPS; i++) soff[i] = min(max(soff[i], i ? soff[i - 1] : e_lo), e_hi);
    }

    // ---- the slice's plan entries (up to kSkEStaged; more are read from
    //      memory in the sparse pass).  Addresses past the slice repeat its
    //      last entry: no bytes beyond the slice's own are fetched.
    uint32_t ereg[SPARSE ? kSkESlots : 1];
    if (SPARSE) {
        const int32_t elast = min(max(e_hi - 1, e_lo), max(a.nnz - 1, 0));
#pragma unroll
        for (int i = 0; i < kSkESlots; i++) ereg[i] = a.pents[min(e_lo + tid + kSkNT * i, elast)];
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
#pragma unroll
    for (int p = 0; p < CPS; p++) {
        if (p < nci) {  // uniform
            const uint32_t words[4] = {wv[p].x, wv[p].y, wv[p].z, wv[p].w};
            uint32_t bq[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) int4x8_to_f16_biased(words[j], bq[j]);
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
                    const f16x8 bfr = __builtin_bit_cast(f16x8, u32x4{bq[j][0], bq[j][1], bq[j][2], bq[j][3]});
                    part = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr, bfr, part, 0, 0, 0);
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

    // ---- sparse term of the slice.  The slice's buckets are sorted by row,
    //      so a count per (bucket, row) and a prefix sum per bucket give each
    //      row's entries; thread (row r, token group tg) then multiplies
    //      them, in entry order, with the staged activations.
    constexpr int MQ = MP / 4;  // tokens per thread: tg, tg + 4, ...
    if (SPARSE) {
        constexpr int NB = 2 * CPS;  // buckets (64-column steps) of a slice
        const int32_t staged_hi = e_lo + min(e_hi - e_lo, kSkEStaged);
        const uint32_t *pents = a.pents;
        // Entries below staged_hi are read from LDS, the rest (slices of more
        // than kSkEStaged entries) from memory, in loops of their own: one
        // accessor for both would become a flat load, which waits for memory
        // latency on every entry.
        // counts: entry i of bucket b (soff[b] <= i < soff[b+1]) adds 1 to
        // (b, row + 1); the staged entries are counted from registers
        auto count = [&](int32_t i, uint32_t e) {
            int b = 0;
#pragma unroll
            for (int k = 1; k < NB; k++) b += i >= soff[k] ? 1 : 0;
            atomicAdd(&ridx[b * 129 + 1 + (int)((e >> 24) & 0x7f)], 1);
        };
#pragma unroll
        for (int i = 0; i < kSkESlots; i++) {
            es[tid + kSkNT * i] = ereg[i];
            const int32_t idx = e_lo + tid + kSkNT * i;
            if (idx < staged_hi) count(idx, ereg[i]);
        }
        for (int32_t i = staged_hi + tid; i < e_hi; i += kSkNT) count(i, pents[i]);
        __syncthreads();
        // prefix sums: ridx[b][r] = first entry of row r in bucket b
        for (int b = wave; b < NB; b += kSkNT / 64) {
            int32_t *t = ridx + b * 129;
            const int v0 = t[1 + 2 * lane], v1 = t[2 + 2 * lane];
            const int incl = wave_inclusive_sum(v0 + v1);
            const int32_t sb = pick(soff, b);
            const int base = sb + incl - v0 - v1;       // before row 2 lane
            t[1 + 2 * lane] = base + v0;                // start of row 2 lane + 1
            t[2 + 2 * lane] = base + v0 + v1;           // start of row 2 lane + 2
            if (lane == 0) t[0] = sb;
        }
        __syncthreads();
        const int r = tid >> 2, tg = tid & 3;
        float sacc[MQ];
#pragma unroll
        for (int i = 0; i < MQ; i++) sacc[i] = 0.f;
        const int xstride = a.xstride;
        auto fma_entry = [&](int cbase, uint32_t e) {
            const int cl = cbase + (int)((e >> 16) & 0x3f);  // column within the slice
            const float v = (float)__builtin_bit_cast(f16, (uint16_t)(e & 0xffffu));
            const int xi = (cl & ~7) | interleaved_pos(cl & 7);
#pragma unroll
            for (int i2 = 0; i2 < MQ; i2++) sacc[i2] += v * (float)xs[(tg + 4 * i2) * xstride + xi];
        };
        // First pass: the first entry of every bucket of row r, GB buckets at
        // a time, so that each round of LDS reads (bounds, entries,
        // activations) is issued together.  An absent entry reads as value 0
        // at column 0 of the slice (a column of a bucket past the host's
        // chunk count would lie outside the staged activations).
        constexpr int GB = (32 / MQ) < 2 ? 2 : (32 / MQ) > NB ? NB : (32 / MQ);
        uint32_t more = 0;  // bit st: bucket st has entries the first pass did not take
#pragma unroll
        for (int s0 = 0; s0 < NB; s0 += GB) {
            int32_t lo[GB], hi[GB];
#pragma unroll
            for (int u = 0; u < GB; u++) {
                const int st = min(s0 + u, NB - 1);
                lo[u] = max(ridx[st * 129 + r], e_lo);
                hi[u] = min(ridx[st * 129 + r + 1], e_hi);
            }
            uint32_t ev[GB];
            int cb[GB];
#pragma unroll
            for (int u = 0; u < GB; u++) {
                const bool ok = s0 + u < NB && lo[u] < hi[u] && lo[u] < staged_hi;
                ev[u] = ok ? es[min(lo[u] - e_lo, kSkEStaged - 1)] : 0u;
                cb[u] = ok ? (s0 + u) * kSkPlanBK : 0;
                if (s0 + u < NB && hi[u] - lo[u] > (ok ? 1 : 0)) more |= 1u << (s0 + u);
            }
#pragma unroll
            for (int u = 0; u < GB; u++) fma_entry(cb[u], ev[u]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Second pass: the remaining entries, bucket by bucket
        while (more) {
            const int st = __builtin_ctz(more);
            more &= more - 1;
            const int32_t lo = max(ridx[st * 129 + r], e_lo), hi = min(ridx[st * 129 + r + 1], e_hi);
            const int32_t hs = min(hi, staged_hi);
            for (int32_t i = lo + 1; i < hs; i++) fma_entry(st * kSkPlanBK, es[i - e_lo]);
            // past the staged block (the first entry too, when it lay there)
            for (int32_t i = max(lo, staged_hi); i < hi; i++) fma_entry(st * kSkPlanBK, pents[i]);
        }
#pragma unroll
        for (int i2 = 0; i2 < MQ; i2++) sp[r * MP + tg + 4 * i2] = sacc[i2];
    }
    __syncthreads();

    // ---- this slice's values: lane (row nl, tokens tt*16 + 4g + i)
    float val[NTT][4];
    const int64_t n = wrow0 + nl;
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = acc[tt][i];
            if (!GROUPED) v = (v - bias_acc[tt][i]) * srow;
            if (SPARSE) v += a.alpha * sp[(wave * 16 + nl) * MP + tt * 16 + 4 * g + i];
            val[tt][i] = v;
        }
    }
    if (a.S == 1) {
#pragma unroll
        for (int tt = 0; tt < NTT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = tt * 16 + 4 * g + i;
                if (m < a.M && n < a.N) a.y[(int64_t)m * a.N + n] = (f16)val[tt][i];
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
__global__ void __launch_bounds__(256) skinny_reduce_kernel(const float *part, f16 *y, int M, int64_t N, int S,
                                                            int vec4) {
    // workgroup blk (on XCD blk % 8, like the slices of row block blk) adds
    // the S partials of rows [128 blk, 128 blk + 128) for every token.  The
    // loads of a group of 8 slices are issued before the first add (addresses
    // clamped to the last slice, the extra ones not added); sums in slice order.
    constexpr int U = 8;
    const int64_t n0 = (int64_t)blockIdx.x * kSkRows;
    const int64_t MN = (int64_t)M * N;
    if (vec4) {
        for (int idx = threadIdx.x; idx < M * (kSkRows / 4); idx += 256) {
            const int m = idx / (kSkRows / 4);
            const int64_t n = n0 + 4 * (idx - m * (kSkRows / 4));
            if (n >= N) continue;
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
            const f16x2 lo = {(f16)v[0], (f16)v[1]}, hi = {(f16)v[2], (f16)v[3]};
            *reinterpret_cast<uint2 *>(y + o) = uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
    } else {
        for (int idx = threadIdx.x; idx < M * kSkRows; idx += 256) {
            const int m = idx / kSkRows;
            const int64_t n = n0 + (idx - m * kSkRows);
            if (n >= N) continue;
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
            y[o] = (f16)v;
        }
    }
}

// ------------------------------------------------------------------ host

struct SkinnyShape {
    int ntt, cps, S, nblocks, xstride;
    int lds_cr, lds_xs, lds_sp, lds_e, lds_idx, lds_bytes;
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
    off += kSkRows * mp * 4;
    sh.lds_e = off;
    off += a.has_ortho ? kSkEStaged * 4 : 0;
    sh.lds_idx = off;
    off += a.has_ortho ? ((2 * cps_max * 129 * 4 + 15) & ~15) : 0;  // the kernel's 2 CPS buckets
    sh.lds_bytes = off;
    return off <= 150 * 1024;
}

bool skinny_supported(const ForwardArgs &a) {
    if (a.M < 1 || a.M > 64) return false;
    if (a.io_dtype != ORTH_DT_F16 || a.scale_dtype != ORTH_DT_F16) return false;
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

template <int NTT, int GMODE, int CPS, bool SPARSE>
static hipError_t skinny_launch_t(const SkinnyArgs &d, int blocks, int lds, hipStream_t s) {
    // more than 64 KB of dynamic LDS must be allowed once per device
    static int allowed[64] = {0};
    int dev = 0;
    if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !allowed[dev]) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(skinny_kernel<NTT, GMODE, CPS, SPARSE>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        if (e != hipSuccess) return e;
        allowed[dev] = 1;
    }
    hipLaunchKernelGGL((skinny_kernel<NTT, GMODE, CPS, SPARSE>), dim3(blocks), dim3(kSkNT), (uint32_t)lds, s, d);
    return hipGetLastError();
}

template <int NTT, int GMODE>
static hipError_t skinny_launch_g(const SkinnyArgs &d, bool sparse, int blocks, int lds, hipStream_t s) {
    constexpr int C = sk_cps_bound(NTT);
    if (d.cps > C) return hipErrorInvalidValue;  // the kernel handles at most C chunks per slice
    if (sparse) return skinny_launch_t<NTT, GMODE, C, true>(d, blocks, lds, s);
    return skinny_launch_t<NTT, GMODE, C, false>(d, blocks, lds, s);
}

template <int NTT>
static hipError_t skinny_launch_n(const SkinnyArgs &d, int gmode, bool sparse, int blocks, int lds, hipStream_t s) {
    switch (gmode) {
        case 0: return skinny_launch_g<NTT, 0>(d, sparse, blocks, lds, s);
        case 1: return skinny_launch_g<NTT, 1>(d, sparse, blocks, lds, s);
        default: return skinny_launch_g<NTT, 2>(d, sparse, blocks, lds, s);
    }
}

// Workspace bytes of a call (0 when K is not split).
int64_t skinny_workspace_bytes(const ForwardArgs &a, int cus) {
    SkinnyShape sh;
    skinny_shape(a, cus, sh);
    return sh.S > 1 ? (int64_t)sh.S * a.M * a.N * 4 : 0;
}

// plan: the ortho plan (required when has_ortho); part: the workspace.
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
    const bool sparse = a.has_ortho && plan != nullptr;
    if (a.has_ortho && !plan) return hipErrorInvalidValue;
    d.nsteps = (int)(a.K / kSkPlanBK);
    if (sparse) {
        const int64_t nb = sh.nblocks;
        d.phdr = static_cast<const uint32_t *>(plan);
        d.poffs = reinterpret_cast<const int32_t *>(static_cast<const char *>(plan) + 64);
        const int64_t ob = ((nb * (d.nsteps + 1) * 4) + 15) & ~int64_t(15);
        d.pents = reinterpret_cast<const uint32_t *>(static_cast<const char *>(plan) + 64 + ob);
    } else {
        d.phdr = nullptr;
        d.poffs = nullptr;
        d.pents = nullptr;
    }
    d.nnz = (int32_t)a.nnz;
    d.x = static_cast<const f16 *>(a.x);
    d.y = static_cast<f16 *>(a.y);
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
    d.lds_e = sh.lds_e;
    d.lds_idx = sh.lds_idx;
    d.alpha = a.alpha;
    d.part = part;
    // pairs of group-128 scales are read as aligned 32-bit words when every
    // row starts on a pair (even group count, 4-byte aligned scales)
    const bool pairs = (a.ngroups & 1) == 0 && (reinterpret_cast<uintptr_t>(a.scales) & 3) == 0;
    const int gmode = a.ngroups == 1 ? 0 : (d.gshift == 0 && pairs ? 1 : 2);
    const int blocks = ((sh.nblocks + 7) / 8) * 8 * sh.S;  // padded: see skinny_kernel
    hipError_t e;
    switch (sh.ntt) {
        case 1: e = skinny_launch_n<1>(d, gmode, sparse, blocks, sh.lds_bytes, stream); break;
        case 2: e = skinny_launch_n<2>(d, gmode, sparse, blocks, sh.lds_bytes, stream); break;
        case 3: e = skinny_launch_n<3>(d, gmode, sparse, blocks, sh.lds_bytes, stream); break;
        default: e = skinny_launch_n<4>(d, gmode, sparse, blocks, sh.lds_bytes, stream); break;
    }
    if (e != hipSuccess || sh.S == 1) return e;
    const int vec4 = (a.N % 4 == 0) ? 1 : 0;
    hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)sh.nblocks), dim3(256), 0, stream, part,
                       static_cast<f16 *>(a.y), (int)a.M, a.N, sh.S, vec4);
    return hipGetLastError();
}

}  // namespace orth
