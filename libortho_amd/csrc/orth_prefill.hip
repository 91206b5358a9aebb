// Prefill dual GEMM for gfx950 (batches above 64 tokens, and 17..64 where
// the mid-batch kernels do not apply), and the ortho plan builder.
//
// Design intent of /root/reference/src/dual_gemm_tensor_core.cu:215-337
// (matrix-core base GEMM with the ortho term fused), built for CDNA4:
//
//  * Workgroup tile 256 tokens x 128 output rows, 8 waves in a 4x2 grid,
//    each wave 64x64 with v_mfma_f32_32x32x16_f16 (FP32 accumulation).
//    K advances in steps of 64 through LDS: activations in 2 stages,
//    dequantised weights in 3.
//  * The activation tile is copied to LDS as is.  The INT4 weight tile is
//    dequantised on the way in: each thread turns one 16-byte load (32
//    nibbles of one row) into 32 FP16 weights q*s (one rounding of the exact
//    product) and writes them to LDS.
//  * The sparse ortho term is folded into that LDS weight tile before the
//    MFMAs read it: the plan (a derived layout of the CSR, built once at load
//    time) lists, per (128-row block, 64-column step), the entries that fall
//    inside the tile, so each entry costs one LDS read-modify-write per 256
//    tokens instead of a gather per token.  alpha <= 0 skips the fold on a
//    uniform branch and never reads the plan.
//  * The weight operand therefore is fp16(fp16(q*s) + alpha*v): within
//    2^-11 relative of the exact weight, far inside the 1e-2*|y|_inf bound.
//    (The decode kernel keeps q exact and scales FP32 partial sums; the
//    dequant entry point gives the bit-exact FP32 weights.)
//  * Tiles are mapped XCD-aware: consecutive workgroup ids land on different
//    XCDs, so the tile order is remapped to give each XCD a contiguous run.
//  * Where the tiles alone leave CUs idle (fewer tokens than the grid needs),
//    K is split over the grid: each tile's workgroups take slices of the
//    64-column steps and write FP32 partials, which split_reduce_kernel
//    (orth_split.hip) adds in slice order (prefill_ksplit).
#include <type_traits>

#include "orth_common.h"

namespace orth {

// ----------------------------------------------------------------- plan
//
// Layout (all little-endian):
//   PlanHeader (64 bytes)
//   int32 offsets[nblocks][nksteps + 1]   absolute entry index per (block, step)
//   uint32 entries[nnz]                   (row_in_block << 24) | (col_in_step << 16) | fp16 bits
//   uint16 chunks[N][K/128 + 1]           (K % 128 == 0 only) per row, the number of
//                                         its CSR entries with column < 128 c
//   uint32 qrecs[ceil(N/16)][4][Wq]      per 16-row group and decode K quarter (the
//                                         columns of decode wave w), the rows' entries
//                                         packed (cell records, see orth_common.h);
//                                         Wq = 256 .. 2048 words, in pad[0]
//   uint32 srecs[ceil(N/16)][ceil(K/1024)][W]  (K % 128 == 0) the same per 1024-column
//                                         slice (the last one may be narrower) for the
//                                         mid-batch kernels; W = 256 or 512 words, in
//                                         pad[1] (0: none)
// Entries of one (block, step) are ordered by row then by CSR position.  The
// chunk table locates a row's entries of columns [128 c0, 128 c1) in the CSR
// itself when the row's columns ascend strictly (flag kPlanUnsorted clear).
// The cell records give the decode and mid-batch kernels each wave's
// entries at an address known before any load returns (a CSR range's start
// is itself a load); a cell whose entries do not fit is read from the CSR.

static const uint32_t kPlanMagic = 0x504f5254u;  // "TROP"
static const uint32_t kPlanVersion = 5;
static const int kPlanBN = 128;
static const int kPlanBK = 64;
static const uint32_t kPlanNonCanonical = 1u;  // duplicate or unsorted columns in a row
static const uint32_t kPlanMalformed = 2u;     // row_ptr not monotone within [0, nnz]
static const uint32_t kPlanUnsorted = 4u;      // some row's columns (any value) do not ascend strictly

struct PlanHeader {
    uint32_t magic, version;
    int32_t bn, bk, nblocks, nksteps;
    int64_t n, k, nnz;
    uint32_t flags;
    uint32_t pad[3];
};
static_assert(sizeof(PlanHeader) == 64, "plan header must be 64 bytes");

int64_t plan_offsets_bytes(int64_t N, int64_t K) {
    const int64_t nblocks = (N + kPlanBN - 1) / kPlanBN;
    const int64_t nk = K / kPlanBK;
    return ((nblocks * (nk + 1) * 4) + 15) & ~int64_t(15);
}

// Byte offset of the chunk table (16-byte aligned, after the entries) and
// its size; K % 128 != 0 has none.
int64_t plan_chunks_at(int64_t N, int64_t K, int64_t nnz) {
    return (((int64_t)sizeof(PlanHeader) + plan_offsets_bytes(N, K) + 4 * nnz) + 15) & ~int64_t(15);
}

int64_t plan_chunks_bytes(int64_t N, int64_t K) {
    return K % 128 == 0 ? ((N * (K / 128 + 1) * 2) + 15) & ~int64_t(15) : 0;
}

// Words of a cell record of `cols` columns: the header plus the mean entry
// count of a 16-row cell plus four times (its square root + 1), in 256-word
// units; 0 (no records) past max_words.
static int cell_words(int64_t N, int64_t K, int64_t nnz, int64_t cols, int max_words) {
    if (nnz <= 0 || N <= 0 || K <= 0) return 0;
    const int64_t mean = (16 * cols * nnz + N * K - 1) / (N * K);
    int64_t s = 0;
    while ((s + 1) * (s + 1) <= mean) s++;
    const int64_t need = kCellHdrWords + mean + 4 * (s + 1);
    const int64_t w = (need + 255) / 256 * 256;
    return w <= max_words ? (int)w : 0;
}

// decode K quarters (K % 128 == 0): a multiple of 256 words, at most 2048
int plan_qrec_words(int64_t N, int64_t K, int64_t nnz) {
    if (K % 128 != 0) return 0;
    return cell_words(N, K, nnz, (int64_t)decode_chunks_per_wave(K) * 128, 2048);
}

// mid-batch slices of 1024 columns (K % 128 == 0; the last slice holds the
// rest of K): 256 or 512 words
int plan_srec_words(int64_t N, int64_t K, int64_t nnz) {
    if (K % 128 != 0) return 0;
    return cell_words(N, K, nnz, 1024, 512);
}

int64_t plan_rec_at(int64_t N, int64_t K, int64_t nnz) {
    return plan_chunks_at(N, K, nnz) + plan_chunks_bytes(N, K);
}

int64_t plan_srec_at(int64_t N, int64_t K, int64_t nnz) {
    return plan_rec_at(N, K, nnz) + ((N + 15) / 16) * 4 * (int64_t)plan_qrec_words(N, K, nnz) * 4;
}

int64_t plan_bytes_for(int64_t N, int64_t K, int64_t nnz) {
    if (nnz <= 0) return 0;
    return plan_srec_at(N, K, nnz) + ((N + 15) / 16) * ((K + 1023) / 1024) * (int64_t)plan_srec_words(N, K, nnz) * 4;
}

// Largest K the plan builder's LDS counters take (int32 per (step, row)).
static const int64_t kPlanMaxK = 12288;

bool plan_supported(const ForwardArgs &a) {
    return a.K % kPlanBK == 0 && a.K <= kPlanMaxK && a.nnz < ((int64_t)1 << 31);
}

__global__ void plan_init_kernel(PlanHeader *h, int nblocks, int nksteps, int64_t N, int64_t K,
                                 int64_t nnz, int qwords, int swords) {
    if (threadIdx.x == 0) {
        h->magic = kPlanMagic;
        h->version = kPlanVersion;
        h->bn = kPlanBN;
        h->bk = kPlanBK;
        h->nblocks = nblocks;
        h->nksteps = nksteps;
        h->n = N;
        h->k = K;
        h->nnz = nnz;
        h->flags = 0;
        h->pad[0] = (uint32_t)qwords;
        h->pad[1] = (uint32_t)swords;
        h->pad[2] = 0;
    }
}

__device__ __forceinline__ uint32_t value_bits_f16(const void *vals, int dtype, int64_t j) {
    if (dtype == ORTH_DT_F16) return ((const uint16_t *)vals)[j];
    const float v = load_as_f32(vals, dtype, j);
    return __builtin_bit_cast(uint16_t, (f16)v);
}

// One workgroup per block of kPlanBN output rows.  Counting sort of the
// block's CSR entries by 64-column step, stable in (row, CSR position).
__global__ void __launch_bounds__(256) plan_build_kernel(ForwardArgs a, PlanHeader *h,
                                                         int32_t *offsets, uint32_t *entries,
                                                         uint16_t *chunks, int nksteps) {
    extern __shared__ __align__(16) int32_t cnt[];  // [nksteps][BN], then partials[256]
    int32_t *partials = cnt + nksteps * kPlanBN;
    __shared__ int32_t s_flags;
    __shared__ int32_t s_total;
    const int tid = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int L = nksteps * kPlanBN;
    for (int i = tid; i < L; i += 256) cnt[i] = 0;
    if (tid == 0) s_flags = 0;
    __syncthreads();

    const int r = tid;
    const int64_t n = b * kPlanBN + r;
    int32_t rs = 0, re = 0;
    uint32_t myflags = 0;
    if (r < kPlanBN && n < a.N) {
        const int64_t ra = a.row_ptr[n], rb = a.row_ptr[n + 1];
        if (ra < 0 || rb < ra || rb > a.nnz) myflags |= kPlanMalformed;
        csr_row_range(a.row_ptr, n, a.nnz, rs, re);
        int32_t prev = -1, praw = INT32_MIN;
        const int nch = chunks ? (int)(a.K / 128) : 0;
        uint16_t *crow = chunks ? chunks + n * (int64_t)(nch + 1) : nullptr;
        int cnext = 0;  // next chunk boundary to record
        for (int32_t j = rs; j < re; j++) {
            const int32_t c = a.col[j];
            if (c <= praw) myflags |= kPlanUnsorted;
            praw = c;
            // boundaries 128 cb <= c end before entry j (meaningful when sorted)
            if (crow)
                for (; cnext <= nch && (int64_t)cnext * 128 <= (int64_t)c; cnext++)
                    crow[cnext] = (uint16_t)min(j - rs, 65535);
            if (c >= 0 && c < a.K) {
                cnt[(c / kPlanBK) * kPlanBN + r] += 1;
                if (c <= prev) myflags |= kPlanNonCanonical;
                prev = c;
            }
        }
        if (crow)
            for (; cnext <= nch; cnext++) crow[cnext] = (uint16_t)min(re - rs, 65535);
        if (re - rs > 65535) myflags |= kPlanUnsorted;  // counts past 16 bits
    }
    if (myflags) atomicOr(&s_flags, (int32_t)myflags);
    __syncthreads();

    // exclusive scan of cnt in (step, row) order: per-thread segments
    const int seg = (L + 255) / 256;
    const int lo = tid * seg, hi = min(L, lo + seg);
    int32_t local = 0;
    for (int i = lo; i < hi; i++) local += cnt[i];
    partials[tid] = local;
    __syncthreads();
    if (tid == 0) {
        int32_t run = 0;
        for (int i = 0; i < 256; i++) {
            const int32_t v = partials[i];
            partials[i] = run;
            run += v;
        }
        s_total = run;
    }
    __syncthreads();
    int32_t run = partials[tid];
    for (int i = lo; i < hi; i++) {
        const int32_t v = cnt[i];
        cnt[i] = run;
        run += v;
    }
    __syncthreads();

    // the block's entries occupy [base, base + total) of the CSR index space
    const int64_t nfirst = b * kPlanBN;
    const int64_t nlast = min((int64_t)a.N, nfirst + kPlanBN);
    int64_t base = a.row_ptr[nfirst], end = a.row_ptr[nlast];
    base = base < 0 ? 0 : (base > a.nnz ? a.nnz : base);
    end = end < base ? base : (end > a.nnz ? a.nnz : end);
    const int64_t total = s_total;
    const bool fits = base + total <= end;
    int32_t *off = offsets + b * (nksteps + 1);
    for (int kt = tid; kt <= nksteps; kt += 256) {
        int64_t o = kt < nksteps ? cnt[kt * kPlanBN] : total;
        off[kt] = (int32_t)(base + (fits ? o : 0));
    }
    __syncthreads();  // the placement below advances the same counters
    if (fits && r < kPlanBN && n < a.N) {
        for (int32_t j = rs; j < re; j++) {
            const int32_t c = a.col[j];
            if (c >= 0 && c < a.K) {
                const int kt = c / kPlanBK;
                const int32_t pos = cnt[kt * kPlanBN + r]++;
                entries[base + pos] = ((uint32_t)r << 24) | ((uint32_t)(c - kt * kPlanBK) << 16) |
                                      value_bits_f16(a.vals, a.val_dtype, j);
            }
        }
    }
    if (tid == 0) {
        uint32_t f = (uint32_t)s_flags | (fits ? 0u : kPlanMalformed);
        if (f) atomicOr(&h->flags, f);
    }
}

// One workgroup of 64 per (16-row group, cell) of `ncells` cells of
// `cols` columns: thread r < 16 counts its row's entries of the cell, thread
// 0 lays out the rows, then each thread writes its row's entries in CSR
// order (those past the record are counted in header word 1).
__global__ void __launch_bounds__(64) plan_cell_kernel(ForwardArgs a, uint32_t *out, int words, int ncells,
                                                       int cols, uint32_t kind) {
    __shared__ int32_t cnt[16], start[17];
    const int64_t g = blockIdx.x / ncells;
    const int c = (int)(blockIdx.x - g * ncells);
    const int t = threadIdx.x;
    uint32_t *rec = out + (g * ncells + c) * (int64_t)words;
    const int cap = words - kCellHdrWords;
    const int64_t c0 = (int64_t)c * cols, c1 = min(c0 + cols, a.K);
    int32_t rs = 0, re = 0;
    const int64_t n = g * 16 + t;
    if (t < 16) {
        if (n < a.N) csr_row_range(a.row_ptr, n, a.nnz, rs, re);
        int32_t k = 0;
        for (int32_t j = rs; j < re; j++) {
            const int32_t cc = a.col[j];
            k += (cc >= c0 && cc < c1) ? 1 : 0;
        }
        cnt[t] = k;
    }
    __syncthreads();
    if (t == 0) {
        int32_t run = 0;
        for (int r = 0; r < 16; r++) {
            start[r] = run;
            run += cnt[r];
        }
        start[16] = run;
        rec[0] = plan_cell_tag(kind, a.N, a.K, a.nnz, words, g, c);
        rec[1] = (uint32_t)(run > cap ? run - cap : 0);
        rec[18] = rec[19] = 0u;
    }
    __syncthreads();
    for (int i = t; i < cap; i += 64) rec[kCellHdrWords + i] = 0xffffu;
    __syncthreads();
    if (t < 16) {
        const int32_t b = min(start[t], cap), e = min(start[t + 1], cap);
        rec[2 + t] = (uint32_t)b | ((uint32_t)e << 16);
        int32_t w = start[t];
        for (int32_t j = rs; j < re; j++) {
            const int32_t cc = a.col[j];
            if (cc >= c0 && cc < c1) {
                if (w < cap) rec[kCellHdrWords + w] = (uint32_t)(cc - c0) | (value_bits_f16(a.vals, a.val_dtype, j) << 16);
                w++;
            }
        }
    }
}

hipError_t launch_plan_build(const ForwardArgs &a, void *plan, hipStream_t stream) {
    const int nblocks = (int)((a.N + kPlanBN - 1) / kPlanBN);
    const int nksteps = (int)(a.K / kPlanBK);
    PlanHeader *h = static_cast<PlanHeader *>(plan);
    int32_t *offsets = reinterpret_cast<int32_t *>(static_cast<char *>(plan) + sizeof(PlanHeader));
    uint32_t *entries = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(offsets) +
                                                     plan_offsets_bytes(a.N, a.K));
    const int qwords = plan_qrec_words(a.N, a.K, a.nnz);
    const int swords = plan_srec_words(a.N, a.K, a.nnz);
    hipLaunchKernelGGL(plan_init_kernel, dim3(1), dim3(64), 0, stream, h, nblocks, nksteps, a.N,
                       a.K, a.nnz, qwords, swords);
    const size_t lds = ((size_t)nksteps * kPlanBN + 256) * sizeof(int32_t);
    uint16_t *chunks = plan_chunks_bytes(a.N, a.K)
                           ? reinterpret_cast<uint16_t *>(static_cast<char *>(plan) + plan_chunks_at(a.N, a.K, a.nnz))
                           : nullptr;
    hipLaunchKernelGGL(plan_build_kernel, dim3(nblocks), dim3(256), lds, stream, a, h, offsets,
                       entries, chunks, nksteps);
    const unsigned ngroups = (unsigned)((a.N + 15) / 16);
    if (qwords > 0) {
        uint32_t *qrec = reinterpret_cast<uint32_t *>(static_cast<char *>(plan) + plan_rec_at(a.N, a.K, a.nnz));
        hipLaunchKernelGGL(plan_cell_kernel, dim3(ngroups * 4), dim3(64), 0, stream, a, qrec, qwords, 4,
                           decode_chunks_per_wave(a.K) * 128, kCellQuarter);
    }
    if (swords > 0) {
        const int nslices = (int)((a.K + 1023) / 1024);
        uint32_t *srec = reinterpret_cast<uint32_t *>(static_cast<char *>(plan) + plan_srec_at(a.N, a.K, a.nnz));
        hipLaunchKernelGGL(plan_cell_kernel, dim3(ngroups * (unsigned)nslices), dim3(64), 0, stream, a, srec,
                           swords, nslices, 1024, kCellSlice);
    }
    return hipGetLastError();
}

// The prefill part of a plan alone (header, offsets, entries; no chunk
// table and no cell records): what a prefill launch without a caller's plan
// builds for itself.  Its header says it holds no records.
int64_t plan_prefill_bytes(int64_t N, int64_t K, int64_t nnz) {
    if (nnz <= 0) return 0;
    return plan_chunks_at(N, K, nnz);
}

hipError_t launch_plan_build_prefill(const ForwardArgs &a, void *plan, hipStream_t stream) {
    const int nblocks = (int)((a.N + kPlanBN - 1) / kPlanBN);
    const int nksteps = (int)(a.K / kPlanBK);
    PlanHeader *h = static_cast<PlanHeader *>(plan);
    int32_t *offsets = reinterpret_cast<int32_t *>(static_cast<char *>(plan) + sizeof(PlanHeader));
    uint32_t *entries = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(offsets) +
                                                     plan_offsets_bytes(a.N, a.K));
    hipLaunchKernelGGL(plan_init_kernel, dim3(1), dim3(64), 0, stream, h, nblocks, nksteps, a.N, a.K, a.nnz, 0, 0);
    const size_t lds = ((size_t)nksteps * kPlanBN + 256) * sizeof(int32_t);
    hipLaunchKernelGGL(plan_build_kernel, dim3(nblocks), dim3(256), lds, stream, a, h, offsets, entries,
                       static_cast<uint16_t *>(nullptr), nksteps);
    return hipGetLastError();
}

// Reads the flags word of a built plan (host side, synchronous).
hipError_t plan_read_flags(const void *plan, hipStream_t stream, uint32_t *flags) {
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    PlanHeader h;
    e = hipMemcpy(&h, plan, sizeof(h), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    *flags = h.flags;
    return hipSuccess;
}

// --------------------------------------------------------------- kernel

struct PrefillArgs {
    const uint8_t *q;
    const f16 *scales;
    int64_t ngroups, G;
    const f16 *x;
    f16 *y;
    int64_t M, K, N;
    float alpha;
    int32_t nnz;
    int fold;                 // apply the ortho plan
    const PlanHeader *plan;
    const int32_t *offsets;   // [nblocks][nksteps+1]
    const uint32_t *entries;
    int nbm, nbn;             // tile grid
    const void *bias;  // [N] added after rounding (out_f16), or null
    int bias_dtype;
    // K split over the grid (256 x 128 kernel): workgroup row y takes the
    // 64-column steps [y * sps, y * sps + sps) and, when part is set, writes
    // its FP32 sums to part[y][M][N] for split_reduce_kernel; else sps = K / 64
    int sps = 1 << 30;
    float *part = nullptr;
};

constexpr int PF_BM = 256, PF_BN = 128, PF_BK = 64;
constexpr int PF_NT = 512;                        // 8 waves: 4 along tokens x 2 along rows
constexpr int PF_ROW = PF_BK;                     // halves per LDS row (no padding: swizzled)
constexpr int PF_A_BYTES = PF_BM * PF_ROW * 2;    // one activation stage (32 KB)
constexpr int PF_B_BYTES = PF_BN * PF_ROW * 2;    // one weight stage (16 KB)
constexpr int PF_OFF_INTS = (int)(kPlanMaxK / kPlanBK + 1);
constexpr int PF_A_STAGES = 2, PF_B_STAGES = 3;
constexpr int PF_B_AT = PF_A_STAGES * PF_A_BYTES;              // LDS byte offsets of the regions
constexpr int PF_OFF_AT = PF_B_AT + PF_B_STAGES * PF_B_BYTES;  // plan offsets of the tile's block
constexpr int PF_TRASH_AT = PF_OFF_AT + PF_OFF_INTS * 4;       // one fold cell per thread (own 4-byte word)
constexpr int PF_LDS_BYTES = PF_TRASH_AT + PF_NT * 4;
static_assert(PF_BN == kPlanBN && PF_BK == kPlanBK, "plan tiling must match the kernel");
static_assert(PF_LDS_BYTES <= 160 * 1024, "prefill LDS budget");

// LDS tiles are rows of 8 chunks of 16 bytes; chunk c of row r sits at
// c ^ ((r >> 1) & 7), so the 16 rows one ds_read_b128 phase touches (and
// the 8 chunks of a row one write phase touches) fall in distinct banks.
__device__ __forceinline__ int pf_swz(int r, int c) { return r * PF_ROW + ((c ^ ((r >> 1) & 7)) << 3); }

// Register sets of the software pipeline: step u's activations and plan
// entries are loaded three steps before they are written to LDS / folded,
// its raw weights four steps before they are dequantised; three statically
// indexed sets of each rotate with the step (the loop is unrolled by
// three), so a load is waited for two steps after its issue.
struct PfA { u32x4 v[4]; };                       // 256 x 64 fp16 tile: 4 x 16 B per thread
struct PfB { uint2 v; uint32_t s; };              // 16 nibbles of one weight row + its scale bits
// (the scale is kept zero-extended in a register of its own: a 16-bit value
// packed into half of a shared register would be waited for at its load)
struct PfE { uint32_t e; };                       // this thread's plan entry of the step

struct PfLane {
    uint32_t xoff[4];  // byte offsets of this thread's activation chunks (step 0)
    uint32_t qoff;     // byte offset of this thread's weight bytes (step 0)
    uint32_t soff;     // element offset of this thread's weight row scales
    int gshift;        // scale group of step u: (u0 + u) >> gshift (G = 64 << gshift; G = K: 31)
    int u0;            // the workgroup's first step (K split)
    int arow[4], achunk[4];
};

__device__ __forceinline__ void pf_load_a(const PrefillArgs &a, const PfLane &L, int u, PfA &r) {
    const char *base = reinterpret_cast<const char *>(a.x) + (int64_t)u * (PF_BK * 2);
#pragma unroll
    for (int i = 0; i < 4; i++) r.v[i] = *reinterpret_cast<const u32x4 *>(base + L.xoff[i]);
}

__device__ __forceinline__ void pf_load_b(const PrefillArgs &a, const PfLane &L, int u, PfB &r) {
    const char *base = reinterpret_cast<const char *>(a.q) + (int64_t)u * (PF_BK / 2);
    r.v = *reinterpret_cast<const uint2 *>(base + L.qoff);
    r.s = reinterpret_cast<const uint16_t *>(a.scales)[L.soff + ((uint32_t)(L.u0 + u) >> L.gshift)];
}

// This thread's plan entry for step u (the range comes from the offsets
// staged in LDS).  Threads past the range read entry 0, always valid when
// the plan is applied, and drop it.
__device__ __forceinline__ void pf_load_e(const PrefillArgs &a, const int32_t *offs, int u, PfE &r) {
    const int32_t e = min(max(offs[u], 0) + (int32_t)threadIdx.x, a.nnz - 1);
    r.e = a.entries[max(e, 0)];
}

__device__ __forceinline__ void pf_store_a(const PfLane &L, const PfA &r, f16 *As) {
#pragma unroll
    for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4 *>(As + pf_swz(L.arow[i], L.achunk[i])) = r.v[i];
}

// Byte i of word w (weights 2i, 2i+1, low nibble first) as the FP16 pair
// (q_2i * s, q_2i+1 * s), one rounding of each exact product: the byte is
// copied into both halves (v_perm), one and-xor keeps the low nibble in
// bits 0..3 of the low half under 1024.0 (0x6400) and the high nibble in
// bits 4..7 of the high half under 64.0 (0x5400), so the halves read
// 1024 + u and 64 + u with u = n ^ 8 = q + 8 (the xor by 8 folded into the
// constant); subtracting (1032, 72) gives q exactly, then the scale.
__device__ __forceinline__ uint32_t dq_byte(uint32_t w, f16x2 s2, int i) {
    const uint32_t sel = 0x0c000c00u | (uint32_t)(i * 0x00010001u);
    const uint32_t b = __builtin_amdgcn_perm(0u, w, sel);
    const uint32_t p = (b & 0x00F0000Fu) ^ 0x54806408u;
    const f16x2 bias = {(f16)-1032.0f, (f16)-72.0f};
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, p) + bias) * s2);
}

// Two FP32 values rounded (nearest even) to BF16 and packed, lo first.  For
// BF16 activations the staged weights are bf16(q * s) with q * s exact in
// FP32 (a 4-bit times an 11-bit significand): one rounding (pf_store_b).
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));  // one v_cvt_pk_bf16_f32
}

template <bool XB>
__device__ __forceinline__ void pf_store_b(const PfB &r, f16 *Bs) {
    const f16 sc = __builtin_bit_cast(f16, (uint16_t)r.s);
    const f16x2 s2 = {sc, sc};
    const float sf = (float)sc;
    const int row = threadIdx.x >> 2, c0 = (threadIdx.x & 3) * 2;
    const uint32_t words[2] = {r.v.x, r.v.y};
#pragma unroll
    for (int j = 0; j < 2; j++) {
        u32x4 o;
        if constexpr (XB) {
            // the word's even-k nibbles (lo) and odd-k nibbles (hi) as bytes
            // u = q + 8; q * s = fma(u, s, -8 s) exactly (-8 s is exact, and
            // q * s fits in the FP32 significand), then one rounding to BF16
            const uint32_t lo = (words[j] & 0x0F0F0F0Fu) ^ 0x08080808u;
            const uint32_t hi = ((words[j] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
            const float s8 = -8.0f * sf;
            auto pair = [&](int i) {
                return pk_bf16(__builtin_fmaf((float)((lo >> (8 * i)) & 0xFFu), sf, s8),
                               __builtin_fmaf((float)((hi >> (8 * i)) & 0xFFu), sf, s8));
            };
            o = u32x4{pair(0), pair(1), pair(2), pair(3)};
        } else
            o = u32x4{dq_byte(words[j], s2, 0), dq_byte(words[j], s2, 1), dq_byte(words[j], s2, 2),
                      dq_byte(words[j], s2, 3)};
        *reinterpret_cast<u32x4 *>(Bs + pf_swz(row, c0 + j)) = o;
    }
}

// A staged weight (FP16, or BF16 when XB) plus alpha * v, rounded back.
template <bool XB>
__device__ __forceinline__ uint16_t fold_add(uint16_t cell, float add) {
    if constexpr (XB) return __builtin_bit_cast(uint16_t, (__bf16)(bf16_bits_to_f32(cell) + add));
    else return __builtin_bit_cast(uint16_t, (f16)((float)__builtin_bit_cast(f16, cell) + add));
}

// Adds alpha * v to the weight cell of entry e; a thread with no entry
// updates its own trash cell instead, so the common path has no branch.
template <bool XB>
__device__ __forceinline__ void fold_fast(f16 *Bs, f16 *trash, uint32_t e, bool valid, float alpha) {
    const int r = (e >> 24) & (PF_BN - 1), c = (e >> 16) & (PF_BK - 1);  // always inside the tile
    const float v = (float)__builtin_bit_cast(f16, (uint16_t)(e & 0xffffu));
    uint16_t *p = reinterpret_cast<uint16_t *>(valid ? Bs + pf_swz(r, c >> 3) + (c & 7) : trash + 2 * threadIdx.x);
    *p = fold_add<XB>(*p, alpha * v);
}

// Folds step u's plan entries into the weight stage Bs.  The first 512
// entries come from the prefetched register; a step with more (dense rows,
// skewed outliers) reads the rest here.
template <bool XB>
__device__ __forceinline__ void pf_fold(const PrefillArgs &a, const int32_t *offs, int u, const PfE &r,
                                        f16 *Bs, f16 *trash, bool canonical) {
    const int tid = threadIdx.x;
    // (the staged offsets are already within [0, nnz]; clamping again keeps
    // every entry read in bounds whatever the LDS holds)
    const int32_t lo = max(offs[u], 0), hi = min(offs[u + 1], a.nnz);
    if (canonical) {
        fold_fast<XB>(Bs, trash, r.e, lo + tid < hi, a.alpha);
        // canonical entries are distinct cells: no ordering between passes
        if (hi - lo > PF_NT)
            for (int32_t e = lo + PF_NT + tid; e < hi; e += PF_NT) fold_fast<XB>(Bs, trash, a.entries[e], true, a.alpha);
    } else if (tid < PF_BN) {
        // rows with duplicate or unsorted columns: one thread per row of the
        // block applies that row's entries of the step one after another in
        // plan order (row, then CSR position), so entries of one cell add in
        // a fixed order (the result is reproducible bit for bit) and no two
        // threads touch one cell.  The step's entries are sorted by row:
        // this row's run starts at the first entry whose row is not below it.
        int32_t b = lo, e_hi = hi;
        while (b < e_hi) {
            const int32_t mid = b + ((e_hi - b) >> 1);
            if ((int)((a.entries[mid] >> 24) & (PF_BN - 1)) < tid) b = mid + 1;
            else e_hi = mid;
        }
        for (int32_t e = b; e < hi; e++) {
            const uint32_t w = a.entries[e];
            if ((int)((w >> 24) & (PF_BN - 1)) != tid) break;
            fold_fast<XB>(Bs, trash, w, true, a.alpha);
        }
    }
}

template <bool XB>
__device__ __forceinline__ void pf_mfma(const f16 *As, const f16 *Bs, int wm, int wn,
                                        f32x16 (&acc)[2][2]) {
    const int lane = threadIdx.x & 63;
    const int lr = lane & 31, kh = lane >> 5;
#pragma unroll
    for (int s = 0; s < PF_BK / 16; s++) {
        f16x8 af[2], bf[2];
#pragma unroll
        for (int bm = 0; bm < 2; bm++)
            af[bm] = *reinterpret_cast<const f16x8 *>(As + pf_swz(wm * 64 + bm * 32 + lr, 2 * s + kh));
#pragma unroll
        for (int bn = 0; bn < 2; bn++)
            bf[bn] = *reinterpret_cast<const f16x8 *>(Bs + pf_swz(wn * 64 + bn * 32 + lr, 2 * s + kh));
#pragma unroll
        for (int bm = 0; bm < 2; bm++)
#pragma unroll
            for (int bn = 0; bn < 2; bn++)
                if constexpr (XB)
                    acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[bm]),
                                                                          __builtin_bit_cast(bf16x8, bf[bn]),
                                                                          acc[bm][bn], 0, 0, 0);
                else
                    acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[bm], bf[bn], acc[bm][bn], 0, 0, 0);
    }
}

// One pipeline step t (J = t mod 3, static): the MFMAs consume step t's
// stages first; then the loads of steps t+3 (activations, plan entries) and
// t+4 (weights) are issued, step t+1's activations written, step t+2's
// weights dequantised and step t+1's plan entries folded (its weights were
// written one step ago); one barrier.  Issuing the MFMAs first lets them run
// while the wave waits for the memory queue, older loads and the fold's LDS
// read-modify-write.  Activations use two LDS stages, weights
// three, so no write touches a stage being read.
template <bool FOLD, int J, bool XB>
__device__ __forceinline__ void pf_step(const PrefillArgs &a, const PfLane &L, int t, int nk, int wm,
                                        int wn, f16 *As0, f16 *Bs0, const int32_t *offs, f16 *trash,
                                        bool canonical, PfA (&ra)[3], PfB (&rb)[3], PfE (&re)[3],
                                        f32x16 (&acc)[2][2]) {
    constexpr int J1 = (J + 1) % 3, J2 = (J + 2) % 3;
    // keep the scheduler from hoisting a later step's register work (which
    // would wait for younger loads) above this step's barrier
    __builtin_amdgcn_sched_barrier(0);
    f16 *B_t = Bs0 + J * (PF_B_BYTES / 2), *B_1 = Bs0 + J1 * (PF_B_BYTES / 2), *B_2 = Bs0 + J2 * (PF_B_BYTES / 2);
    pf_mfma<XB>(As0 + (t & 1) * (PF_A_BYTES / 2), B_t, wm, wn, acc);
    pf_load_a(a, L, min(t + 3, nk - 1), ra[J]);
    pf_load_b(a, L, min(t + 4, nk - 1), rb[J1]);
    if (FOLD) pf_load_e(a, offs, min(t + 3, nk - 1), re[J]);
    pf_store_a(L, ra[J1], As0 + ((t + 1) & 1) * (PF_A_BYTES / 2));
    pf_store_b<XB>(rb[J2], B_2);
    if (FOLD) pf_fold<XB>(a, offs, min(t + 1, nk - 1), re[J1], B_1, trash, canonical);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
}

// XB: BF16 activations and output (v_mfma_f32_32x32x16_bf16, the staged
// weights bf16(q*s), the fold in BF16).
template <bool FOLD, bool XB>
__global__ void __launch_bounds__(PF_NT) prefill_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    f16 *As0 = reinterpret_cast<f16 *>(smem);
    f16 *Bs0 = reinterpret_cast<f16 *>(smem + PF_B_AT);
    int32_t *offs = reinterpret_cast<int32_t *>(smem + PF_OFF_AT);
    f16 *trash = reinterpret_cast<f16 *>(smem + PF_TRASH_AT);

    // XCD-aware tile order: workgroup ids are dealt round-robin to the 8
    // XCDs; give each XCD a contiguous run of tiles (N-block fastest).
    const int ntiles = a.nbm * a.nbn;
    int tile = blockIdx.x;
    if ((ntiles & 7) == 0) tile = (blockIdx.x & 7) * (ntiles >> 3) + (blockIdx.x >> 3);
    const int bm_i = tile / a.nbn, bn_i = tile - bm_i * a.nbn;
    const int64_t m0 = (int64_t)bm_i * PF_BM, n0 = (int64_t)bn_i * PF_BN;

    const int tid = threadIdx.x, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // this workgroup's steps of K (the host sizes the grid so that every
    // workgroup row has at least one)
    const int nk_all = (int)(a.K / PF_BK);
    const int u0 = (int)blockIdx.y * a.sps;
    const int nk = min(a.sps, nk_all - u0);

    // per-thread offsets, fixed for the whole K loop (rows past M / N repeat
    // the last row; their outputs are never stored)
    PfLane L;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int idx = tid + PF_NT * i;
        L.arow[i] = idx >> 3;
        L.achunk[i] = idx & 7;
        const int64_t m = min(m0 + L.arow[i], a.M - 1);
        L.xoff[i] = (uint32_t)((m * a.K + (int64_t)u0 * PF_BK + L.achunk[i] * 8) * 2);
    }
    {
        const int64_t n = min(n0 + (tid >> 2), a.N - 1);
        L.qoff = (uint32_t)(n * (a.K >> 1) + (int64_t)u0 * (PF_BK / 2) + (tid & 3) * 8);
        L.soff = (uint32_t)(n * a.ngroups);
        L.gshift = a.ngroups == 1 ? 31 : __builtin_ctzll(a.G / PF_BK);
        L.u0 = u0;
    }

    bool canonical = true;
    if (FOLD) {
        // the plan's offsets of this tile's row block, clamped to [0, nnz]:
        // a stale or foreign plan can lose the ortho term but never makes a
        // read outside the entry array (a pair with hi < lo is an empty step,
        // and every entry lands inside the tile).  A plan built for another
        // layer shape is ignored rather than trusted.
        const PlanHeader *h = a.plan;
        const bool ok = h->magic == kPlanMagic && h->version == kPlanVersion && h->n == a.N &&
                        h->k == a.K && h->nnz == a.nnz;
        for (int i = tid; i <= nk; i += PF_NT)
            offs[i] = ok ? min(max(a.offsets[(int64_t)bn_i * (nk_all + 1) + u0 + i], 0), a.nnz) : 0;
        canonical = !ok || (h->flags & kPlanNonCanonical) == 0;
        __syncthreads();
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
        for (int bn = 0; bn < 2; bn++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[bm][bn][i] = 0.f;

    // prologue: step 0 in its stages (folded), step 1's weights dequantised;
    // activations 1, 2, weights 2, 3 and plan entries 1, 2 in flight
    PfA ra[3];
    PfB rb[3];
    PfE re[3];
    pf_load_a(a, L, 0, ra[0]);
    pf_load_b(a, L, 0, rb[0]);
    pf_load_b(a, L, min(1, nk - 1), rb[1]);
    if (FOLD) pf_load_e(a, offs, 0, re[0]);
    pf_store_a(L, ra[0], As0);
    pf_store_b<XB>(rb[0], Bs0);
    pf_store_b<XB>(rb[1], Bs0 + PF_B_BYTES / 2);
    __syncthreads();
    if (FOLD) pf_fold<XB>(a, offs, 0, re[0], Bs0, trash, canonical);
    // (issued in the loop's own order, so the wait counts at the loop head
    // are the same from the prologue as from the back edge)
    __builtin_amdgcn_sched_barrier(0);
    pf_load_a(a, L, min(1, nk - 1), ra[1]);
    pf_load_b(a, L, min(2, nk - 1), rb[2]);
    if (FOLD) pf_load_e(a, offs, min(1, nk - 1), re[1]);
    __builtin_amdgcn_sched_barrier(0);
    pf_load_a(a, L, min(2, nk - 1), ra[2]);
    pf_load_b(a, L, min(3, nk - 1), rb[0]);
    if (FOLD) pf_load_e(a, offs, min(2, nk - 1), re[2]);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    int t = 0;
    for (; t + 3 <= nk; t += 3) {
        pf_step<FOLD, 0, XB>(a, L, t, nk, wm, wn, As0, Bs0, offs, trash, canonical, ra, rb, re, acc);
        pf_step<FOLD, 1, XB>(a, L, t + 1, nk, wm, wn, As0, Bs0, offs, trash, canonical, ra, rb, re, acc);
        pf_step<FOLD, 2, XB>(a, L, t + 2, nk, wm, wn, As0, Bs0, offs, trash, canonical, ra, rb, re, acc);
    }
    if (t < nk) pf_step<FOLD, 0, XB>(a, L, t, nk, wm, wn, As0, Bs0, offs, trash, canonical, ra, rb, re, acc);
    if (t + 1 < nk) pf_step<FOLD, 1, XB>(a, L, t + 1, nk, wm, wn, As0, Bs0, offs, trash, canonical, ra, rb, re, acc);

    // epilogue: lane holds D[token 8(i/4) + 4(lane/32) + i%4][row lane%32]
    // of each 32 x 32 tile, one output column per lane.  Each wave stages
    // its 32-token halves in LDS (the stages are free now) and stores whole
    // token rows: 4 consecutive outputs per lane (16 bytes of FP32 partials,
    // 8 of FP16 / BF16 output) instead of one.  Measured: the direct stores
    // took 3.3-4.6 us of a launch.
    const int lane = tid & 63;
    float *part = a.part ? a.part + (int64_t)blockIdx.y * a.M * a.N : nullptr;
    // (row stride 72 floats: the two token halves of a write land in
    // different banks, and 16-byte reads of a token row stay aligned)
    constexpr int ES = 72;
    static_assert(PF_NT / 64 * 32 * ES * 4 <= PF_LDS_BYTES, "epilogue staging fits the LDS");
    float *stg = reinterpret_cast<float *>(smem) + wave * (32 * ES);
    const bool vec = (a.N & 3) == 0;
    __syncthreads();
#pragma unroll
    for (int bm = 0; bm < 2; bm++) {
#pragma unroll
        for (int bn = 0; bn < 2; bn++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                stg[(8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * ES + bn * 32 + (lane & 31)] = acc[bm][bn][i];
        __syncthreads();
        const int c4 = (lane & 15) * 4;
        const int64_t n = n0 + wn * 64 + c4;
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int tt = it * 4 + (lane >> 4);
            const int64_t m = m0 + wm * 64 + bm * 32 + tt;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(stg + tt * ES + c4);
            if (m >= a.M || n >= a.N) continue;
            if (vec) {
                // (N % 4 == 0 and n % 4 == 0: all four inside the row, aligned)
                if (part) {
                    *reinterpret_cast<f32x4 *>(part + m * a.N + n) = v;
                } else {
                    uint32_t h[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if constexpr (XB) h[e] = out_bf16(v[e], a.bias, a.bias_dtype, n + e);
                        else h[e] = __builtin_bit_cast(uint16_t, out_f16(v[e], a.bias, a.bias_dtype, n + e));
                    }
                    *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(a.y) + m * a.N + n) =
                        uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (n + e >= a.N) break;
                    if (part) part[m * a.N + n + e] = v[e];
                    else if constexpr (XB)
                        reinterpret_cast<uint16_t *>(a.y)[m * a.N + n + e] = out_bf16(v[e], a.bias, a.bias_dtype, n + e);
                    else
                        a.y[m * a.N + n + e] = out_f16(v[e], a.bias, a.bias_dtype, n + e);
                }
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------- wide-row prefill tile
//
// For layers wide enough to give every CU one tile in one round (4096 ->
// 11008 at 2048 tokens: 8 token tiles x 32 row ranges of 352 rows = 256
// workgroups; the 256 x 128 tile above needs 688 tiles, 2.69 rounds), and
// with 128-row tiles in 64-column steps for narrower layers (c3: 256
// workgroups of 256 x 128).
//
//  * Workgroup tile 256 tokens x R = 32 * NRT rows, 8 waves (two per SIMD,
//    so one's MFMAs run beside the other's dequantisation) in a 4 x 2 grid,
//    each 64 tokens x 16 NRT rows with v_mfma_f32_16x16x32_f16, the weights
//    as the first operand: 4 x NRT accumulator tiles (176 registers at NRT
//    = 11).  Each operand read from LDS feeds NRT (activations) or 4
//    (weights) MFMAs.
//  * K advances 32 KS columns a step: activations in 2 LDS stages, loaded
//    straight into LDS (buffer_load ... lds); dequantised weights (the same
//    fp16(q * s) as above, one 4-byte word of nibbles per job, 4 KS threads
//    per row) in 3 stages; group scales loaded only at the steps that start
//    a group.
//  * The ortho plan's (128-row block, 64-column step) entries of the up to
//    four blocks the row range touches are folded into the weight stage one
//    step after its dequantisation (each 64-column plan step in two halves
//    when KS = 1), late in the step, so one barrier a step orders
//    everything and an entry load has nearly a step to land.
//  * Each step is laid out by hand in 4 NRT KS slots, one MFMA each.
//  * Workgroup b takes token tile b % TT and row range b / TT: with 8 token
//    tiles each XCD holds one token tile's activations in its L2.
constexpr int PW_BM = 256, PW_BK = 32, PW_NT = 512;
constexpr int PW_A_BYTES = PW_BM * PW_BK * 2;  // one activation stage (16 KB)
constexpr int PW_MAX_BLOCKS = 4;               // plan blocks a row range may touch
constexpr int PW_E = 1;                        // plan entries per thread prefetched per 64-column step

// LDS layout of a stage: rows r and r + 1 (r even) share a 128-byte line,
// chunk c (16 bytes, 8 columns) of row r at slot ((r % 2) * 4 + c) ^ (line
// % 8) of line r / 2.  Measured with a probe of ds_read_b128 access tables
// on gfx950 (SQ_LDS_BANK_CONFLICT): conflict-free for the MFMA operand
// read (16 rows of one chunk per 16 lanes) and for writes of 4 lanes per
// row (the 4 chunks of a row: the coalesced loads' mapping, used for both
// stages); row-major 64-byte rows conflicted 2-way on the operand read
// whatever their XOR swizzle (43 % of the LDS's active cycles stalled),
// and a chunk-major tile 4-way on these writes.  Result in halves.
__device__ __forceinline__ int pw_swz(int r, int c) {
    const int line = r >> 1;
    return line * 64 + (((((r & 1) << 2) | c) ^ (line & 7)) << 3);
}

// A step is ks sub-steps of 32 columns (ks = 1 or 2); a stage holds ks
// sub-stages of the layout above.  A weight stage holds the rows the chunk
// jobs reach (a thread's last job lands in rows past R when there is none:
// never read; no branch).
__host__ __device__ constexpr int pw_njobs(int nrt, int ks) { return (4 * ks * 32 * nrt + PW_NT - 1) / PW_NT; }
__host__ __device__ constexpr int pw_b_rows(int nrt, int ks) { return pw_njobs(nrt, ks) * PW_NT / (4 * ks); }
__host__ __device__ constexpr int pw_b_bytes(int nrt, int ks) { return pw_b_rows(nrt, ks) * PW_BK * 2 * ks; }
__host__ __device__ constexpr int pw_off_at(int nrt, int ks) { return 2 * PW_A_BYTES * ks + 3 * pw_b_bytes(nrt, ks); }
__host__ __device__ constexpr int pw_trash_at(int nrt, int ks) {
    return pw_off_at(nrt, ks) + PW_MAX_BLOCKS * (int)(kPlanMaxK / kPlanBK + 1) * 4;
}
// (a thread's trash cell: the low half of its own 4-byte word, so that a
// wave's trash writes fall in distinct banks)
__host__ __device__ constexpr int pw_lds_bytes(int nrt, int ks) { return pw_trash_at(nrt, ks) + PW_NT * 4; }

struct PwB { uint32_t v[3]; uint32_t s[3]; };  // up to 3 chunks (a 4-byte word of nibbles each) + scale bits
// a thread's plan entries of one 64-column step: the entry words and the
// row offset of their block in the range (even; bit 0 of brow[0]: the block
// holds more entries than its threads prefetch)
struct PwE { uint32_t e[PW_E]; int brow[PW_E]; };

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4
// ... lds): lane i's land at lds + 16 i (lds the same in every lane)
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
}

// f(integral_constant<int, k>) for k = 0 .. N-1, unrolled at compile time
template <class F, int... Is>
__device__ __forceinline__ void pw_static_for(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}

// Slot plan of a step (4 NRT MFMA slots, the barrier before the last 4):
// the 4 NJ dequantised byte pairs spread evenly over the slots before the
// barrier, the rest in the gaps.  pw_dq_at: the byte pair of slot k, or -1.
constexpr int pw_dq_slot(int b, int nslots, int nbytes) { return (b * nslots) / nbytes; }
constexpr int pw_dq_at(int k, int nslots, int nbytes) {
    for (int b = 0; b < nbytes; b++)
        if (pw_dq_slot(b, nslots, nbytes) == k) return b;
    return -1;
}

// KS: 32-column sub-steps per step (1, or 2 for a 128-row tile, whose
// step would otherwise hold too few MFMAs for its barrier and loads)
template <int NRT, int KS, bool FOLD, bool XB>
__global__ void __launch_bounds__(PW_NT, 1) prefill_wide_kernel(PrefillArgs a) {
    constexpr int R = 32 * NRT;                 // rows of the workgroup tile
    constexpr int NJ = pw_njobs(NRT, KS);  // chunk jobs per thread (dequantisation: 8 weights each)
    constexpr int RS = pw_b_rows(NRT, KS);  // rows of a weight sub-stage
    constexpr int JW = 4 * KS;              // 4-byte words of a row per step (= threads per row)
    static_assert(NJ <= 3 && (KS == 1 || KS == 2), "three chunk jobs per thread at most");
    extern __shared__ __align__(16) unsigned char smem[];
    f16 *As0 = reinterpret_cast<f16 *>(smem);
    f16 *Bs0 = reinterpret_cast<f16 *>(smem + 2 * PW_A_BYTES * KS);
    int32_t *offs = reinterpret_cast<int32_t *>(smem + pw_off_at(NRT, KS));
    f16 *trash = reinterpret_cast<f16 *>(smem + pw_trash_at(NRT, KS));

    const int tt = (int)(blockIdx.x % (unsigned)a.nbm), rr = (int)(blockIdx.x / (unsigned)a.nbm);
    const int64_t m0 = (int64_t)tt * PW_BM, n0 = (int64_t)rr * R;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: scalar addressing)
    // the thread id formed again where the loop needs it (wave in a scalar
    // register, the lane from v_mbcnt): keeping it live costs a register
    auto tid_now = [&]() -> int {
        return wave * 64 + (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    };
    const int wm = wave & 3, wn = wave >> 2;
    const int nk = (int)(a.K / (PW_BK * KS));
    const int nk64 = (int)(a.K / kPlanBK);
    // plan step and half (columns 32 h .. + 31 of it, KS == 1) of step v
    auto pstep = [&](int v) -> int { return KS == 2 ? v : v >> 1; };

    // per-thread byte offsets (step 0) of the first chunk / job; the others
    // are formed at each load (registers are the limit here).  Rows past M
    // / N repeat the last row.
    // activations: loaded straight into LDS (buffer_load_dwordx4 ... lds:
    // lane i of a wave's load lands at its base + 16 i).  Load c of wave w
    // fills rows 16 (2 w + c) .. + 15 (8 lines of the swizzled stage, 1 KB):
    // lane i takes line i / 8, slot i % 8, i.e. row 2 (i / 8) + (s >> 2),
    // chunk s & 3 with s = (i % 8) ^ (i / 8), so the two rows of a line are
    // read as two 64-byte runs (4 lanes each)
    const int xs = (lane & 7) ^ (lane >> 3);
    const uint32_t xrow = (uint32_t)(m0 + 32 * wave + 2 * (lane >> 3) + (xs >> 2));
    const uint32_t xcol = (uint32_t)((xs & 3) * 16);
    auto xoff = [&](int c) -> uint32_t {
        return min(xrow + (uint32_t)(16 * c), (uint32_t)(a.M - 1)) * (uint32_t)(a.K * 2) + xcol;
    };
    // weight job i of this thread: j = tid + 512 i, row j / JW, word j % JW:
    // sub-stage word / 4, chunk word % 4 (the same mapping as the
    // activations: JW lanes read a row's 16 KS contiguous bytes of nibbles);
    // past R rows it writes the stage's spare rows
    auto job = [&](int i) -> int { return tid + PW_NT * i; };
    static_assert(PW_NT * NJ / JW <= RS && RS >= R, "chunk jobs stay inside the stage");
    // LDS write offset (halves) of job 0 (job i: + 512 / JW i rows; the
    // swizzle leaves bits 4 and up of a row alone)
    const int awo = ((tid % JW) >> 2) * (RS * PW_BK) + pw_swz(tid / JW, tid & 3);
    const uint32_t qrow0 = (uint32_t)(n0 + tid / JW), qh = (uint32_t)(tid % JW) * 4;
    auto qrow_of = [&](int i) -> uint32_t { return min(qrow0 + (uint32_t)(i * (PW_NT / JW)), (uint32_t)(a.N - 1)); };
    const int gshift = a.ngroups == 1 ? 31 : __builtin_ctzll(a.G / (PW_BK * KS));
    const uint32_t gmask = (1u << gshift) - 1u;  // steps u with u & gmask == 0 start a group

    // plan blocks of the row range, their offsets staged in LDS
    const int nblk = (int)((a.N + kPlanBN - 1) / kPlanBN);
    const int b_lo = (int)(n0 / kPlanBN);
    const int nb = FOLD ? max(0, min(PW_MAX_BLOCKS, min(nblk, (int)((n0 + R - 1) / kPlanBN) + 1) - b_lo)) : 0;
    bool canonical = true;  // (set with the offsets' staging, in the prologue)

    // buffer loads: a 32-bit lane offset that stays the same for the whole
    // K loop plus the step's offset in a scalar register (one VGPR per
    // stream instead of a 64-bit address each; registers are the limit)
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16 *>(a.x), (short)0, (int)(uint32_t)(a.M * a.K * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(a.q), (short)0, (int)(uint32_t)(a.N * (a.K / 2)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16 *>(a.scales), (short)0, (int)(uint32_t)(a.N * a.ngroups * 2), 0x00020000);
    // load c (0, 1) of A(u) into stage As; no register holds the data, so
    // the compiler inserts no wait for it: whoever reads the stage waits
    // for the loads (vmcnt) before the barrier that publishes it
    // (sub-stage c / 2 of the step, half c % 2 of the wave's rows)
    auto dma_a = [&](int u, int c, f16 *As) {
        buffer_load_lds16(rx, As + (c >> 1) * (PW_A_BYTES / 2) + (PW_A_BYTES / 16) * wave + (PW_A_BYTES / 32) * (c & 1),
                          xoff(c & 1) + (uint32_t)(c >> 1) * (PW_BK * 2), u * (PW_BK * 2 * KS));
    };
    auto load_b = [&](int u, PwB &r) {
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            const uint32_t n = qrow_of(i);
            r.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rq, n * (uint32_t)(a.K >> 1) + qh, u * (PW_BK / 2 * KS), 0);
            r.s[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, n * (uint32_t)(a.ngroups * 2), ((uint32_t)u >> gshift) * 2, 0);
        }
    };
    // one chunk (8 weights) of a word of nibbles, fp16(q * s) or bf16(q * s)
    auto dq_chunk = [&](uint32_t word, uint32_t sbits) -> u32x4 {
        const f16 sc = __builtin_bit_cast(f16, (uint16_t)sbits);
        if constexpr (XB) {
            const float sf = (float)sc;
            const uint32_t lo = (word & 0x0F0F0F0Fu) ^ 0x08080808u;
            const uint32_t hi = ((word >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
            auto pair = [&](int b) {
                return pk_bf16(__builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), sf, -8.0f * sf),
                               __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), sf, -8.0f * sf));
            };
            return u32x4{pair(0), pair(1), pair(2), pair(3)};
        } else {
            const f16x2 s2 = {sc, sc};
            return u32x4{dq_byte(word, s2, 0), dq_byte(word, s2, 1), dq_byte(word, s2, 2), dq_byte(word, s2, 3)};
        }
    };
    auto store_b = [&](const PwB &r, f16 *Bs) {
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            *reinterpret_cast<u32x4 *>(Bs + awo + i * (PW_NT / JW) * PW_BK) = dq_chunk(r.v[i], r.s[i]);
        }
    };

    // thread tid takes entries tid % 128 (+ 128 e) of block tid / 128 of the
    // row range (the range touches at most 4 blocks): two offset reads, no
    // search
    constexpr int EPB = PW_NT / PW_MAX_BLOCKS;  // threads per block
    auto load_e = [&](int u, PwE &r) {
        const int eb = tid_now() >> 7, ep = tid_now() & (EPB - 1);
        u = min(u, nk64 - 1);
        const bool vb = eb < nb;
        const int o = (vb ? eb : 0) * (nk64 + 1) + u;
        const int l = offs[o], h = max(l, offs[o + 1]);
        const int total = vb ? h - l : 0;  // (this thread's block)
#pragma unroll
        for (int e = 0; e < PW_E; e++) {
            r.e[e] = a.entries[min(max(l + ep + EPB * e, 0), a.nnz - 1)];
            r.brow[e] = ep + EPB * e < total ? (b_lo + eb) * kPlanBN - (int)n0 : -(1 << 20);
        }
        r.brow[0] |= total > PW_E * EPB ? 1 : 0;
    };
    // alpha * v of every entry of 64-column plan step u whose column falls
    // in half `half` (KS == 1; KS == 2: the whole plan step is the stage)
    // into the weight stage Bs (rows of the range only).  The cell of (local
    // row, column c of the 64) gets alpha * v; a thread with nothing to add
    // updates its own trash cell (no branch).
    auto cell_at = [&](f16 *Bs, int local, int c) -> f16 * {
        return Bs + (KS == 2 ? (c >> 5) * (RS * PW_BK) : 0) + pw_swz(min(max(local, 0), R - 1), (c & 31) >> 3) + (c & 7);
    };
    auto in_half = [&](int c, int half) -> bool { return KS == 2 || (c >> 5) == half; };
    auto cell = [&](f16 *Bs, int local, int c, uint32_t w, bool ok) {
        const float v = (float)__builtin_bit_cast(f16, (uint16_t)(w & 0xffffu));
        uint16_t *p = reinterpret_cast<uint16_t *>(ok ? cell_at(Bs, local, c) : trash + 2 * tid_now());
        *p = fold_add<XB>(*p, a.alpha * v);
    };
    auto one = [&](f16 *Bs, int half, uint32_t w, int brow) {
        const int local = (brow & ~1) + (int)(w >> 24);
        const int c = (int)((w >> 16) & (kPlanBK - 1));
        cell(Bs, local, c, w, local >= 0 && local < R && in_half(c, half));
    };
    // the prefetched entries (canonical plans), no branch
    auto fold_common = [&](int half, const PwE &r, f16 *Bs) {
#pragma unroll
        for (int e = 0; e < PW_E; e++) one(Bs, half, r.e[e], canonical ? r.brow[e] : -(1 << 20));
    };
    // the rest (uniform branch): entries past the prefetched ones, or the
    // whole step for a plan with duplicate or unsorted columns
    auto fold_rare = [&](int u, int half, f16 *Bs) {
        u = min(u, nk64 - 1);
        if (canonical) {
            // this thread's block holds more entries than the prefetched ones
            const int eb = tid_now() >> 7, ep = tid_now() & (EPB - 1);
            const int o = (eb < nb ? eb : 0) * (nk64 + 1) + u;
            const int l = offs[o], total = eb < nb ? max(l, offs[o + 1]) - l : 0;
            for (int v = PW_E * EPB + ep; v < total; v += EPB)
                one(Bs, half, a.entries[min(max(l + v, 0), a.nnz - 1)], (b_lo + eb) * kPlanBN - (int)n0);
        } else {
            // one thread per row applies the row's entries of the step in
            // plan order (the result is reproducible bit for bit)
            for (int lr = tid_now(); lr < R; lr += PW_NT) {
                const int64_t n = n0 + lr;
                if (n >= a.N) break;
                const int bb = (int)(n / kPlanBN) - b_lo;
                if (bb < 0 || bb >= nb) continue;
                const int rib = (int)(n % kPlanBN);
                const int32_t lo = offs[bb * (nk64 + 1) + u], hi = min(offs[bb * (nk64 + 1) + u + 1], a.nnz);
                int32_t b = lo, e_hi = hi;
                while (b < e_hi) {
                    const int32_t mid = b + ((e_hi - b) >> 1);
                    if ((int)(a.entries[mid] >> 24) < rib) b = mid + 1;
                    else e_hi = mid;
                }
                for (int32_t e = b; e < hi; e++) {
                    const uint32_t w = a.entries[e];
                    if ((int)(w >> 24) != rib) break;
                    const int c = (int)((w >> 16) & (kPlanBK - 1));
                    if (in_half(c, half)) cell(Bs, lr, c, w, true);
                }
            }
        }
    };

    f32x4 acc[4][NRT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NRT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};


    // one register set each for the raw weights and the plan entries: a
    // step writes the set it holds to LDS (or folds it), then loads the next
    // step's into it (a load still has a full step to land)
    PwB rb;
    PwE re;
    auto Bst = [&](int s) { return Bs0 + s * (pw_b_bytes(NRT, KS) / 2); };
    auto Ast = [&](int s) { return As0 + s * (PW_A_BYTES / 2 * KS); };

    // prologue: stage 0 folded, stage 1 dequantised; A(1), B(2) and the
    // entries of stage 1's fold in flight.  The first stages' loads are
    // issued before the plan offsets are staged, so that their round trips
    // overlap (one at the start of the kernel instead of three in a row).
    PwB rb1;  // B(1)
#pragma unroll
    for (int c = 0; c < 2 * KS; c++) dma_a(0, c, Ast(0));
#pragma unroll
    for (int c = 0; c < 2 * KS; c++) dma_a(min(1, nk - 1), c, Ast(1));
    // (A(0) and A(1) have landed once B(0)'s loads, issued after them, have:
    // the memory counter retires in order)
    load_b(0, rb);
    load_b(min(1, nk - 1), rb1);
    if (FOLD) {
        const PlanHeader *h = a.plan;
        const bool ok = h->magic == kPlanMagic && h->version == kPlanVersion && h->n == a.N &&
                        h->k == a.K && h->nnz == a.nnz;
        for (int i = tid; i < nb * (nk64 + 1); i += PW_NT) {
            const int bb = i / (nk64 + 1), u = i - bb * (nk64 + 1);
            offs[i] = ok ? min(max(a.offsets[(int64_t)(b_lo + bb) * (nk64 + 1) + u], 0), a.nnz) : 0;
        }
        canonical = !ok || (h->flags & kPlanNonCanonical) == 0;
        __syncthreads();
    }
    if (FOLD) load_e(0, re);
    store_b(rb, Bst(0));
    load_b(min(2, nk - 1), rb);
    store_b(rb1, Bst(1));
    __syncthreads();
    if (FOLD) {
        fold_common(0, re, Bst(0));
        if (!canonical || (re.brow[0] & 1)) fold_rare(0, 0, Bst(0));
        load_e(pstep(1), re);
    }
    __syncthreads();

    // step t: MFMAs on A(t % 2), B(t % 3); A(t+1) written and A(t+2) loaded,
    // B(t+2) dequantised and B(t+3) loaded, B(t+1) folded (64-column step
    // (t+1)/2, half (t+1)%2) and the entries of the next step's fold loaded;
    // one barrier.
    //
    // The step is laid out by hand in 4 NRT slots, one MFMA each followed by
    // a slice of the rest (sched_barrier between slots): the dequantisation
    // and the LDS and memory traffic of the next stages run while the
    // matrix core works.  (Left to the scheduler, each wave issued its MFMAs
    // back to back and its VALU work after them, and the step's barrier kept
    // the two waves of a SIMD in the same phase: 3,600 cycles a step
    // against 1,408 of MFMAs.)
    int b3 = 0;  // t % 3
    constexpr int NS = 4 * NRT * KS;  // slots of a step
    constexpr int PRE = NS - 4;       // slots before the step's barrier
    const int aro = pw_swz(lane & 15, lane >> 4);
    // operand reads: row 16 m + lr, chunk lc sits at aro + 16 m rows (the
    // swizzle depends on the row's bits 1..3 only).  A step's A operands and
    // its first B operand are read at the end of the step before (after its
    // barrier), into the registers its last MFMAs free.
    f16x8 af[4], bcur, bnext;
    {
        const f16 *Ar = Ast(0) + aro + 64 * wm * PW_BK, *Br = Bst(0) + aro + (R / 2) * wn * PW_BK;  // (sub-stage 0)
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *reinterpret_cast<const f16x8 *>(Ar + 16 * i * PW_BK);
        bnext = *reinterpret_cast<const f16x8 *>(Br);
    }
    for (int t = 0; t < nk; t++) {
        __builtin_amdgcn_sched_barrier(0);
        const int b3_1 = b3 == 2 ? 0 : b3 + 1, b3_2 = b3 == 0 ? 2 : b3 - 1;
        const int u1 = pstep(t + 1), h1 = (t + 1) & 1;
        const bool rare = FOLD && (!canonical || (re.brow[0] & 1));  // (per thread: its block overflows)
        const int u3 = min(t + 3, nk - 1);                         // B loads of this step: step u3
        const bool sload = ((uint32_t)u3 & gmask) == 0u;           // (uniform) u3 starts a group
        const f16 *Bs = Bst(b3);
        f16 *Bw = Bst(b3_2), *Bf = Bst(b3_1), *Aw2 = Ast(t & 1);

        const f16 *Br = Bs + aro + (R / 2) * wn * PW_BK;
        // the next step's operands (read after this step's barrier)
        const f16 *An = Ast((t + 1) & 1) + aro + 64 * wm * PW_BK, *Bn = Bst(b3_1) + aro + (R / 2) * wn * PW_BK;

        // dequantisation state of the current job and word
        f16x2 s2 = {};
        float sf = 0.f;
        uint32_t wlo = 0, whi = 0, out[4] = {0, 0, 0, 0};
        // fold state
        uint16_t *fp = nullptr;
        uint16_t fold_old = 0;

        pw_static_for([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            constexpr int sub = k / (4 * NRT), j = (k % (4 * NRT)) / 4, i = k % 4;
            if constexpr (i == 0) {
                bcur = bnext;
                if constexpr (j + 1 < NRT)
                    bnext = *reinterpret_cast<const f16x8 *>(Br + sub * (RS * PW_BK) + 16 * (j + 1) * PW_BK);
                else if constexpr (sub + 1 < KS)
                    bnext = *reinterpret_cast<const f16x8 *>(Br + (sub + 1) * (RS * PW_BK));
            }
            if constexpr (k == PRE) {
                // every LDS write of the step is issued: the rest of an
                // overflowing fold, then the barrier; the step's last four
                // MFMAs then cover the next step's first operand reads.
                // A(t+1) (loaded into LDS in the step before) must have
                // landed: younger than its loads are this step's weight word
                // loads, (fold) its entry loads and, at a group's first
                // step, its scale loads (more in a rare fold: a longer wait)
                if (rare) fold_rare(u1, h1, Bf);
                constexpr int younger = NJ + (FOLD ? PW_E : 0), ys = younger + NJ;
                if (sload) __builtin_amdgcn_s_waitcnt((ys & 15) | (7 << 4) | (15 << 8) | ((ys >> 4) << 14));
                else __builtin_amdgcn_s_waitcnt((younger & 15) | (7 << 4) | (15 << 8) | ((younger >> 4) << 14));
                __syncthreads();
            }
            // (weights as the first operand: a lane's four results are four
            // adjacent output rows of one token, stored as one 8-byte word)
            if constexpr (XB)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, bcur),
                                                                    __builtin_bit_cast(bf16x8, af[i]), acc[i][j], 0, 0, 0);
            else
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bcur, af[i], acc[i][j], 0, 0, 0);
            if constexpr (k >= PRE) {
                af[i] = *reinterpret_cast<const f16x8 *>(An + 16 * i * PW_BK);
                if constexpr (i == 0) bnext = *reinterpret_cast<const f16x8 *>(Bn);
            } else if constexpr (sub + 1 < KS && j == NRT - 1) {
                // the next sub-step's A operands, into the registers this
                // sub-step's last MFMAs free
                af[i] = *reinterpret_cast<const f16x8 *>(Ast(t & 1) + (sub + 1) * (PW_A_BYTES / 2) + aro + 64 * wm * PW_BK +
                                                         16 * i * PW_BK);
            }

            constexpr int q = pw_dq_at(k, PRE, 4 * NJ);
            if constexpr (q >= 0) {
                // B(t+2): job q / 4, byte pair q % 4 of its word
                constexpr int jb = q / 4, b = q % 4;
                const uint32_t word = rb.v[jb];
                if constexpr (b == 0) {
                    const f16 sc = __builtin_bit_cast(f16, (uint16_t)rb.s[jb]);
                    s2 = f16x2{sc, sc};
                    sf = (float)sc;
                }
                if constexpr (XB) {
                    if constexpr (b == 0) {
                        wlo = (word & 0x0F0F0F0Fu) ^ 0x08080808u;
                        whi = ((word >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
                    }
                    out[b] = pk_bf16(__builtin_fmaf((float)((wlo >> (8 * b)) & 0xFFu), sf, -8.0f * sf),
                                     __builtin_fmaf((float)((whi >> (8 * b)) & 0xFFu), sf, -8.0f * sf));
                } else {
                    out[b] = dq_byte(word, s2, b);
                }
                if constexpr (b == 3)
                    *reinterpret_cast<u32x4 *>(Bw + awo + jb * (PW_NT / JW) * PW_BK) = u32x4{out[0], out[1], out[2], out[3]};
            }
            // A(t+2) into the stage A(t) held (every wave read A(t) before
            // this step's barrier): 2 KS loads in the slots after it
            constexpr int dd = KS == 1 ? ((k == PRE + 1) ? 0 : (k == PRE + 3) ? 1 : -1) : (k >= PRE ? k - PRE : -1);
            if constexpr (dd >= 0) dma_a(min(t + 2, nk - 1), dd, Aw2);
            // B(t+3) loads of job c, in the slot after job c's last byte pair
            constexpr int bl = (k == pw_dq_slot(4 * 0 + 3, PRE, 4 * NJ) + 1)              ? 0
                               : (NJ > 1 && k == pw_dq_slot(4 * 1 + 3, PRE, 4 * NJ) + 1) ? 1
                               : (NJ > 2 && k == pw_dq_slot(4 * 2 + 3, PRE, 4 * NJ) + 1) ? 2
                                                                                          : -1;
            if constexpr (bl >= 0) {
                const int u = u3;
                const uint32_t n = qrow_of(bl);
                rb.v[bl] = __builtin_amdgcn_raw_buffer_load_b32(rq, n * (uint32_t)(a.K >> 1) + qh, u * (PW_BK / 2 * KS), 0);
                if (bl == NJ - 1 && sload) {
                    // the jobs' scales only where step u starts a group (one
                    // uniform branch, after every job of the step has read its
                    // scale): else the registers still hold the scales of step
                    // u - 1's group, the same rows'.  (The loads' issue bounds
                    // the step: without the scale loads a step took 8-11 % less.)
#pragma unroll
                    for (int i = 0; i < NJ; i++)
                        rb.s[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, qrow_of(i) * (uint32_t)(a.ngroups * 2),
                                                                       ((uint32_t)u >> gshift) * 2, 0);
                }
            }
            // the fold late in the step (read, write, then the next step's
            // entries loaded right after): an entry load has nearly a step
            // to land, and it comes from the Infinity Cache or HBM
            constexpr int FR = PRE - 8, FW = PRE - 3, FE = PRE - 2;
            if constexpr (FOLD && k == FR) {
                // fold of B(t+1), prefetched entry: the cell (or the trash cell)
                const uint32_t w = re.e[0];
                const int local = (canonical ? (re.brow[0] & ~1) : -(1 << 20)) + (int)(w >> 24);
                const int c = (int)((w >> 16) & (kPlanBK - 1));
                const bool ok = local >= 0 && local < R && in_half(c, h1);
                fp = reinterpret_cast<uint16_t *>(ok ? cell_at(Bf, local, c) : trash + 2 * tid_now());
                fold_old = *fp;
            }
            if constexpr (FOLD && k == FW)  // (the value recomputed here: one register less across the slots)
                *fp = fold_add<XB>(fold_old, a.alpha * (float)__builtin_bit_cast(f16, (uint16_t)(re.e[0] & 0xffffu)));
            if constexpr (FOLD && k == FE) load_e(pstep(t + 2), re);  // the next step's entries
            __builtin_amdgcn_sched_barrier(0);
        }, std::make_integer_sequence<int, NS>{});
        static_assert(pw_dq_slot(4 * NJ - 1, PRE, 4 * NJ) + 1 < PRE && PRE > 10, "every slice of the step needs a slot");
        b3 = b3_1;
    }

    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // (the last activation loads into LDS land first)

    // epilogue: lane holds D[row 16 j + 4 (lane / 16) + r][token 16 i + lane % 16],
    // four adjacent rows of one token: one 8-byte store where the rows are
    // whole and aligned (N % 4 == 0), else 2-byte stores
    const bool vec = (a.N & 3) == 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + 64 * wm + 16 * i + (lane & 15);
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < NRT; j++) {
            const int64_t n = n0 + (R / 2) * wn + 16 * j + 4 * (lane >> 4);
            uint16_t h[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t nb = min(n + r, a.N - 1);  // (a bias read past the last row is not kept)
                if constexpr (XB) h[r] = out_bf16(acc[i][j][r], a.bias, a.bias_dtype, nb);
                else h[r] = __builtin_bit_cast(uint16_t, out_f16(acc[i][j][r], a.bias, a.bias_dtype, nb));
            }
            uint16_t *yp = reinterpret_cast<uint16_t *>(a.y) + m * a.N + n;
            if (vec && n + 3 < a.N) {
                *reinterpret_cast<uint2 *>(yp) = uint2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (n + r < a.N) yp[r] = h[r];
            }
        }
    }
}

bool prefill_supported(const ForwardArgs &a) {
    if ((a.io_dtype != ORTH_DT_F16 && a.io_dtype != ORTH_DT_BF16) || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.K % PF_BK != 0) return false;
    if (a.ngroups != 1 && (a.G % PF_BK != 0 || ((a.G / PF_BK) & (a.G / PF_BK - 1)) != 0)) return false;
    if (a.has_ortho && !plan_supported(a)) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    // per-lane 32-bit byte offsets into x and q
    if (a.M * a.K * 2 > (int64_t)UINT32_MAX || a.N * (a.K / 2) > (int64_t)UINT32_MAX) return false;
    if (a.N * a.ngroups > (int64_t)UINT32_MAX) return false;
    const int64_t nbm = (a.M + PF_BM - 1) / PF_BM, nbn = (a.N + PF_BN - 1) / PF_BN;
    if (nbm * nbn > ((int64_t)1 << 31) - 1) return false;
    return true;
}

// K split of the 256 x 128 kernel: a grid of tiles that leaves CUs idle
// (c3 at 512 tokens: 64 tiles for 256 CUs) gives each tile S workgroups over
// slices of K, their FP32 sums added in slice order by split_reduce_kernel.
// S minimises a cost measured on MI355X (kernel traces of c3 at 65, 512
// and 1024 tokens and c2 at 65): a round of the grid takes ~12 us (the
// workgroup's latency chain: plan offsets, first loads) plus ~0.95 us per
// 64-column step, and the reduction ~3 us plus its partials at ~6 TB/s;
// the smallest S on a tie.  Slices keep at least 4 steps, and the partials
// fit the no-allocation scratch array, so that both entry points split a
// call alike.
int prefill_ksplit(const ForwardArgs &a, int cus) {
    if (!prefill_supported(a) || cus <= 0) return 1;
    const int64_t tiles = ((a.M + PF_BM - 1) / PF_BM) * ((a.N + PF_BN - 1) / PF_BN);
    const int nk = (int)(a.K / PF_BK);
    auto cost = [&](int s) {
        const int64_t rounds = (tiles * s + cus - 1) / cus;
        const int steps = (nk + s - 1) / s;
        double t = (double)rounds * (12.0 + 0.95 * steps);
        if (s > 1) t += 3.0 + (double)s * a.M * a.N * 4 / 6.0e6;
        return t;
    };
    int best = 1;
    double best_t = cost(1);
    for (int s = 2; s <= 8; s++) {
        if (nk / s < 4 || (int64_t)s * a.M * a.N * 4 > (int64_t)ORTH_NOALLOC_SCRATCH_BYTES) break;
        const double t = cost(s);
        if (t < best_t) best = s, best_t = t;
    }
    return best;
}

hipError_t launch_slice_reduce(const ForwardArgs &a, const float *part, int S, hipStream_t stream);  // orth_split.hip

// part: S * M * N floats when S > 1 (the K split), else unused
hipError_t launch_prefill(const ForwardArgs &a, const void *plan, hipStream_t stream, float *part, int S) {
    PrefillArgs p;
    p.q = a.q;
    p.scales = static_cast<const f16 *>(a.scales);
    p.ngroups = a.ngroups;
    p.G = a.G;
    p.x = static_cast<const f16 *>(a.x);
    p.y = static_cast<f16 *>(a.y);
    p.bias = a.bias;
    p.bias_dtype = a.bias_dtype;
    p.M = a.M;
    p.K = a.K;
    p.N = a.N;
    p.alpha = a.alpha;
    p.nnz = (int32_t)a.nnz;
    p.fold = a.has_ortho && plan != nullptr;
    p.plan = static_cast<const PlanHeader *>(plan);
    p.offsets = plan ? reinterpret_cast<const int32_t *>(static_cast<const char *>(plan) + sizeof(PlanHeader))
                     : nullptr;
    p.entries = plan ? reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(p.offsets) +
                                                          plan_offsets_bytes(a.N, a.K))
                     : nullptr;
    p.nbm = (int)((a.M + PF_BM - 1) / PF_BM);
    p.nbn = (int)((a.N + PF_BN - 1) / PF_BN);
    const unsigned blocks = (unsigned)(p.nbm * p.nbn);
    if (p.fold && p.nnz <= 0) return hipErrorInvalidValue;
    // slices of sps steps, every one non-empty (ny <= S)
    const int nk = (int)(a.K / PF_BK);
    if (S > 1 && !part) return hipErrorInvalidValue;
    p.sps = S > 1 ? (nk + S - 1) / S : nk;
    p.part = S > 1 ? part : nullptr;
    const unsigned ny = (unsigned)((nk + p.sps - 1) / p.sps);
    const bool xb = a.io_dtype == ORTH_DT_BF16;
    const dim3 grid(blocks, ny);
    if (p.fold && xb) hipLaunchKernelGGL((prefill_kernel<true, true>), grid, dim3(PF_NT), PF_LDS_BYTES, stream, p);
    else if (p.fold) hipLaunchKernelGGL((prefill_kernel<true, false>), grid, dim3(PF_NT), PF_LDS_BYTES, stream, p);
    else if (xb) hipLaunchKernelGGL((prefill_kernel<false, true>), grid, dim3(PF_NT), PF_LDS_BYTES, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<false, false>), grid, dim3(PF_NT), PF_LDS_BYTES, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ny == 1) return e;
    return launch_slice_reduce(a, part, (int)ny, stream);
}

// The wide-row tile: rows per workgroup 32 * kPwNrt.  Taken when the layer
// has at least 16 row ranges (every workgroup a full MFMA load of rows);
// layers with fewer rows take 128-row tiles (kPwNrtS) in 64-column steps.
constexpr int kPwNrt = 11, kPwNrtS = 4;
static_assert(pw_lds_bytes(kPwNrt, 1) <= 160 * 1024 && pw_lds_bytes(kPwNrtS, 2) <= 160 * 1024, "wide prefill LDS budget");

bool prefill_wide_supported(const ForwardArgs &a) {
    if (!prefill_supported(a)) return false;
    return a.ngroups == 1 || (a.G % PW_BK == 0 && ((a.G / PW_BK) & (a.G / PW_BK - 1)) == 0);
}

// Wide rows pay where the 256 x 128 tile needs more rounds of the grid than
// the wide tile: 4096 -> 11008 at 2048 tokens, 688 tiles (2.69 rounds)
// against 256 (one).
static bool wide_rows_pay(const ForwardArgs &a, int cus) {
    if (!prefill_wide_supported(a) || a.M < 512 || a.N < 16 * 32 * kPwNrt) return false;
    const int64_t tt = (a.M + PW_BM - 1) / PW_BM;
    const int64_t wide = tt * ((a.N + 32 * kPwNrt - 1) / (32 * kPwNrt));
    const int64_t tiles = ((a.M + PF_BM - 1) / PF_BM) * ((a.N + PF_BN - 1) / PF_BN);
    const double t_wide = (double)((wide + cus - 1) / cus) * (32 * kPwNrt);
    const double t_tile = (double)((tiles + cus - 1) / cus) * PF_BN;
    return t_wide <= t_tile;
}

// The wide kernel's 128-row tile has the 256 x 128 kernel's grid: faster
// from 1024 tokens (c3 at 2048: 78-80 against 83-86 us at alpha = 1; at
// 1536: 73 against 77), level at 1024, 2-4 % slower at 512-768 (c3 70.6
// against 72.2 us at 512, 70.7 against 73.3 at 768).  So the wide kernel
// takes a call where its 352-row tile needs fewer rounds of the grid, or
// from 1024 tokens (the dispatcher asks only for calls that the K split of
// the 256 x 128 kernel does not take: c3 up to 1024 tokens is split).
bool prefill_wide_preferred(const ForwardArgs &a, int cus) {
    return prefill_wide_supported(a) && (wide_rows_pay(a, cus) || a.M >= 1024);
}

hipError_t launch_prefill_wide(const ForwardArgs &a, const void *plan, hipStream_t stream, int cus) {
    PrefillArgs p;
    p.q = a.q;
    p.scales = static_cast<const f16 *>(a.scales);
    p.ngroups = a.ngroups;
    p.G = a.G;
    p.x = static_cast<const f16 *>(a.x);
    p.y = static_cast<f16 *>(a.y);
    p.bias = a.bias;
    p.bias_dtype = a.bias_dtype;
    p.M = a.M;
    p.K = a.K;
    p.N = a.N;
    p.alpha = a.alpha;
    p.nnz = (int32_t)a.nnz;
    p.fold = a.has_ortho && plan != nullptr;
    p.plan = static_cast<const PlanHeader *>(plan);
    p.offsets = plan ? reinterpret_cast<const int32_t *>(static_cast<const char *>(plan) + sizeof(PlanHeader))
                     : nullptr;
    p.entries = plan ? reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(p.offsets) +
                                                          plan_offsets_bytes(a.N, a.K))
                     : nullptr;
    if (p.fold && p.nnz <= 0) return hipErrorInvalidValue;
    const bool xb = a.io_dtype == ORTH_DT_BF16;
    p.nbm = (int)((a.M + PW_BM - 1) / PW_BM);
    auto go = [&](auto nrt, auto ks) {
        constexpr int NRT = decltype(nrt)::value, KS = decltype(ks)::value;
        p.nbn = (int)((a.N + 32 * NRT - 1) / (32 * NRT));
        const unsigned blocks = (unsigned)(p.nbm * p.nbn);
        const int lds = pw_lds_bytes(NRT, KS);
        if (p.fold && xb) hipLaunchKernelGGL((prefill_wide_kernel<NRT, KS, true, true>), dim3(blocks), dim3(PW_NT), lds, stream, p);
        else if (p.fold) hipLaunchKernelGGL((prefill_wide_kernel<NRT, KS, true, false>), dim3(blocks), dim3(PW_NT), lds, stream, p);
        else if (xb) hipLaunchKernelGGL((prefill_wide_kernel<NRT, KS, false, true>), dim3(blocks), dim3(PW_NT), lds, stream, p);
        else hipLaunchKernelGGL((prefill_wide_kernel<NRT, KS, false, false>), dim3(blocks), dim3(PW_NT), lds, stream, p);
    };
    if (wide_rows_pay(a, cus)) go(std::integral_constant<int, kPwNrt>{}, std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, kPwNrtS>{}, std::integral_constant<int, 2>{});
    return hipGetLastError();
}

}  // namespace orth

namespace orth {

// Kernels that use more than 64 KB of dynamic LDS must say so per device.
hipError_t prefill_prepare_device() {
    const void *ks[4] = {reinterpret_cast<const void *>(prefill_kernel<true, false>),
                         reinterpret_cast<const void *>(prefill_kernel<false, false>),
                         reinterpret_cast<const void *>(prefill_kernel<true, true>),
                         reinterpret_cast<const void *>(prefill_kernel<false, true>)};
    for (const void *k : ks) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS_BYTES);
        if (e != hipSuccess) return e;
    }
    const void *kw[4] = {reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrt, 1, true, false>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrt, 1, false, false>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrt, 1, true, true>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrt, 1, false, true>)};
    for (const void *k : kw) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, pw_lds_bytes(kPwNrt, 1));
        if (e != hipSuccess) return e;
    }
    const void *kn[4] = {reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrtS, 2, true, false>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrtS, 2, false, false>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrtS, 2, true, true>),
                         reinterpret_cast<const void *>(prefill_wide_kernel<kPwNrtS, 2, false, true>)};
    for (const void *k : kn) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, pw_lds_bytes(kPwNrtS, 2));
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t plan_prepare_device() {
    const int bytes = (int)(((kPlanMaxK / kPlanBK) * kPlanBN + 256) * sizeof(int32_t));
    return hipFuncSetAttribute(reinterpret_cast<const void *>(plan_build_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

}  // namespace orth
