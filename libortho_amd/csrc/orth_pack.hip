// Packing on the device: the load-time steps in front of the dual GEMM.
//
//  * Base: /root/reference/torch_bind/ortho_linear.py:89-120 — per-row (or
//    per-group) scales max|W| / 7 clamped at 1e-6, q = clamp(round(W / s),
//    -8, 7) with the scales as computed (not their FP16 copy), nibble pairs
//    of the flattened [N, K] array packed low = even index.
//  * Ortho: /root/reference/tools/sieve.py:119-152 — the entries W != 0 in
//    row-major order (columns ascending within a row), row_ptr = [0,
//    cumsum(row counts)].
//
// The arithmetic is what torch does for those ops on a GPU tensor:
//  * max|W| / 7.0 divides by a CPU scalar, which torch computes as a
//    multiplication by the FP32 reciprocal fp32(1/7) (in FP32 for FP16 and
//    BF16 tensors too), rounded to W's dtype; clamp(min=1e-6) compares with
//    1e-6 rounded to W's dtype.  NaN propagates through max and clamp.
//  * W / s is an IEEE division in FP32 rounded to the promoted dtype of W
//    and s (W's own when the scales were computed here; FP32 when given
//    scales of another dtype), then round-half-to-even and the clamp.
//  * The FP16 scales stored are the scales rounded to nearest even.
//
// Bandwidth: every kernel reads W once from HBM (the per-row kernel keeps
// the row in registers between its two passes) and writes q, the scales or
// the CSR arrays once.  The CSR is built in three launches: per-row counts
// (which also record each element's nonzero bit in a mask when the caller
// gives one), one scan, and a fill that reads the mask and only the nonzero
// elements of W (without a mask it reads W again); the counts place each
// row's entries, and the host reads row_ptr[N] between the first two and
// the fill to size the outputs.
#include "orth_common.h"

namespace orth {

namespace {

constexpr int kPackNT = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ float round_to(int dt, float v) { return round_as(dt, v); }

// |v| as bits: for non-negative floats the integer order is the float order,
// and NaN patterns sort above +inf, so a max over these bits propagates NaN
__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off));
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int DT> struct Elem;
template <> struct Elem<ORTH_DT_F32> {
    static constexpr int kSize = 4;
    __device__ static float get(const uint32_t *wd, int i) { return __uint_as_float(wd[i]); }
    __device__ static bool nonzero(const uint32_t *wd, int i) { return (wd[i] & 0x7fffffffu) != 0u; }
    __device__ static uint32_t bits(const uint32_t *wd, int i) { return wd[i]; }
};
template <> struct Elem<ORTH_DT_F16> {
    static constexpr int kSize = 2;
    __device__ static uint32_t bits(const uint32_t *wd, int i) { return (wd[i >> 1] >> (16 * (i & 1))) & 0xffffu; }
    __device__ static float get(const uint32_t *wd, int i) { return (float)__builtin_bit_cast(f16, (uint16_t)bits(wd, i)); }
    __device__ static bool nonzero(const uint32_t *wd, int i) { return (bits(wd, i) & 0x7fffu) != 0u; }
};
template <> struct Elem<ORTH_DT_BF16> {
    static constexpr int kSize = 2;
    __device__ static uint32_t bits(const uint32_t *wd, int i) { return (wd[i >> 1] >> (16 * (i & 1))) & 0xffffu; }
    __device__ static float get(const uint32_t *wd, int i) { return bf16_bits_to_f32((uint16_t)bits(wd, i)); }
    __device__ static bool nonzero(const uint32_t *wd, int i) { return (bits(wd, i) & 0x7fffu) != 0u; }
};

// NW consecutive 32-bit words from p (aligned to 4 * the largest piece used)
template <int NW>
__device__ __forceinline__ void load_words(const uint32_t *p, uint32_t *out) {
    if constexpr (NW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 4; i++) {
            const u32x4 v = reinterpret_cast<const u32x4 *>(p)[i];
            out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
        }
    } else if constexpr (NW % 2 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 2; i++) {
            const uint2 v = reinterpret_cast<const uint2 *>(p)[i];
            out[2 * i] = v.x; out[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NW; i++) out[i] = p[i];
    }
}

}  // namespace

struct PackBaseArgs {
    const void *w;
    int wdt;
    int64_t N, K, G, ng;
    const void *s_in;  // given scales [N * ng], or null
    int sdt;
    uint8_t *q;        // [N, K/2]
    f16 *s_out;        // [N * ng]
};

namespace {

// the scale of cell si from the absmax bits of its elements (or the given scale)
__device__ __forceinline__ float scale_of(const PackBaseArgs &a, int64_t si, uint32_t mbits) {
    if (a.s_in) return load_as_f32(a.s_in, a.sdt, si);
    const float m = __uint_as_float(mbits);
    const float s = round_to(a.wdt, m * (1.0f / 7.0f));
    const float lo = round_to(a.wdt, 1e-6f);
    return s < lo ? lo : s;  // (NaN stays NaN)
}

__device__ __forceinline__ uint32_t quant_nibble(int prom, float w, float s) {
    float v = rintf(round_to(prom, w / s));
    v = v < -8.f ? -8.f : (v > 7.f ? 7.f : v);
    return (uint32_t)(int)v & 15u;
}

__device__ __forceinline__ int prom_dtype(const PackBaseArgs &a) {
    return (a.s_in && a.sdt != a.wdt) ? ORTH_DT_F32 : a.wdt;
}

// Per-group scales, G = EPL * LPG in 128 .. 2048: LPG consecutive lanes
// take one (row, group) cell, lane holding EPL consecutive elements in
// registers (one pass over W); a wave takes 64 / LPG cells per step and
// STEPS steps, their loads issued together.
template <int EPL, int LPG, int DT>
__global__ void __launch_bounds__(kPackNT) pack_group_kernel(PackBaseArgs a) {
    using E = Elem<DT>;
    constexpr int NW = EPL * E::kSize / 4;  // words of W per lane per step
    constexpr int CPS = 64 / LPG;           // cells per wave per step
    constexpr int STEPS = 32 / EPL;         // 4, 2 or 1
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPG;
    const int64_t total = a.N * a.ng;
    const int64_t wave = (int64_t)blockIdx.x * (kPackNT / 64) + (threadIdx.x >> 6);
    const int64_t cell0 = wave * (CPS * STEPS) + lane / LPG;
    uint32_t wd[STEPS][NW];
#pragma unroll
    for (int st = 0; st < STEPS; st++) {
        const int64_t cell = min(cell0 + st * CPS, total - 1);  // (clamped; stores masked)
        const int64_t e0 = cell * (EPL * LPG) + sub * EPL;     // cell * G = n * K + g * G
        load_words<NW>(reinterpret_cast<const uint32_t *>(static_cast<const char *>(a.w) + e0 * E::kSize), wd[st]);
    }
    const int prom = prom_dtype(a);
#pragma unroll
    for (int st = 0; st < STEPS; st++) {
        const int64_t cell = cell0 + st * CPS;
        const bool ok = cell < total;
        uint32_t mb = 0u;
        if (!a.s_in) {
#pragma unroll
            for (int i = 0; i < EPL; i++) mb = max(mb, abs_bits(E::get(wd[st], i)));
#pragma unroll
            for (int off = LPG / 2; off > 0; off >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off));
        }
        const float s = scale_of(a, ok ? cell : 0, mb);
        if (ok && sub == 0) a.s_out[cell] = (f16)s;
        uint32_t qb[EPL / 8];
#pragma unroll
        for (int j = 0; j < EPL / 8; j++) qb[j] = 0u;
#pragma unroll
        for (int i = 0; i < EPL; i++) qb[i / 8] |= quant_nibble(prom, E::get(wd[st], i), s) << (4 * (i % 8));
        if (ok) {
            uint8_t *dst = a.q + (cell * (EPL * LPG) + sub * EPL) / 2;
            if constexpr (EPL == 8) {
                *reinterpret_cast<uint32_t *>(dst) = qb[0];
            } else if constexpr (EPL == 16) {
                *reinterpret_cast<uint2 *>(dst) = uint2{qb[0], qb[1]};
            } else {
                *reinterpret_cast<u32x4 *>(dst) = u32x4{qb[0], qb[1], qb[2], qb[3]};
            }
        }
    }
}

// One workgroup per row with one scale per row (G == K): thread t holds the
// element pairs t + 256 i (i < PPT) in registers; block max, then q.
template <int PPT, int DT>
__global__ void __launch_bounds__(kPackNT) pack_row_kernel(PackBaseArgs a) {
    using E = Elem<DT>;
    constexpr int NW = 2 * E::kSize / 4;  // words per pair: 2 (F32) or 1
    __shared__ uint32_t wmax[kPackNT / 64];
    const int64_t n = blockIdx.x;
    const int t = threadIdx.x;
    const int64_t npairs = a.K / 2;
    const char *row = static_cast<const char *>(a.w) + n * a.K * E::kSize;
    uint32_t wd[PPT][NW];
#pragma unroll
    for (int i = 0; i < PPT; i++) {
        const int64_t p = min((int64_t)t + kPackNT * i, npairs - 1);  // (clamped; masked below)
        load_words<NW>(reinterpret_cast<const uint32_t *>(row + p * 2 * E::kSize), wd[i]);
    }
    uint32_t mb = 0u;
    if (!a.s_in) {
#pragma unroll
        for (int i = 0; i < PPT; i++)
            if ((int64_t)t + kPackNT * i < npairs)
                mb = max(mb, max(abs_bits(E::get(wd[i], 0)), abs_bits(E::get(wd[i], 1))));
        mb = wave_max_u32(mb);
        if ((t & 63) == 0) wmax[t >> 6] = mb;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kPackNT / 64; w++) mb = max(mb, wmax[w]);
    }
    const float s = scale_of(a, n, mb);
    if (t == 0) a.s_out[n] = (f16)s;
    const int prom = prom_dtype(a);
    uint8_t *dst = a.q + n * npairs;
#pragma unroll
    for (int i = 0; i < PPT; i++) {
        const int64_t p = (int64_t)t + kPackNT * i;
        if (p < npairs)
            dst[p] = (uint8_t)(quant_nibble(prom, E::get(wd[i], 0), s) | (quant_nibble(prom, E::get(wd[i], 1), s) << 4));
    }
}

// Any even G dividing K: one thread per (row, group) cell, two passes over
// the cell (the second from cache).
__global__ void __launch_bounds__(kPackNT) pack_generic_kernel(PackBaseArgs a) {
    const int64_t cell = (int64_t)blockIdx.x * kPackNT + threadIdx.x;
    if (cell >= a.N * a.ng) return;
    const int64_t e0 = cell * a.G;
    uint32_t mb = 0u;
    if (!a.s_in)
        for (int64_t k = 0; k < a.G; k++) mb = max(mb, abs_bits(load_as_f32(a.w, a.wdt, e0 + k)));
    const float s = scale_of(a, cell, mb);
    a.s_out[cell] = (f16)s;
    const int prom = prom_dtype(a);
    for (int64_t k = 0; k < a.G; k += 2)
        a.q[(e0 + k) / 2] = (uint8_t)(quant_nibble(prom, load_as_f32(a.w, a.wdt, e0 + k), s) |
                                      (quant_nibble(prom, load_as_f32(a.w, a.wdt, e0 + k + 1), s) << 4));
}

// ---- CSR

// words of the nonzero mask of one row: 8 per step of 256 elements
__host__ __device__ inline int64_t csr_mask_words(int64_t K) { return (K + 255) / 256 * 8; }

// row_ptr[n + 1] = nonzeros of row n (one wave per row); row_ptr[0] = 0.
// V elements per lane per step (vector loads when V > 1).
template <int DT, int V>
__global__ void __launch_bounds__(kPackNT) csr_count_kernel(const void *w, int64_t N, int64_t K, int32_t *row_ptr,
                                                            uint32_t *mask) {
    using E = Elem<DT>;
    constexpr int NW = V * E::kSize / 4 > 0 ? V * E::kSize / 4 : 1;
    const int64_t n = (int64_t)blockIdx.x * (kPackNT / 64) + (threadIdx.x >> 6);
    if (n >= N) return;
    const int lane = threadIdx.x & 63;
    const char *row = static_cast<const char *>(w) + n * K * E::kSize;
    int cnt = 0;
    if constexpr (V == 1) {
        for (int64_t k = lane; k < K; k += 64) {
            const uint32_t wd[1] = {DT == ORTH_DT_F32 ? reinterpret_cast<const uint32_t *>(row)[k]
                                                     : (uint32_t)reinterpret_cast<const uint16_t *>(row)[k]};
            cnt += E::nonzero(wd, 0) ? 1 : 0;
        }
    } else {
        // U steps of 64 * V elements, their loads issued together (addresses
        // clamped into the row, elements past it not counted).  With a mask
        // (V == 4) each step's nonzero pattern is kept, lane l's 4 bits at
        // bits 4 (l % 8) of word l / 8 of the step's 8 words.
        constexpr int U = 4;
        uint32_t *mrow = mask ? mask + n * csr_mask_words(K) : nullptr;
        for (int64_t kb = 0; kb < K; kb += 64 * V * U) {
            uint32_t wd[U][NW];
#pragma unroll
            for (int u = 0; u < U; u++)
                load_words<NW>(reinterpret_cast<const uint32_t *>(
                                   row + min(kb + 64 * V * u + (int64_t)lane * V, K - V) * E::kSize), wd[u]);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int64_t k = kb + 64 * V * u + (int64_t)lane * V;
                uint32_t nib = 0u;
#pragma unroll
                for (int j = 0; j < V; j++) nib |= (k + j < K && E::nonzero(wd[u], j)) ? (1u << j) : 0u;
                cnt += __builtin_popcount(nib);
                if (V == 4 && mrow) {  // (uniform)
                    uint32_t m = nib << (4 * (lane & 7));
                    m |= (uint32_t)__shfl_xor((int)m, 1);
                    m |= (uint32_t)__shfl_xor((int)m, 2);
                    m |= (uint32_t)__shfl_xor((int)m, 4);
                    const int64_t st = kb / (64 * V) + u;
                    if ((lane & 7) == 0 && st * 64 * V < K) mrow[st * 8 + (lane >> 3)] = m;
                }
            }
        }
    }
    cnt = wave_sum_i32(cnt);
    if (lane == 0) {
        row_ptr[n + 1] = cnt;
        if (n == 0) row_ptr[0] = 0;
    }
}

constexpr int kScanPer = 16;

// In-place inclusive scan of row_ptr[1 .. N] by one workgroup of 1024
// threads, kScanPer consecutive counts per thread per pass (one pass up
// to 16,384 rows): thread sums, a wave
// scan with lane shuffles, the 16 wave totals scanned through LDS.  A
// running total past 2^31 - 1 stores -1 from there on.
__global__ void __launch_bounds__(1024) csr_scan_kernel(int32_t *row_ptr, int64_t N) {
    __shared__ int64_t wsum[16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    int64_t carry = 0;
    for (int64_t base = 0; base < N; base += kScanPer * 1024) {
        const int64_t i0 = base + kScanPer * (int64_t)t;
        int64_t v[kScanPer];
        int64_t tsum = 0;
#pragma unroll
        for (int j = 0; j < kScanPer; j++) {
            v[j] = i0 + j < N ? (int64_t)row_ptr[i0 + j + 1] : 0;
            tsum += v[j];
            v[j] = tsum;  // inclusive within the thread
        }
        int64_t incl = tsum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int64_t up = __shfl_up(incl, off);
            if (lane >= off) incl += up;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int64_t before = carry, all = carry;
        for (int w = 0; w < 16; w++) {
            if (w < wave) before += wsum[w];
            all += wsum[w];
        }
        before += incl - tsum;  // lanes before this one in the wave
#pragma unroll
        for (int j = 0; j < kScanPer; j++) {
            if (i0 + j < N) {
                const int64_t tot = before + v[j];
                row_ptr[i0 + j + 1] = (carry < 0 || tot > 0x7fffffffLL) ? -1 : (int32_t)tot;
            }
        }
        __syncthreads();  // wsum is rewritten by the next pass
        carry = (carry < 0 || all > 0x7fffffffLL) ? -1 : all;
    }
}

// Writes row n's entries at row_ptr[n] .. (one wave per row): per step each
// lane takes V consecutive elements, the wave's exclusive prefix of the
// lanes' counts places them in column order.
template <int DT, int V>
__global__ void __launch_bounds__(kPackNT) csr_fill_kernel(const void *w, int64_t N, int64_t K,
                                                           const int32_t *row_ptr, const uint32_t *mask,
                                                           int32_t *col, void *vals, int vdt) {
    using E = Elem<DT>;
    constexpr int NW = V * E::kSize / 4 > 0 ? V * E::kSize / 4 : 1;
    const int64_t n = (int64_t)blockIdx.x * (kPackNT / 64) + (threadIdx.x >> 6);
    if (n >= N) return;
    const int lane = threadIdx.x & 63;
    const char *row = static_cast<const char *>(w) + n * K * E::kSize;
    int64_t pos = row_ptr[n];
    const int64_t end = row_ptr[n + 1];
    constexpr int U = 4;
    auto store_entry = [&](int64_t at, int64_t k, uint32_t bits) {
        col[at] = (int32_t)k;
        if (vdt == DT) {
            if (DT == ORTH_DT_F32) static_cast<uint32_t *>(vals)[at] = bits;
            else static_cast<uint16_t *>(vals)[at] = (uint16_t)bits;
        } else {
            const uint32_t one[1] = {bits};
            store_from_f32(vals, vdt, at, DT == ORTH_DT_F32 ? __uint_as_float(bits) : E::get(one, 0));
        }
    };
    if (V == 4 && mask) {
        // with the count pass's mask: only the elements it marked are read
        const uint32_t *mrow = mask + n * csr_mask_words(K);
        const int64_t nst = (K + 64 * V - 1) / (64 * V);
        for (int64_t s0 = 0; s0 < nst; s0 += U) {
            uint32_t nib[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t m = mrow[min(s0 + u, nst - 1) * 8 + (lane >> 3)];
                nib[u] = s0 + u < nst ? (m >> (4 * (lane & 7))) & 15u : 0u;
            }
            uint32_t vb[U][V];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int64_t k = (s0 + u) * 64 * V + (int64_t)lane * V;
#pragma unroll
                for (int j = 0; j < V; j++) {
                    vb[u][j] = 0u;
                    if ((nib[u] >> j) & 1u)
                        vb[u][j] = DT == ORTH_DT_F32 ? reinterpret_cast<const uint32_t *>(row)[k + j]
                                                    : (uint32_t)reinterpret_cast<const uint16_t *>(row)[k + j];
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int64_t k = (s0 + u) * 64 * V + (int64_t)lane * V;
                const int cnt = __builtin_popcount(nib[u]);
                int incl = cnt;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const int up = __shfl_up(incl, off);
                    if (lane >= off) incl += up;
                }
                int64_t at = pos + incl - cnt;
#pragma unroll
                for (int j = 0; j < V; j++) {
                    if (((nib[u] >> j) & 1u) && at < end) {
                        store_entry(at, k + j, vb[u][j]);
                        at++;
                    }
                }
                pos += __shfl(incl, 63);
            }
        }
        return;
    }
    // U steps' loads issued together (addresses clamped into the row)
    for (int64_t kb = 0; kb < K; kb += 64 * V * U) {
        uint32_t wd[U][NW];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t k = min(kb + 64 * V * u + (int64_t)lane * V, K - V);
            if constexpr (V == 1)
                wd[u][0] = DT == ORTH_DT_F32 ? reinterpret_cast<const uint32_t *>(row)[k]
                                             : (uint32_t)reinterpret_cast<const uint16_t *>(row)[k];
            else
                load_words<NW>(reinterpret_cast<const uint32_t *>(row + k * E::kSize), wd[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t k = kb + 64 * V * u + (int64_t)lane * V;
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < V; j++) cnt += (k + j < K && E::nonzero(wd[u], j)) ? 1 : 0;
            int incl = cnt;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int up = __shfl_up(incl, off);
                if (lane >= off) incl += up;
            }
            int64_t at = pos + incl - cnt;
#pragma unroll
            for (int j = 0; j < V; j++) {
                if (k + j < K && E::nonzero(wd[u], j) && at < end) {
                    store_entry(at, k + j, E::bits(wd[u], j));
                    at++;
                }
            }
            pos += __shfl(incl, 63);
        }
    }
}

template <int EPL, int LPG>
hipError_t launch_group(const PackBaseArgs &a, hipStream_t s) {
    const int64_t per_block = (kPackNT / 64) * (64 / LPG) * (32 / EPL);
    const unsigned blocks = (unsigned)((a.N * a.ng + per_block - 1) / per_block);
    if (a.wdt == ORTH_DT_F32) hipLaunchKernelGGL((pack_group_kernel<EPL, LPG, ORTH_DT_F32>), dim3(blocks), dim3(kPackNT), 0, s, a);
    else if (a.wdt == ORTH_DT_F16) hipLaunchKernelGGL((pack_group_kernel<EPL, LPG, ORTH_DT_F16>), dim3(blocks), dim3(kPackNT), 0, s, a);
    else hipLaunchKernelGGL((pack_group_kernel<EPL, LPG, ORTH_DT_BF16>), dim3(blocks), dim3(kPackNT), 0, s, a);
    return hipGetLastError();
}

template <int PPT>
hipError_t launch_row(const PackBaseArgs &a, hipStream_t s) {
    const unsigned blocks = (unsigned)a.N;
    if (a.wdt == ORTH_DT_F32) hipLaunchKernelGGL((pack_row_kernel<PPT, ORTH_DT_F32>), dim3(blocks), dim3(kPackNT), 0, s, a);
    else if (a.wdt == ORTH_DT_F16) hipLaunchKernelGGL((pack_row_kernel<PPT, ORTH_DT_F16>), dim3(blocks), dim3(kPackNT), 0, s, a);
    else hipLaunchKernelGGL((pack_row_kernel<PPT, ORTH_DT_BF16>), dim3(blocks), dim3(kPackNT), 0, s, a);
    return hipGetLastError();
}

int dt_size(int dt) { return dt == ORTH_DT_F32 ? 4 : 2; }

}  // namespace

// Which base kernel a call takes: 1 per-group waves, 2 per-row workgroups,
// 3 the per-cell fallback.
int pack_base_path(const void *w, int wdt, int64_t K, int64_t G, const void *q) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(w);
    if ((G == 128 || G == 256 || G == 512 || G == 1024 || G == 2048) && (p % 16) == 0 &&
        (reinterpret_cast<uintptr_t>(q) % 16) == 0)
        return 1;
    if (G == K && K / 2 <= 32 * kPackNT && (p % 8) == 0) return 2;
    return 3;
}

hipError_t launch_pack_base(const void *w, int wdt, int64_t N, int64_t K, int64_t G, const void *s_in,
                            int sdt, uint8_t *q, void *s_out, hipStream_t stream) {
    PackBaseArgs a{w, wdt, N, K, G, K / G, s_in, sdt, q, static_cast<f16 *>(s_out)};
    switch (pack_base_path(w, wdt, K, G, q)) {
        case 1:
            switch (G) {
                case 128: return launch_group<8, 16>(a, stream);
                case 256: return launch_group<8, 32>(a, stream);
                case 512: return launch_group<8, 64>(a, stream);
                case 1024: return launch_group<16, 64>(a, stream);
                default: return launch_group<32, 64>(a, stream);
            }
        case 2: {
            const int64_t ppt = (K / 2 + kPackNT - 1) / kPackNT;
            if (ppt <= 4) return launch_row<4>(a, stream);
            if (ppt <= 8) return launch_row<8>(a, stream);
            if (ppt <= 16) return launch_row<16>(a, stream);
            return launch_row<32>(a, stream);
        }
        default: {
            const unsigned blocks = (unsigned)((N * (K / G) + kPackNT - 1) / kPackNT);
            hipLaunchKernelGGL(pack_generic_kernel, dim3(blocks), dim3(kPackNT), 0, stream, a);
            return hipGetLastError();
        }
    }
}

namespace {
// elements per lane per step of the CSR kernels: 4 with 16-byte (F32) or
// 8-byte (16-bit) aligned rows, else 1
int csr_vec(const void *w, int wdt, int64_t K) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(w);
    return (K % 4 == 0 && p % (4 * dt_size(wdt)) == 0) ? 4 : 1;
}
}  // namespace

int64_t csr_mask_bytes(const void *w, int wdt, int64_t N, int64_t K) {
    return csr_vec(w, wdt, K) == 4 ? N * csr_mask_words(K) * 4 : 0;
}

hipError_t launch_csr_rows(const void *w, int wdt, int64_t N, int64_t K, int32_t *row_ptr, void *mask_v,
                           hipStream_t stream) {
    const unsigned blocks = (unsigned)((N + 3) / 4);
    const bool v4 = csr_vec(w, wdt, K) == 4;
    uint32_t *mask = static_cast<uint32_t *>(mask_v);
#define ORTH_COUNT(DT, V) hipLaunchKernelGGL((csr_count_kernel<DT, V>), dim3(blocks), dim3(kPackNT), 0, stream, w, N, K, row_ptr, mask)
    if (wdt == ORTH_DT_F32) { if (v4) ORTH_COUNT(ORTH_DT_F32, 4); else ORTH_COUNT(ORTH_DT_F32, 1); }
    else if (wdt == ORTH_DT_F16) { if (v4) ORTH_COUNT(ORTH_DT_F16, 4); else ORTH_COUNT(ORTH_DT_F16, 1); }
    else { if (v4) ORTH_COUNT(ORTH_DT_BF16, 4); else ORTH_COUNT(ORTH_DT_BF16, 1); }
#undef ORTH_COUNT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, stream, row_ptr, N);
    return hipGetLastError();
}

hipError_t launch_csr_fill(const void *w, int wdt, int64_t N, int64_t K, const int32_t *row_ptr,
                           const void *mask_v, int32_t *col, void *vals, int vdt, hipStream_t stream) {
    const unsigned blocks = (unsigned)((N + 3) / 4);
    const bool v4 = csr_vec(w, wdt, K) == 4;
    const uint32_t *mask = static_cast<const uint32_t *>(mask_v);
#define ORTH_FILL(DT, V) hipLaunchKernelGGL((csr_fill_kernel<DT, V>), dim3(blocks), dim3(kPackNT), 0, stream, w, N, K, row_ptr, mask, col, vals, vdt)
    if (wdt == ORTH_DT_F32) { if (v4) ORTH_FILL(ORTH_DT_F32, 4); else ORTH_FILL(ORTH_DT_F32, 1); }
    else if (wdt == ORTH_DT_F16) { if (v4) ORTH_FILL(ORTH_DT_F16, 4); else ORTH_FILL(ORTH_DT_F16, 1); }
    else { if (v4) ORTH_FILL(ORTH_DT_BF16, 4); else ORTH_FILL(ORTH_DT_BF16, 1); }
#undef ORTH_FILL
    return hipGetLastError();
}

}  // namespace orth
