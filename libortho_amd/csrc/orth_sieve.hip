// The offline Base/Ortho sieve on the device: what /root/reference/tools/sieve.py:13-95
// computes with torch ops, as four small kernels with the arithmetic of
// those ops on a GPU tensor (so that the results carry the same bits).
//
//  quantize_int4 (:13-23)   one workgroup per row: max|w| (NaN propagates),
//                            clamp at 1e-8 in w's dtype, s = max * fp32(1/7)
//                            (torch divides a GPU tensor by a host scalar
//                            through its reciprocal; a CPU tensor by IEEE
//                            division, the ieee_div mode), q = clamp(rint(w / s), -8, 7),
//                            w_base = q * s, non-finite results 0.  Every
//                            intermediate is rounded to w's dtype, as the
//                            torch ops round each result.
//  hessian_sieve (:25-76)   the same pass also writes the residual w - w_base
//                            and the score residual^2 / (H_inv + 1e-6); with a
//                            sparsity target, the k-th largest score is found by
//                            a radix select over the order-preserving key of
//                            each FP32 score (NaN largest, as torch.topk),
//                            8 bits per pass; then w_ortho = residual * (score > t).
//  compute_hessian_diag_approx (:79-95)  diag(X^T X) / n + 1e-6: the
//                            diagonal only (column sums of squares, FP32
//                            partial sums over row slices added in slice
//                            order), not the K x K product.
//
// Off the forward path: these run once per weight matrix when a model is
// split, and are measured as load-time work.
#include "orth_common.h"

namespace orth {

constexpr int kSieveNT = 256;

__device__ __forceinline__ float sieve_max_nan(float a, float b) {
    // torch's max propagates NaN
    return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

// Order-preserving key of an FP32 value, NaN above everything (the key
// torch.topk selects on).
__device__ __forceinline__ uint32_t sieve_key(float f) {
    const uint32_t x = __float_as_uint(f);
    if (f != f) return 0xffffffffu;
    return x ^ ((x & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}

__device__ __forceinline__ float sieve_unkey(uint32_t k) {
    if (k == 0xffffffffu) return __builtin_nanf("");
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

struct SieveArgs {
    const void *w;
    int dt;
    int64_t N, K;
    void *w_base;
    void *resid;        // w_ortho buffer: the residual, masked later (or null)
    float *score;       // [N*K] score values (exact in FP32), or null
    const void *h;      // H_inv: element k at h[k * h_stride]
    int hdt;
    int64_t h_stride;
    int score_dt;       // dtype of the score (torch's promotion of w's and H's)
    int ieee_div;       // 1: division by a host scalar as IEEE division (CPU
                        // tensors), 0: as a product with its FP32 reciprocal
};

// v / d for a host scalar d, as torch computes it on the tensor's device.
__device__ __forceinline__ float sieve_scalar_div(float v, float d, int ieee_div) {
    return ieee_div ? v / d : v * (1.0f / d);
}

__global__ void __launch_bounds__(kSieveNT) sieve_quant_kernel(SieveArgs a) {
    __shared__ float red[kSieveNT / 64];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t base = r * a.K;
    float m = 0.f;
    for (int64_t k = tid; k < a.K; k += kSieveNT) m = sieve_max_nan(m, fabsf(load_as_f32(a.w, a.dt, base + k)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = sieve_max_nan(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < kSieveNT / 64; i++) m = sieve_max_nan(m, red[i]);
    // clamp(min=1e-8): the bound in w's dtype (0 in FP16), NaN kept
    const float lo = round_as(a.dt, 1e-8f);
    const float mc = (m != m) ? m : fmaxf(m, lo);
    const float s = round_as(a.dt, sieve_scalar_div(mc, 7.0f, a.ieee_div));
    for (int64_t k = tid; k < a.K; k += kSieveNT) {
        const float wv = load_as_f32(a.w, a.dt, base + k);
        float t = rintf(round_as(a.dt, wv / s));
        t = (t != t) ? t : fminf(fmaxf(t, -8.f), 7.f);
        float wb = round_as(a.dt, t * s);
        if (!__builtin_isfinite(wb)) wb = 0.f;
        store_from_f32(a.w_base, a.dt, base + k, wb);
        if (a.resid) {
            const float rr = round_as(a.dt, wv - wb);
            store_from_f32(a.resid, a.dt, base + k, rr);
            const float r2 = round_as(a.dt, rr * rr);
            const float hs = round_as(a.hdt, load_as_f32(a.h, a.hdt, k * a.h_stride) + 1e-6f);
            a.score[base + k] = round_as(a.score_dt, r2 / hs);
        }
    }
}

// Radix-select state: the key prefix found so far, its mask, the rank still
// sought within the prefix (1 = largest), and the histogram of the pass.
struct SieveSel {
    uint32_t prefix, mask, k, pad;
    uint32_t hist[256];
};

__global__ void sieve_sel_init_kernel(SieveSel *st, uint32_t k) {
    const int t = threadIdx.x;
    st->hist[t] = 0;
    if (t == 0) {
        st->prefix = 0;
        st->mask = 0;
        st->k = k;
        st->pad = 0;
    }
}

__global__ void __launch_bounds__(kSieveNT) sieve_hist_kernel(const float *score, int64_t n, SieveSel *st,
                                                              int shift) {
    __shared__ uint32_t h[256];
    const int tid = threadIdx.x;
    h[tid] = 0;
    __syncthreads();
    const uint32_t prefix = st->prefix, mask = st->mask;
    for (int64_t i = (int64_t)blockIdx.x * kSieveNT + tid; i < n; i += (int64_t)gridDim.x * kSieveNT) {
        const uint32_t key = sieve_key(score[i]);
        if ((key & mask) == prefix) atomicAdd(&h[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (h[tid]) atomicAdd(&st->hist[tid], h[tid]);
}

// One thread: the bin (from the top) that holds the k-th largest key; the
// histogram is cleared for the next pass.
__global__ void sieve_pick_kernel(SieveSel *st, int shift) {
    if (threadIdx.x == 0) {
        uint32_t k = st->k;
        for (int b = 255; b >= 0; b--) {
            const uint32_t c = st->hist[b];
            if (k <= c) {
                st->prefix |= (uint32_t)b << shift;
                st->mask |= 255u << shift;
                break;
            }
            k -= c;
        }
        st->k = k;
    }
    __syncthreads();
    st->hist[threadIdx.x] = 0;
}

// w_ortho = residual * (score > t): t the selected k-th largest score
// (from_sel) or the caller's threshold rounded to the score's dtype (torch
// compares a tensor with a host scalar in the tensor's dtype); NaN compares
// false.
__global__ void __launch_bounds__(kSieveNT) sieve_mask_kernel(void *resid, int dt, const float *score, int64_t n,
                                                              const SieveSel *st, int from_sel, float thresh,
                                                              int score_dt) {
    const float t = from_sel ? sieve_unkey(st->prefix) : round_as(score_dt, thresh);
    for (int64_t i = (int64_t)blockIdx.x * kSieveNT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kSieveNT) {
        const float r = load_as_f32(resid, dt, i);
        store_from_f32(resid, dt, i, round_as(dt, r * (score[i] > t ? 1.f : 0.f)));
    }
}

// Column sums of squares of x [n, K] over row slice blockIdx.y (slices of
// `rows` rows), in FP32: partial[y][k].
__global__ void __launch_bounds__(kSieveNT) sieve_hdiag_partial_kernel(const void *x, int dt, int64_t n, int64_t K,
                                                                       int64_t rows, float *partial) {
    const int64_t k = (int64_t)blockIdx.x * kSieveNT + threadIdx.x;
    if (k >= K) return;
    const int64_t r0 = (int64_t)blockIdx.y * rows, r1 = min(n, r0 + rows);
    float s = 0.f;
    for (int64_t r = r0; r < r1; r++) {
        const float v = load_as_f32(x, dt, r * K + k);
        s = __builtin_fmaf(v, v, s);
    }
    partial[(int64_t)blockIdx.y * K + k] = s;
}

// diag / n + 1e-6 with torch's steps: the diagonal rounded to x's dtype,
// divided by n (a host scalar: times its FP32 reciprocal, or IEEE division
// in the ieee_div mode), rounded, plus 1e-6, rounded.
__global__ void __launch_bounds__(kSieveNT) sieve_hdiag_final_kernel(const float *partial, int slices, int64_t n,
                                                                     int64_t K, int dt, void *out, int ieee_div) {
    const int64_t k = (int64_t)blockIdx.x * kSieveNT + threadIdx.x;
    if (k >= K) return;
    float s = 0.f;
    for (int i = 0; i < slices; i++) s += partial[(int64_t)i * K + k];
    const float d = round_as(dt, s);
    const float q = round_as(dt, sieve_scalar_div(d, (float)n, ieee_div));
    store_from_f32(out, dt, k, round_as(dt, q + 1e-6f));
}

static unsigned sieve_grid(int64_t n) {
    const int64_t b = (n + kSieveNT - 1) / kSieveNT;
    return (unsigned)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

hipError_t launch_sieve_quantize(const void *w, int dt, int64_t N, int64_t K, void *w_base, int ieee_div,
                                 hipStream_t stream) {
    SieveArgs a{};
    a.ieee_div = ieee_div;
    a.w = w;
    a.dt = dt;
    a.N = N;
    a.K = K;
    a.w_base = w_base;
    hipLaunchKernelGGL(sieve_quant_kernel, dim3((unsigned)N), dim3(kSieveNT), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_sieve_split(const void *w, int dt, int64_t N, int64_t K, const void *h, int hdt, int64_t h_stride,
                              int score_dt, int use_rank, int64_t rank, float thresh, void *w_base, void *w_ortho,
                              float *score, void *sel, int ieee_div, hipStream_t stream) {
    SieveArgs a{};
    a.ieee_div = ieee_div;
    a.w = w;
    a.dt = dt;
    a.N = N;
    a.K = K;
    a.w_base = w_base;
    a.resid = w_ortho;
    a.score = score;
    a.h = h;
    a.hdt = hdt;
    a.h_stride = h_stride;
    a.score_dt = score_dt;
    hipLaunchKernelGGL(sieve_quant_kernel, dim3((unsigned)N), dim3(kSieveNT), 0, stream, a);
    const int64_t n = N * K;
    SieveSel *st = static_cast<SieveSel *>(sel);
    int from_sel = 0;
    if (use_rank) {
        if (rank > 0) {
            hipLaunchKernelGGL(sieve_sel_init_kernel, dim3(1), dim3(256), 0, stream, st, (uint32_t)rank);
            for (int shift = 24; shift >= 0; shift -= 8) {
                hipLaunchKernelGGL(sieve_hist_kernel, dim3(sieve_grid(n)), dim3(kSieveNT), 0, stream, score, n, st,
                                   shift);
                hipLaunchKernelGGL(sieve_pick_kernel, dim3(1), dim3(256), 0, stream, st, shift);
            }
            from_sel = 1;
        } else {
            // k == 0: the reference keeps nothing (threshold max + 1)
            thresh = __builtin_nanf("");
        }
    }
    hipLaunchKernelGGL(sieve_mask_kernel, dim3(sieve_grid(n)), dim3(kSieveNT), 0, stream, w_ortho, dt, score, n,
                       st, from_sel, thresh, score_dt);
    return hipGetLastError();
}

int64_t sieve_hdiag_slices(int64_t n) {
    const int64_t s = (n + 255) / 256;
    return s < 64 ? (s > 0 ? s : 1) : 64;
}

hipError_t launch_sieve_hdiag(const void *x, int dt, int64_t n, int64_t K, float *partial, void *out, int ieee_div,
                              hipStream_t stream) {
    const int64_t slices = sieve_hdiag_slices(n);
    const int64_t rows = (n + slices - 1) / slices;
    const unsigned cb = (unsigned)((K + kSieveNT - 1) / kSieveNT);
    hipLaunchKernelGGL(sieve_hdiag_partial_kernel, dim3(cb, (unsigned)slices), dim3(kSieveNT), 0, stream, x, dt, n, K,
                       rows, partial);
    hipLaunchKernelGGL(sieve_hdiag_final_kernel, dim3(cb), dim3(kSieveNT), 0, stream, partial, (int)slices, n, K, dt,
                       out, ieee_div);
    return hipGetLastError();
}

}  // namespace orth
