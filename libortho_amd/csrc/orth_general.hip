// General-shape dual GEMM and the FP32 dequant entry.
//
// The general kernel takes every layer the fast kernels do not: any even K,
// any group size dividing K, FP16/BF16/FP32 activations, FP16/FP32 scales and
// values, any CSR (unsorted or duplicate columns are summed as given).  One
// wave per output row and up to MT tokens: lanes split K, then a wave
// reduction per token, so the row's weights are read once for MT tokens.  It
// follows /root/reference/src/dual_gemm.cu:176-225 in what it computes (base
// dot product with x*(q*s) per element, CSR row sum, acc += alpha*sum) but not
// in how: the reference gives each thread a whole row and reads one byte per
// nibble with lanes 2 KB apart.  Here, when K % 8 == 0 and the weights are
// 4-byte aligned, each lane reads a 32-bit word (8 nibbles) per 256-byte
// stride of the row, with one scale per word when the group size is a
// multiple of 8, and the word's 8 activations of a token as 16-byte vectors
// when the activations are 16-byte aligned; otherwise a byte (2 nibbles) per
// lane, as the shapes allow.
#include "orth_common.h"

namespace orth {

// Activations k .. k + 7 of row offset i (k % 8 == 0, 16-byte aligned base).
template <int IO>
__device__ __forceinline__ void load_x8(const void *x, int64_t i, float out[8]) {
    if constexpr (IO == ORTH_DT_F32) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(x) + i);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(x) + i + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            out[e] = a[e];
            out[4 + e] = b[e];
        }
    } else {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(x) + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if constexpr (IO == ORTH_DT_BF16) {
                out[2 * e] = bf16_bits_to_f32((uint16_t)(w[e] & 0xffffu));
                out[2 * e + 1] = bf16_bits_to_f32((uint16_t)(w[e] >> 16));
            } else {
                out[2 * e] = (float)__builtin_bit_cast(f16, (uint16_t)(w[e] & 0xffffu));
                out[2 * e + 1] = (float)__builtin_bit_cast(f16, (uint16_t)(w[e] >> 16));
            }
        }
    }
}

template <int IO, int MT>
__global__ void __launch_bounds__(256) general_kernel(ForwardArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + wave;
    if (n >= a.N) return;
    const int64_t K = a.K;
    const uint8_t *qrow = a.q + n * (K >> 1);
    const int64_t srow = n * a.ngroups;
    // group of element k: 32-bit division while K fits (K may reach 2^40 / N)
    const bool k32 = K <= 0xffffffffLL;
    const uint32_t G32 = (uint32_t)a.G;
    auto grp = [&](int64_t k) -> int64_t { return k32 ? (int64_t)((uint32_t)k / G32) : k / a.G; };
    // uniform shape tests: 32-bit words of the row, 16-byte activation vectors
    const bool words = (K & 7) == 0 && (reinterpret_cast<uintptr_t>(a.q) & 3) == 0;
    const bool xvec = words && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
    const bool word_scale = a.ngroups == 1 || (a.G & 7) == 0;  // one group per word
    for (int64_t m0 = (int64_t)blockIdx.y * MT; m0 < a.M; m0 += (int64_t)gridDim.y * MT) {
        const int mt = (int)(a.M - m0 < MT ? a.M - m0 : MT);  // live tokens (uniform)
        float acc[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i] = 0.0f;
        if (words) {
            const uint32_t *qw = reinterpret_cast<const uint32_t *>(qrow);
            for (int64_t w = lane; w < (K >> 3); w += 64) {
                const uint32_t word = qw[w];
                const int64_t k0 = 8 * w;
                float wf[8];
                if (word_scale) {
                    const float s = load_as_f32(a.scales, a.scale_dtype,
                                                srow + (a.ngroups == 1 ? 0 : grp(k0)));
#pragma unroll
                    for (int e = 0; e < 8; e++) wf[e] = (float)sext4((word >> (4 * e)) & 0xfu) * s;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        wf[e] = (float)sext4((word >> (4 * e)) & 0xfu) *
                                load_as_f32(a.scales, a.scale_dtype, srow + grp(k0 + e));
                }
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    if (i < mt) {
                        const int64_t xi = (m0 + i) * K + k0;
                        float xv[8];
                        if (xvec) {
                            load_x8<IO>(a.x, xi, xv);
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; e++) xv[e] = load_as_f32(a.x, IO, xi + e);
                        }
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[i] = __builtin_fmaf(xv[e], wf[e], acc[i]);
                    }
                }
            }
        } else {
            // each lane takes one byte (two consecutive k) per 64-byte stride
            for (int64_t b = lane; b < (K >> 1); b += 64) {
                const uint32_t byte = qrow[b];
                const int64_t k0 = 2 * b;
                const float w0 = (float)sext4(byte & 0xfu) *
                                 load_as_f32(a.scales, a.scale_dtype, srow + grp(k0));
                const float w1 = (float)sext4(byte >> 4) *
                                 load_as_f32(a.scales, a.scale_dtype, srow + grp(k0 + 1));
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    if (i < mt) {
                        const int64_t xi = (m0 + i) * K + k0;
                        acc[i] = __builtin_fmaf(load_as_f32(a.x, IO, xi), w0, acc[i]);
                        acc[i] = __builtin_fmaf(load_as_f32(a.x, IO, xi + 1), w1, acc[i]);
                    }
                }
            }
        }
        float sp[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) sp[i] = 0.0f;
        if (a.has_ortho) {
            int32_t rs, re;
            csr_row_range(a.row_ptr, n, a.nnz, rs, re);
            for (int32_t j = rs + lane; j < re; j += 64) {
                const int32_t c = a.col[j];
                if (c >= 0 && c < K) {
                    const float v = load_as_f32(a.vals, a.val_dtype, j);
#pragma unroll
                    for (int i = 0; i < MT; i++)
                        if (i < mt) sp[i] = __builtin_fmaf(v, load_as_f32(a.x, IO, (m0 + i) * K + c), sp[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < MT; i++) {
            float v = wave_sum(acc[i]);
            const float s = wave_sum(sp[i]);
            if (lane == 0 && i < mt) {
                if (a.has_ortho) v += a.alpha * s;
                // with a bias: y rounded, then y + bias in FP32 rounded (as out_f16)
                if (a.bias) v = round_as(IO, v) + load_as_f32(a.bias, a.bias_dtype, n);
                store_from_f32(a.y, IO, (m0 + i) * a.N + n, v);
            }
        }
    }
}

template <int IO>
static hipError_t launch_general_io(const ForwardArgs &a, hipStream_t stream) {
    // (tiles of 8 tokens, or the word loop unrolled 4 deep, measured slower)
    const int64_t mt = a.M <= 1 ? 1 : a.M == 2 ? 2 : 4;
    const int64_t tiles = (a.M + mt - 1) / mt;
    const dim3 grid((unsigned)((a.N + 3) / 4), (unsigned)(tiles < 65535 ? tiles : 65535));
    if (mt == 1) hipLaunchKernelGGL((general_kernel<IO, 1>), grid, dim3(256), 0, stream, a);
    else if (mt == 2) hipLaunchKernelGGL((general_kernel<IO, 2>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((general_kernel<IO, 4>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_general(const ForwardArgs &a, hipStream_t stream) {
    if (a.io_dtype == ORTH_DT_F32) return launch_general_io<ORTH_DT_F32>(a, stream);
    if (a.io_dtype == ORTH_DT_BF16) return launch_general_io<ORTH_DT_BF16>(a, stream);
    return launch_general_io<ORTH_DT_F16>(a, stream);
}

// out[n*K + k] = float(q[n,k]) * float(s[n, k/G]); one thread per byte.
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t *q, const void *scales,
                                                      int scale_dtype, int64_t ngroups,
                                                      int64_t G, int64_t N, int64_t K,
                                                      float *out) {
    const int64_t nbytes = N * (K >> 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nbytes;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = 2 * i;  // flat element index of the low nibble
        const int64_t n = e / K, k = e - n * K;
        const uint32_t byte = q[i];
        const float s0 = load_as_f32(scales, scale_dtype, n * ngroups + k / G);
        const float s1 = load_as_f32(scales, scale_dtype, n * ngroups + (k + 1) / G);
        out[e] = (float)sext4(byte & 0xfu) * s0;
        out[e + 1] = (float)sext4(byte >> 4) * s1;
    }
}

hipError_t launch_dequant(const ForwardArgs &a, float *out, hipStream_t stream) {
    const int64_t nbytes = a.N * (a.K >> 1);
    int64_t blocks = (nbytes + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a.q,
                       a.scales, a.scale_dtype, a.ngroups, a.G, a.N, a.K, out);
    return hipGetLastError();
}

}  // namespace orth
