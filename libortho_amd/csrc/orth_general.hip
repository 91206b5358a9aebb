// General-shape dual GEMM and the FP32 dequant entry.
//
// The general kernel takes every layer the fast kernels do not: any even K,
// any group size dividing K, FP16/BF16/FP32 activations, FP16/FP32 scales and
// values, any CSR (unsorted or duplicate columns are summed as given).  One
// wave per (token, output row): lanes split K, then a wave reduction.  It
// follows /root/reference/src/dual_gemm.cu:176-225 in what it computes (base
// dot product with x*(q*s) per element, CSR row sum, acc += alpha*sum) but not
// in how: the reference gives each thread a whole row and reads one byte per
// nibble with lanes 2 KB apart.
#include "orth_common.h"

namespace orth {

__global__ void __launch_bounds__(256) general_kernel(ForwardArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + wave;
    if (n >= a.N) return;
    const int64_t K = a.K;
    const uint8_t *qrow = a.q + n * (K >> 1);
    const int64_t srow = n * a.ngroups;
    for (int64_t m = blockIdx.y; m < a.M; m += gridDim.y) {
        const int64_t xrow = m * K;

        float acc = 0.0f;
        // each lane takes one byte (two consecutive k) per 64-byte stride
        for (int64_t b = lane; b < (K >> 1); b += 64) {
            const uint32_t byte = qrow[b];
            const int64_t k0 = 2 * b;
            const float s0 = load_as_f32(a.scales, a.scale_dtype, srow + k0 / a.G);
            const float s1 = load_as_f32(a.scales, a.scale_dtype, srow + (k0 + 1) / a.G);
            const float w0 = (float)sext4(byte & 0xfu) * s0;
            const float w1 = (float)sext4(byte >> 4) * s1;
            acc += load_as_f32(a.x, a.io_dtype, xrow + k0) * w0;
            acc += load_as_f32(a.x, a.io_dtype, xrow + k0 + 1) * w1;
        }
        float sp = 0.0f;
        if (a.has_ortho) {
            int32_t rs, re;
            csr_row_range(a.row_ptr, n, a.nnz, rs, re);
            for (int32_t j = rs + lane; j < re; j += 64) {
                const int32_t c = a.col[j];
                if (c >= 0 && c < K)
                    sp += load_as_f32(a.vals, a.val_dtype, j) * load_as_f32(a.x, a.io_dtype, xrow + c);
            }
        }
        acc = wave_sum(acc);
        sp = wave_sum(sp);
        if (lane == 0) {
            if (a.has_ortho) acc += a.alpha * sp;
            // with a bias: y rounded, then y + bias in FP32 rounded (as out_f16)
            if (a.bias) acc = round_as(a.io_dtype, acc) + load_as_f32(a.bias, a.bias_dtype, n);
            store_from_f32(a.y, a.io_dtype, m * a.N + n, acc);
        }
    }
}

hipError_t launch_general(const ForwardArgs &a, hipStream_t stream) {
    const int64_t gy = a.M < 65535 ? a.M : 65535;
    dim3 grid((unsigned)((a.N + 3) / 4), (unsigned)gy);
    hipLaunchKernelGGL(general_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
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
