/*
 * CPU baseline: the reference CPU forward, restated, for timing beside the
 * GPU path.  TEST/BENCH INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).
 *
 * Follows /root/reference/src/ortho.c:327-402 (orth_layer_forward): one
 * thread, FP32, loop order batch -> output row -> input column with
 * acc += x * (w * s), then the sparse update y[row] += alpha * v * x[col].
 * Compiled with the reference's flags, /root/reference/tests/Makefile:4
 * (-O3 -ffast-math -funroll-loops).
 *
 * Two restatement details the reference cannot express at these shapes:
 *   - the scale is indexed by group, s[n, k/G] (G == K is the reference);
 *   - the sparse term walks CSR rows (the reference's uint16 COO index
 *     addresses at most 65536 weights, /root/reference/include/ortho.h:48).
 * The per-group inner loop keeps the reference's arithmetic order: the
 * scale is constant inside a group, so hoisting it changes nothing.
 */
#include <stdint.h>
#include <stddef.h>
#include <time.h>

static inline int unpack_nib(const uint8_t *packed, size_t idx) {
    unsigned byte = packed[idx >> 1];
    unsigned nib = (idx & 1) ? (byte >> 4) : (byte & 0x0f);
    return (nib & 0x8) ? (int)nib - 16 : (int)nib;
}

int orc_baseline_forward_f32(const uint8_t *q, const float *scales, int64_t ngroups,
                             const int32_t *row_ptr, const int32_t *col,
                             const float *vals, int64_t nnz, float alpha,
                             const float *x, float *y, int64_t M, int64_t K, int64_t N) {
    if (!q || !scales || !x || !y || ngroups <= 0 || K % ngroups != 0) return -1;
    const int64_t G = K / ngroups;
    const int has_ortho = alpha > 0.0f && nnz > 0 && row_ptr && col && vals;
    for (int64_t b = 0; b < M; b++) {
        const float *xr = x + b * K;
        float *yr = y + b * N;
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            const size_t base = (size_t)(n * K);
            for (int64_t g = 0; g < ngroups; g++) {
                const float s = scales[n * ngroups + g];
                for (int64_t k = g * G; k < (g + 1) * G; k++) {
                    int w = unpack_nib(q, base + (size_t)k);
                    acc += xr[k] * ((float)w * s);
                }
            }
            yr[n] = acc;
        }
        if (has_ortho) {
            for (int64_t n = 0; n < N; n++) {
                for (int32_t j = row_ptr[n]; j < row_ptr[n + 1]; j++) {
                    int32_t c = col[j];
                    if (c >= 0 && c < K) yr[n] += alpha * vals[j] * xr[c];
                }
            }
        }
    }
    return 0;
}

/* Times `iters` calls after `warmup` calls on the calling thread; returns
 * the mean seconds per call (CLOCK_MONOTONIC, as the reference's
 * benchmark does, /root/reference/tests/benchmark_null_test.c:63-67). */
double orc_baseline_time(const uint8_t *q, const float *scales, int64_t ngroups,
                         const int32_t *row_ptr, const int32_t *col, const float *vals,
                         int64_t nnz, float alpha, const float *x, float *y, int64_t M,
                         int64_t K, int64_t N, int warmup, int iters) {
    for (int i = 0; i < warmup; i++)
        orc_baseline_forward_f32(q, scales, ngroups, row_ptr, col, vals, nnz, alpha, x, y,
                                 M, K, N);
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < iters; i++)
        orc_baseline_forward_f32(q, scales, ngroups, row_ptr, col, vals, nnz, alpha, x, y,
                                 M, K, N);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    double dt = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    return iters > 0 ? dt / iters : 0.0;
}
