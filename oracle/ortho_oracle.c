/*
 * CPU oracle for libortho's fused dual GEMM.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (libortho_amd/,
 * the C-ABI library, OrthoLinear) may link, load or call this file.  The
 * only permitted users are tests/, __graft_entry__.smoke() (as the checker)
 * and bench.py's cpu_baseline leg.
 *
 * It restates the reference algorithm from the reference sources:
 *
 *   y[m,n] = sum_k x[m,k] * (float(q[n,k]) * s[n, k/G])
 *          + [alpha > 0 && nnz > 0] * alpha * sum_{j in row n} v_j * x[m, c_j]
 *
 *   - nibble decode:           /root/reference/src/ortho.c:315-325
 *   - base loop + accumulation: /root/reference/src/ortho.c:346-366
 *   - alpha gate:              /root/reference/src/ortho.c:343
 *   - sparse update order:     /root/reference/src/ortho.c:384-398
 *     (restated over CSR rows; the reference COO walk visits entries in
 *     row-major order, which is the order CSR stores them in,
 *     /root/reference/tools/sieve.py:131-136)
 *   - column guard:            /root/reference/src/dual_gemm.cu:124
 *
 * Group scales (G < K) are an extension the reference does not have: the
 * scale index is n*(K/G) + k/G; G == K reproduces the reference's per-row
 * scale exactly.
 *
 * Parity pins (see tests/test_oracle.py):
 *   orc_unpack_int4        exhaustive over all 256 byte values (closed form)
 *   orc_forward_ref_f32    golden vectors written by the reference's own
 *                          orth_layer_forward (oracle/_ref), plus a live
 *                          comparison against it when it is built
 *   orc_forward_f64        numpy float64 dense brute force (a different code
 *                          path: dequantise the whole matrix, matmul)
 *   orc_dequant_f32        closed form float(q)*float(s), exact in FP32
 *   orc_forward_ref_coo_f32  the reference's own test harness inputs
 *                          (srand(42)) and outputs, bit-for-bit tolerance
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

/* ---------------- IEEE binary16 / bfloat16 <-> binary32 ---------------- */
/* Written from the format definitions (1 sign, 5 exponent bias 15,
 * 10 mantissa bits; bfloat16 is the top half of binary32). */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: value = mant * 2^-24 */
            float v = (float)mant * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) { /* inf or nan */
        return sign | 0x7c00 | (absx > 0x7f800000u ? 0x200 : 0);
    }
    if (absx >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return sign | 0x7c00;
    }
    if (absx < 0x38800000u) { /* below min normal 2^-14: subnormal or zero */
        /* value / 2^-24 rounded to nearest even integer */
        float a;
        memcpy(&a, &absx, 4);
        float scaled = a * 16777216.0f; /* exact: power-of-two scaling */
        float r = nearbyintf(scaled);   /* default rounding mode: RNE */
        return sign | (uint16_t)r;
    }
    uint32_t e = (absx >> 23) - 112;
    uint32_t mant = absx & 0x7fffff;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fff;
    if (rest > 0x1000 || (rest == 0x1000 && (h & 1))) {
        h += 1; /* carry into the exponent is the correct result */
    }
    return sign | (uint16_t)h;
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_f16_array_to_f32(const uint16_t *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f32_array_to_f16(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ---------------- nibble decode (ortho.c:315-325) ---------------- */
/* Element i of the row-major [N, K] matrix lives in byte i/2; even i in the
 * low nibble, odd i in the high nibble; two's complement, sign bit 3. */
int orc_unpack_int4(const uint8_t *packed, size_t idx) {
    unsigned byte = packed[idx >> 1];
    unsigned nib = (idx & 1) ? (byte >> 4) : (byte & 0x0f);
    return (nib & 0x8) ? (int)nib - 16 : (int)nib;
}

/* ---------------- dequantised base weights, FP32 ---------------- */
/* out[n*K + k] = float(q[n,k]) * s[n, k/G]; exact in FP32 because |q| <= 8
 * has 3 significant bits and a binary16 scale has 11. */
void orc_dequant_f32(const uint8_t *q, const float *scales, int64_t N, int64_t K,
                     int64_t ngroups, float *out) {
    int64_t G = K / ngroups;
    for (int64_t n = 0; n < N; n++) {
        for (int64_t k = 0; k < K; k++) {
            int w = orc_unpack_int4(q, (size_t)(n * K + k));
            out[n * K + k] = (float)w * scales[n * ngroups + k / G];
        }
    }
}

static int has_ortho(float alpha, int64_t nnz) { return alpha > 0.0f && nnz > 0; }

/* ---------------- reference-order FP32 forward ---------------- */
/* ortho.c:346-366: per output row one FP32 accumulator, acc += x*(w*s) in
 * k order; then ortho.c:384-398: y[row] += alpha*v*x[col] in entry order. */
int orc_forward_ref_f32(const uint8_t *q, const float *scales, int64_t ngroups,
                        const int32_t *row_ptr, const int32_t *col, const float *vals,
                        int64_t nnz, float alpha, const float *x, float *y,
                        int64_t M, int64_t K, int64_t N) {
    if (!q || !scales || !x || !y || K <= 0 || N <= 0 || M < 0 || ngroups <= 0 ||
        K % ngroups != 0)
        return -1;
    int64_t G = K / ngroups;
    int ortho = has_ortho(alpha, nnz) && row_ptr && col && vals;
    for (int64_t b = 0; b < M; b++) {
        const float *xr = x + b * K;
        float *yr = y + b * N;
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int64_t k = 0; k < K; k++) {
                int w = orc_unpack_int4(q, (size_t)(n * K + k));
                float s = scales[n * ngroups + k / G];
                acc += xr[k] * ((float)w * s);
            }
            yr[n] = acc;
        }
        if (ortho) {
            for (int64_t n = 0; n < N; n++) {
                for (int64_t j = row_ptr[n]; j < row_ptr[n + 1]; j++) {
                    int32_t c = col[j];
                    if (c >= 0 && c < K) yr[n] += alpha * vals[j] * xr[c];
                }
            }
        }
    }
    return 0;
}

/* ---------------- FP64 accumulation of the same formula ---------------- */
int orc_forward_f64(const uint8_t *q, const float *scales, int64_t ngroups,
                    const int32_t *row_ptr, const int32_t *col, const float *vals,
                    int64_t nnz, float alpha, const float *x, double *y,
                    int64_t M, int64_t K, int64_t N) {
    if (!q || !scales || !x || !y || K <= 0 || N <= 0 || M < 0 || ngroups <= 0 ||
        K % ngroups != 0)
        return -1;
    int64_t G = K / ngroups;
    int ortho = has_ortho(alpha, nnz) && row_ptr && col && vals;
    for (int64_t b = 0; b < M; b++) {
        const float *xr = x + b * K;
        double *yr = y + b * N;
        for (int64_t n = 0; n < N; n++) {
            double acc = 0.0;
            for (int64_t g = 0; g < ngroups; g++) {
                double part = 0.0;
                for (int64_t k = g * G; k < (g + 1) * G; k++) {
                    int w = orc_unpack_int4(q, (size_t)(n * K + k));
                    part += (double)xr[k] * (double)w;
                }
                acc += part * (double)scales[n * ngroups + g];
            }
            if (ortho) {
                double sp = 0.0;
                for (int64_t j = row_ptr[n]; j < row_ptr[n + 1]; j++) {
                    int32_t c = col[j];
                    if (c >= 0 && c < K) sp += (double)vals[j] * (double)xr[c];
                }
                acc += (double)alpha * sp;
            }
            yr[n] = acc;
        }
    }
    return 0;
}

/* ---------------- legacy COO (uint16 flat index) forward ---------------- */
/* The reference's own CPU test path (ortho.c:384-398 with its COO index):
 * per-row FP32 scales; flat index -> (idx / K, idx % K); out-of-range
 * entries skipped.  Used only to pin the oracle against the reference's
 * golden vectors and its compiled code. */
int orc_forward_ref_coo_f32(const uint8_t *q, const float *scales, const uint16_t *idx,
                            const float *vals, int64_t count, float alpha,
                            const float *x, float *y, int64_t M, int64_t K, int64_t N) {
    if (!q || !scales || !x || !y || K <= 0 || N <= 0 || M < 0) return -1;
    int ortho = has_ortho(alpha, count) && idx && vals;
    for (int64_t b = 0; b < M; b++) {
        const float *xr = x + b * K;
        float *yr = y + b * N;
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            float s = scales[n];
            for (int64_t k = 0; k < K; k++) {
                int w = orc_unpack_int4(q, (size_t)(n * K + k));
                acc += xr[k] * ((float)w * s);
            }
            yr[n] = acc;
        }
        if (ortho) {
            for (int64_t i = 0; i < count; i++) {
                int64_t row = idx[i] / K, c = idx[i] % K;
                if (row < N && c < K) yr[row] += alpha * vals[i] * xr[c];
            }
        }
    }
    return 0;
}
