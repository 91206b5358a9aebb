/* Runs the CPU oracle (oracle/ortho_oracle.c, oracle/cpu_baseline.c) under
 * AddressSanitizer and UBSan (tests/test_sanitizers.py): random layers with
 * per-row and group scales, empty rows, columns outside [0, K) (skipped by
 * the column guard), negative / zero alpha, and the COO path; the FP32
 * restatements must stay within 1e-4 relative of the FP64 accumulation.
 * Prints "oracle ok" and exits 0 on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int orc_forward_ref_f32(const uint8_t *q, const float *scales, int64_t ngroups, const int32_t *row_ptr,
                        const int32_t *col, const float *vals, int64_t nnz, float alpha, const float *x, float *y,
                        int64_t M, int64_t K, int64_t N);
int orc_forward_f64(const uint8_t *q, const float *scales, int64_t ngroups, const int32_t *row_ptr,
                    const int32_t *col, const float *vals, int64_t nnz, float alpha, const float *x, double *y,
                    int64_t M, int64_t K, int64_t N);
int orc_forward_ref_coo_f32(const uint8_t *q, const float *scales, const uint16_t *idx, const float *vals,
                            int64_t count, float alpha, const float *x, float *y, int64_t M, int64_t K, int64_t N);
int orc_baseline_forward_f32(const uint8_t *q, const float *scales, int64_t ngroups, const int32_t *row_ptr,
                             const int32_t *col, const float *vals, int64_t nnz, float alpha, const float *x,
                             float *y, int64_t M, int64_t K, int64_t N);
void orc_dequant_f32(const uint8_t *q, const float *scales, int64_t N, int64_t K, int64_t ngroups, float *out);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);

static uint64_t st = 88172645463325252ull;
static uint32_t rnd(void) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    return (uint32_t)st;
}
static float frand(void) { return (float)(rnd() % 20001) / 10000.0f - 1.0f; }

static int one_case(int64_t M, int64_t K, int64_t N, int64_t ngroups, float alpha, int per_row_max) {
    uint8_t *q = malloc((size_t)(N * K / 2));
    float *s = malloc(sizeof(float) * (size_t)(N * ngroups));
    float *x = malloc(sizeof(float) * (size_t)(M * K));
    int32_t *rp = malloc(sizeof(int32_t) * (size_t)(N + 1));
    int32_t *col = malloc(sizeof(int32_t) * (size_t)(N * per_row_max + 1));
    float *v = malloc(sizeof(float) * (size_t)(N * per_row_max + 1));
    float *y1 = malloc(sizeof(float) * (size_t)(M * N)), *y2 = malloc(sizeof(float) * (size_t)(M * N));
    double *yd = malloc(sizeof(double) * (size_t)(M * N));
    float *wd = malloc(sizeof(float) * (size_t)(N * K));
    for (int64_t i = 0; i < N * K / 2; i++) q[i] = (uint8_t)rnd();
    for (int64_t i = 0; i < N * ngroups; i++) s[i] = 0.02f * fabsf(frand());
    for (int64_t i = 0; i < M * K; i++) x[i] = frand();
    int64_t nnz = 0;
    rp[0] = 0;
    for (int64_t n = 0; n < N; n++) {
        int c = (int)(rnd() % (uint32_t)(per_row_max + 1));
        for (int j = 0; j < c; j++) {
            int32_t cc = (int32_t)(rnd() % (uint32_t)K);
            if (rnd() % 17 == 0) cc = (rnd() & 1) ? -3 : (int32_t)(K + 5); /* outside [0, K) */
            col[nnz] = cc;
            v[nnz++] = 0.05f * frand();
        }
        rp[n + 1] = (int32_t)nnz;
    }
    int bad = 0;
    bad |= orc_forward_ref_f32(q, s, ngroups, rp, col, v, nnz, alpha, x, y1, M, K, N);
    bad |= orc_baseline_forward_f32(q, s, ngroups, rp, col, v, nnz, alpha, x, y2, M, K, N);
    bad |= orc_forward_f64(q, s, ngroups, rp, col, v, nnz, alpha, x, yd, M, K, N);
    orc_dequant_f32(q, s, N, K, ngroups, wd);
    double ymax = 1e-30;
    for (int64_t i = 0; i < M * N; i++) ymax = fmax(ymax, fabs(yd[i]));
    for (int64_t i = 0; i < M * N; i++)
        if (fabs(y1[i] - yd[i]) > 1e-4 * ymax || fabs(y2[i] - yd[i]) > 1e-4 * ymax) bad = 1;
    if (ngroups == 1 && N * K <= 65536) {
        uint16_t *idx = malloc(sizeof(uint16_t) * (size_t)(nnz + 1));
        float *vv = malloc(sizeof(float) * (size_t)(nnz + 1));
        int64_t c = 0;
        for (int64_t n = 0; n < N; n++)
            for (int32_t j = rp[n]; j < rp[n + 1]; j++)
                if (col[j] >= 0 && col[j] < K) {
                    idx[c] = (uint16_t)(n * K + col[j]);
                    vv[c++] = v[j];
                }
        bad |= orc_forward_ref_coo_f32(q, s, idx, vv, c, alpha, x, y2, M, K, N);
        for (int64_t i = 0; i < M * N; i++)
            if (fabs(y2[i] - yd[i]) > 1e-4 * ymax) bad = 1;
        free(idx);
        free(vv);
    }
    free(q); free(s); free(x); free(rp); free(col); free(v); free(y1); free(y2); free(yd); free(wd);
    return bad;
}

int main(void) {
    int bad = 0;
    for (int h = 0; h < 65536; h++) {
        float f = orc_f16_to_f32((uint16_t)h);
        if (f == f && orc_f32_to_f16(f) != (uint16_t)h) bad = 1;
    }
    bad |= one_case(3, 64, 48, 1, 1.0f, 6);
    bad |= one_case(2, 256, 40, 2, 0.5f, 20);
    bad |= one_case(5, 128, 33, 4, 0.0f, 9);
    bad |= one_case(1, 256, 256, 1, -1.0f, 3);
    bad |= one_case(4, 512, 17, 4, 1.0f, 0);
    bad |= one_case(0, 64, 8, 1, 1.0f, 2);
    if (bad) {
        printf("oracle FAILED\n");
        return 1;
    }
    printf("oracle ok\n");
    return 0;
}
