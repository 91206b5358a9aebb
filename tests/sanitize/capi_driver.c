/* Drives the host side of the C ABI (include/orth_hip.h) through malformed
 * and valid arguments without a GPU, built with AddressSanitizer and UBSan
 * by tests/test_sanitizers.py.  Each call must return the documented
 * status and leave a message; none may touch memory it does not own.
 * Prints "capi ok" and exits 0 when every expectation holds. */
#include <pthread.h>
#include <stdio.h>
#include <string.h>

#include "orth_hip.h"

static int failures = 0;

static void expect(int got, int want, const char *what) {
    if (got != want) {
        printf("FAIL %s: status %d, expected %d (%s)\n", what, got, want, orth_hip_last_error());
        failures++;
    } else if (want != ORTH_OK && strlen(orth_hip_last_error()) == 0) {
        printf("FAIL %s: no message\n", what);
        failures++;
    }
}

static char qbuf[4096], sbuf[4096], xbuf[4096], ybuf[4096], zbuf[4096];
static int32_t rp[65], col[64];
static unsigned short vals[64];

static orth_hip_layer_t good(void) {
    orth_hip_layer_t L;
    memset(&L, 0, sizeof(L));
    L.base.q_weight = qbuf;
    L.base.q_scales = sbuf;
    L.base.q_bits = 4;
    L.base.scale_dtype = ORTH_DT_F16;
    L.base.scale_groups = 2;
    L.base.in_features = 256;
    L.base.out_features = 64;
    L.ortho.row_ptr = rp;
    L.ortho.col_indices = col;
    L.ortho.values = vals;
    L.ortho.value_dtype = ORTH_DT_F16;
    L.ortho.count = 64;
    L.alpha = 1.0f;
    return L;
}

static void *thread_main(void *arg) {
    (void)arg;
    for (int i = 0; i < 2000; i++) {
        orth_hip_layer_t L = good();
        L.base.q_bits = 3 + (i & 1);
        int rc = orth_layer_check_hip(&L, xbuf, ybuf, 4, ORTH_DT_F16);
        if (rc != ((i & 1) ? ORTH_OK : ORTH_ERR_UNSUPPORTED)) failures++;
    }
    return NULL;
}

int main(void) {
    for (int i = 0; i <= 64; i++) rp[i] = i;
    orth_hip_layer_t L = good();
    expect(orth_layer_check_hip(&L, xbuf, ybuf, 4, ORTH_DT_F16), ORTH_OK, "valid layer");
    expect(orth_layer_check_hip(NULL, xbuf, ybuf, 4, ORTH_DT_F16), ORTH_ERR_INVALID_ARGUMENT, "NULL layer");
#define BAD(field, value, status)                                                   \
    do {                                                                            \
        orth_hip_layer_t B = good();                                                \
        B.field = value;                                                            \
        expect(orth_layer_check_hip(&B, xbuf, ybuf, 4, ORTH_DT_F16), status, #field); \
        expect((int)(orth_ortho_plan_bytes(&B) < 0 ? -orth_ortho_plan_bytes(&B) : 0), \
               status, "plan bytes " #field);                                       \
    } while (0)
    BAD(base.q_weight, NULL, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.q_scales, NULL, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.q_bits, 8, ORTH_ERR_UNSUPPORTED);
    BAD(base.in_features, 0, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.in_features, 255, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.in_features, -256, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.in_features, (int64_t)1 << 62, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.out_features, 0, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.out_features, -5, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.scale_groups, 0, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.scale_groups, 3, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.scale_groups, -2, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.scale_dtype, ORTH_DT_BF16, ORTH_ERR_INVALID_ARGUMENT);
    BAD(base.scale_dtype, 99, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.count, -1, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.count, (int64_t)1 << 31, ORTH_ERR_UNSUPPORTED);
    BAD(ortho.row_ptr, NULL, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.col_indices, NULL, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.values, NULL, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.value_dtype, ORTH_DT_BF16, ORTH_ERR_INVALID_ARGUMENT);
    BAD(ortho.value_dtype, -7, ORTH_ERR_INVALID_ARGUMENT);
    expect(orth_layer_check_hip(&L, xbuf, ybuf, -1, ORTH_DT_F16), ORTH_ERR_INVALID_ARGUMENT, "negative batch");
    expect(orth_layer_check_hip(&L, xbuf, ybuf, 4, 3), ORTH_ERR_INVALID_ARGUMENT, "io dtype");
    expect(orth_layer_check_hip(&L, NULL, ybuf, 4, ORTH_DT_F16), ORTH_ERR_INVALID_ARGUMENT, "NULL input");
    expect(orth_layer_check_hip(&L, xbuf, NULL, 4, ORTH_DT_F16), ORTH_ERR_INVALID_ARGUMENT, "NULL output");
    expect(orth_layer_check_hip(&L, xbuf, ybuf, (int64_t)1 << 60, ORTH_DT_F16), ORTH_ERR_INVALID_ARGUMENT,
           "huge batch");
    /* empty ortho: NULL CSR allowed */
    orth_hip_layer_t E = good();
    E.ortho.count = 0;
    E.ortho.row_ptr = NULL;
    E.ortho.col_indices = NULL;
    E.ortho.values = NULL;
    expect(orth_layer_check_hip(&E, xbuf, ybuf, 4, ORTH_DT_F16), ORTH_OK, "empty ortho");
    expect((int)orth_ortho_plan_bytes(&E), 0, "empty ortho plan bytes");
    /* forward: batch 0 is a no-op; a real call stops at the device check */
    expect(orth_layer_forward_hip(&L, xbuf, ybuf, 0, ORTH_DT_F16, NULL), ORTH_OK, "batch 0");
    expect(orth_layer_forward_hip(&L, xbuf, ybuf, 2, ORTH_DT_F16, NULL), ORTH_ERR_NO_DEVICE, "no device");
    expect(orth_layer_forward_hip_planned(&L, qbuf, 1, xbuf, ybuf, 2, ORTH_DT_F16, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "short plan");
    expect(orth_layer_forward_hip_ex(&L, NULL, 0, sbuf, 9, xbuf, ybuf, 2, ORTH_DT_F16, NULL),
           ORTH_ERR_INVALID_ARGUMENT, "bias dtype");
    expect(orth_ortho_plan_build(&L, NULL, 0, NULL), ORTH_ERR_INVALID_ARGUMENT, "plan build NULL");
    expect(orth_layer_forward_hip_noalloc(&L, NULL, 0, NULL, 0, xbuf, ybuf, 2, ORTH_DT_F16, NULL), ORTH_ERR_NO_DEVICE,
           "noalloc no device");
    expect(orth_layer_forward_hip_noalloc(NULL, NULL, 0, NULL, 0, xbuf, ybuf, 2, ORTH_DT_F16, NULL),
           ORTH_ERR_INVALID_ARGUMENT, "noalloc NULL layer");
    if (orth_noalloc_scratch_bytes() != (int64_t)ORTH_NOALLOC_SCRATCH_BYTES) failures++;
    /* grouped forward: count, NULL arrays, overlapping outputs, batch 0 */
    {
        const orth_hip_layer_t *ls[2] = {&L, &L};
        void *outs[2] = {ybuf, ybuf};
        expect(orth_layers_forward_hip(ls, NULL, NULL, NULL, NULL, 0, xbuf, outs, 2, ORTH_DT_F16, NULL),
               ORTH_ERR_INVALID_ARGUMENT, "group count 0");
        expect(orth_layers_forward_hip(ls, NULL, NULL, NULL, NULL, ORTH_GROUP_MAX + 1, xbuf, outs, 2, ORTH_DT_F16,
                                       NULL), ORTH_ERR_INVALID_ARGUMENT, "group count above max");
        expect(orth_layers_forward_hip(NULL, NULL, NULL, NULL, NULL, 2, xbuf, outs, 2, ORTH_DT_F16, NULL),
               ORTH_ERR_INVALID_ARGUMENT, "group NULL layers");
        expect(orth_layers_forward_hip(ls, NULL, NULL, NULL, NULL, 2, xbuf, outs, 2, ORTH_DT_F16, NULL),
               ORTH_ERR_INVALID_ARGUMENT, "group overlapping outputs");
        outs[1] = zbuf;
        expect(orth_layers_forward_hip(ls, NULL, NULL, NULL, NULL, 2, xbuf, outs, 0, ORTH_DT_F16, NULL), ORTH_OK,
               "group batch 0");
        expect(orth_layers_forward_hip(ls, NULL, NULL, NULL, NULL, 2, xbuf, outs, 2, ORTH_DT_F16, NULL),
               ORTH_ERR_NO_DEVICE, "group no device");
    }
    expect(orth_base_dequant_hip(&L, NULL, NULL), ORTH_ERR_INVALID_ARGUMENT, "dequant NULL out");
    /* packing and sieve argument checks */
    expect(orth_pack_base_hip(NULL, ORTH_DT_F32, 4, 8, 8, NULL, 0, qbuf, sbuf, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "pack NULL w");
    expect(orth_pack_base_hip(xbuf, ORTH_DT_F32, 4, 7, 8, NULL, 0, qbuf, sbuf, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "pack odd K");
    expect(orth_pack_base_hip(xbuf, ORTH_DT_F32, 4, 8, 3, NULL, 0, qbuf, sbuf, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "pack group");
    expect(orth_pack_base_hip(xbuf, 5, 4, 8, 8, NULL, 0, qbuf, sbuf, NULL), ORTH_ERR_INVALID_ARGUMENT, "pack dtype");
    expect(orth_pack_csr_rows_hip(xbuf, ORTH_DT_F32, 4, 8, NULL, NULL, 0, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "csr rows NULL");
    expect(orth_pack_csr_rows_hip(xbuf, ORTH_DT_F32, 4, 8, rp, ybuf, 1, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "csr short mask");
    expect(orth_pack_csr_fill_hip(xbuf, ORTH_DT_F32, 4, 8, rp, NULL, 0, col, vals, 9, NULL),
           ORTH_ERR_INVALID_ARGUMENT, "csr fill dtype");
    expect(orth_sieve_quantize_hip(xbuf, ORTH_DT_F32, 4, 8, NULL, 0, NULL), ORTH_ERR_INVALID_ARGUMENT, "sieve NULL");
    expect(orth_sieve_quantize_hip(xbuf, ORTH_DT_F32, 4, 8, qbuf, 6, NULL), ORTH_ERR_INVALID_ARGUMENT, "sieve flags");
    expect(orth_sieve_split_hip(xbuf, ORTH_DT_F32, 4, 8, NULL, ORTH_DT_F32, 1, ORTH_DT_F32, 0, 0, 1.0f, qbuf, sbuf,
                                (float *)ybuf, NULL, 0, NULL), ORTH_ERR_INVALID_ARGUMENT, "split NULL h");
    expect(orth_sieve_split_hip(xbuf, ORTH_DT_F32, 4, 8, sbuf, ORTH_DT_F32, 1, ORTH_DT_F32, 1, 33, 1.0f, qbuf, sbuf,
                                (float *)ybuf, ybuf, ORTH_SIEVE_IEEE_DIV, NULL), ORTH_ERR_INVALID_ARGUMENT, "split rank");
    expect(orth_sieve_hdiag_hip(xbuf, ORTH_DT_F32, 4, 8, (float *)ybuf, 1, sbuf, 0, NULL), ORTH_ERR_INVALID_ARGUMENT,
           "hdiag workspace");
    expect(orth_hip_set_kernel_policy(9), ORTH_ERR_INVALID_ARGUMENT, "policy");
    expect(orth_hip_set_kernel_policy(0), ORTH_OK, "policy auto");
    orth_hip_device_info_t info;
    expect(orth_hip_device_info(0, NULL), ORTH_ERR_INVALID_ARGUMENT, "device info NULL");
    if (orth_hip_abi_version() < 100) failures++;
    /* per-thread error strings under concurrent calls */
    pthread_t th[4];
    for (int i = 0; i < 4; i++) pthread_create(&th[i], NULL, thread_main, NULL);
    for (int i = 0; i < 4; i++) pthread_join(th[i], NULL);
    (void)info;
    if (failures) {
        printf("%d failures\n", failures);
        return 1;
    }
    printf("capi ok\n");
    return 0;
}
