// Host-only stand-ins for the kernel launchers of libortho_amd, so that the
// C ABI's host side (orth_capi.hip: validation, dispatch, error reporting)
// can be built alone under AddressSanitizer and UBSan and driven on a
// machine without a GPU (tests/test_sanitizers.py).  Every launcher fails
// and every capability query says "no"; the driver only reaches them through
// paths that stop at the device check.
#include "orth_common.h"

namespace orth {
hipError_t launch_general(const ForwardArgs &, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_dequant(const ForwardArgs &, float *, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_pack_base(const void *, int, int64_t, int64_t, int64_t, const void *, int, uint8_t *, void *,
                            hipStream_t) { return hipErrorInvalidValue; }
int pack_base_path(const void *, int, int64_t, int64_t, const void *) { return 3; }
int64_t csr_mask_bytes(const void *, int, int64_t N, int64_t K) { return ((N * K + 31) / 32) * 4; }
hipError_t launch_csr_rows(const void *, int, int64_t, int64_t, int32_t *, void *, hipStream_t) {
    return hipErrorInvalidValue;
}
hipError_t launch_csr_fill(const void *, int, int64_t, int64_t, const int32_t *, const void *, int32_t *, void *, int,
                           hipStream_t) { return hipErrorInvalidValue; }
bool decode_supported(const ForwardArgs &) { return false; }
bool decode_bf16_supported(const ForwardArgs &, const void *) { return false; }
hipError_t launch_decode(const ForwardArgs &, const void *, int, hipStream_t) { return hipErrorInvalidValue; }
bool decode_group_ok(const ForwardArgs *, const void *const *, int) { return false; }
bool mid_supported(const ForwardArgs &, const void *) { return false; }
bool quarter_supported(const ForwardArgs &, const void *) { return false; }
int64_t quarter_workspace_bytes(const ForwardArgs &) { return 0; }
hipError_t launch_quarter(const ForwardArgs &, const void *, float *, hipStream_t) { return hipErrorInvalidValue; }
bool split_supported(const ForwardArgs &, const void *) { return false; }
bool prefill_wide_supported(const ForwardArgs &) { return false; }
bool prefill_wide_preferred(const ForwardArgs &, int) { return false; }
hipError_t launch_prefill_wide(const ForwardArgs &, const void *, hipStream_t, int) { return hipErrorInvalidValue; }
int64_t split_workspace_bytes(const ForwardArgs &) { return 0; }
hipError_t launch_split(const ForwardArgs &, const void *, float *, hipStream_t) { return hipErrorInvalidValue; }
bool split_group_ok(const ForwardArgs *, const void *const *, int) { return false; }
int64_t split_group_workspace_bytes(const ForwardArgs *, int) { return 0; }
hipError_t launch_split_group(const ForwardArgs *, const void *const *, int, float *, hipStream_t) {
    return hipErrorInvalidValue;
}
hipError_t launch_mid(const ForwardArgs &, const void *, int, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_decode_group(const ForwardArgs *, const void *const *, int, int, hipStream_t) {
    return hipErrorInvalidValue;
}
bool prefill_supported(const ForwardArgs &) { return false; }
bool plan_supported(const ForwardArgs &a) { return a.K % 64 == 0 && a.K <= 12288; }
int64_t plan_bytes_for(int64_t N, int64_t K, int64_t nnz) { return nnz > 0 ? 64 + 4 * nnz + N + K : 0; }
hipError_t launch_plan_build(const ForwardArgs &, void *, hipStream_t) { return hipErrorInvalidValue; }
int64_t plan_prefill_bytes(int64_t N, int64_t K, int64_t nnz) { return nnz > 0 ? 64 + 4 * nnz + N + K : 0; }
hipError_t launch_plan_build_prefill(const ForwardArgs &, void *, hipStream_t) { return hipErrorInvalidValue; }
hipError_t plan_read_flags(const void *, hipStream_t, uint32_t *) { return hipErrorInvalidValue; }
hipError_t launch_prefill(const ForwardArgs &, const void *, hipStream_t, float *, int) { return hipErrorInvalidValue; }
int prefill_ksplit(const ForwardArgs &, int) { return 1; }
hipError_t prefill_prepare_device() { return hipSuccess; }
hipError_t plan_prepare_device() { return hipSuccess; }
bool skinny_supported(const ForwardArgs &) { return false; }
int64_t skinny_workspace_bytes(const ForwardArgs &, int) { return 0; }
hipError_t launch_skinny(const ForwardArgs &, const void *, int, float *, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_sieve_quantize(const void *, int, int64_t, int64_t, void *, int, hipStream_t) {
    return hipErrorInvalidValue;
}
hipError_t launch_sieve_split(const void *, int, int64_t, int64_t, const void *, int, int64_t, int, int, int64_t, float,
                              void *, void *, float *, void *, int, hipStream_t) { return hipErrorInvalidValue; }
int64_t sieve_hdiag_slices(int64_t n) { return n < 64 ? (n > 0 ? n : 1) : 64; }
hipError_t launch_clock_stamp(uint64_t *, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_sieve_hdiag(const void *, int, int64_t, int64_t, float *, void *, int, hipStream_t) {
    return hipErrorInvalidValue;
}
}  // namespace orth
