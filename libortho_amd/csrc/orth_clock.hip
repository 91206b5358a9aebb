// Device clock stamps for measuring stream-ordered intervals on the GPU.
//
// A timed segment of K kernel launches is bracketed by two launches of
// clock_stamp_kernel: each of its workgroups reads the 100 MHz constant
// clock (s_memrealtime) as it starts and writes it with the id of the XCD
// it ran on.  The interval between two stamps taken on the same XCD covers
// the K launches and one launch gap, with no cache flush or host round trip
// in between (an event record can cost several microseconds at a segment's
// ends).  Not part of the forward path; no counterpart in the reference.
#include "orth_common.h"

namespace orth {

constexpr int kClockGroups = 8;  // one workgroup per XCD of an MI355X, usually

__global__ void __launch_bounds__(64) clock_stamp_kernel(uint64_t *dst) {
    if (threadIdx.x == 0) {
        const uint64_t t = __builtin_amdgcn_s_memrealtime();
        // HW_REG_XCC_ID (hardware register 20), bits [3:0]: the XCD
        const uint32_t xcc = __builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15u;
        dst[2 * blockIdx.x] = t;
        dst[2 * blockIdx.x + 1] = xcc;
    }
}

hipError_t launch_clock_stamp(uint64_t *dst, hipStream_t stream) {
    hipLaunchKernelGGL(clock_stamp_kernel, dim3(kClockGroups), dim3(64), 0, stream, dst);
    return hipGetLastError();
}

}  // namespace orth
