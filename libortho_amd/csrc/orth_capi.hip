// Host side of the C ABI declared in include/orth_hip.h: argument
// validation, kernel choice, temporary plans and error reporting.
//
// Replaces the reference's host wrappers /root/reference/src/dual_gemm.cu:295-372
// (which launch on the legacy default stream and synchronise the device on
// every call) and /root/reference/torch_bind/bindings.cpp:9-44 (which checks
// nothing and drops the return code).  Here every call is validated on the
// host, launched asynchronously on the caller's stream, and reported through
// a status code plus a per-thread message.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "orth_common.h"

namespace orth {
hipError_t launch_general(const ForwardArgs &a, hipStream_t stream);
hipError_t launch_dequant(const ForwardArgs &a, float *out, hipStream_t stream);
hipError_t launch_pack_base(const void *w, int wdt, int64_t N, int64_t K, int64_t G, const void *s_in,
                            int sdt, uint8_t *q, void *s_out, hipStream_t stream);
int pack_base_path(const void *w, int wdt, int64_t K, int64_t G, const void *q);
int64_t csr_mask_bytes(const void *w, int wdt, int64_t N, int64_t K);
hipError_t launch_csr_rows(const void *w, int wdt, int64_t N, int64_t K, int32_t *row_ptr, void *mask,
                           hipStream_t stream);
hipError_t launch_csr_fill(const void *w, int wdt, int64_t N, int64_t K, const int32_t *row_ptr,
                           const void *mask, int32_t *col, void *vals, int vdt, hipStream_t stream);
bool decode_supported(const ForwardArgs &a);
hipError_t launch_decode(const ForwardArgs &a, const void *plan, int cus, hipStream_t stream);
bool decode_group_ok(const ForwardArgs *as, const void *const *plans, int n);
hipError_t launch_decode_group(const ForwardArgs *as, const void *const *plans, int n, int cus, hipStream_t stream);
bool prefill_supported(const ForwardArgs &a);
bool decode_bf16_supported(const ForwardArgs &a, const void *plan);
bool plan_supported(const ForwardArgs &a);
int64_t plan_bytes_for(int64_t N, int64_t K, int64_t nnz);
hipError_t launch_plan_build(const ForwardArgs &a, void *plan, hipStream_t stream);
int64_t plan_prefill_bytes(int64_t N, int64_t K, int64_t nnz);
hipError_t launch_plan_build_prefill(const ForwardArgs &a, void *plan, hipStream_t stream);
hipError_t plan_read_flags(const void *plan, hipStream_t stream, uint32_t *flags);
hipError_t launch_prefill(const ForwardArgs &a, const void *plan, hipStream_t stream, float *part, int S);
int prefill_ksplit(const ForwardArgs &a, int cus);
bool prefill_wide_supported(const ForwardArgs &a);
bool prefill_wide_preferred(const ForwardArgs &a, int cus);
hipError_t launch_prefill_wide(const ForwardArgs &a, const void *plan, hipStream_t stream, int cus);
hipError_t prefill_prepare_device();
hipError_t plan_prepare_device();
bool mid_supported(const ForwardArgs &a, const void *plan);
bool quarter_supported(const ForwardArgs &a, const void *plan);
int64_t quarter_workspace_bytes(const ForwardArgs &a);
hipError_t launch_quarter(const ForwardArgs &a, const void *plan, float *part, hipStream_t stream);
bool split_supported(const ForwardArgs &a, const void *plan);
int64_t split_workspace_bytes(const ForwardArgs &a);
hipError_t launch_split(const ForwardArgs &a, const void *plan, float *part, hipStream_t stream);
bool split_group_ok(const ForwardArgs *as, const void *const *plans, int count);
int64_t split_group_workspace_bytes(const ForwardArgs *as, int count);
hipError_t launch_split_group(const ForwardArgs *as, const void *const *plans, int count, float *part,
                              hipStream_t stream);
hipError_t launch_mid(const ForwardArgs &a, const void *plan, int cus, hipStream_t stream);
bool skinny_supported(const ForwardArgs &a);
int64_t skinny_workspace_bytes(const ForwardArgs &a, int cus);
hipError_t launch_skinny(const ForwardArgs &a, const void *plan, int cus, float *part, hipStream_t stream);
hipError_t launch_sieve_quantize(const void *w, int dt, int64_t N, int64_t K, void *w_base, int ieee_div,
                                 hipStream_t stream);
hipError_t launch_sieve_split(const void *w, int dt, int64_t N, int64_t K, const void *h, int hdt, int64_t h_stride,
                              int score_dt, int use_rank, int64_t rank, float thresh, void *w_base, void *w_ortho,
                              float *score, void *sel, int ieee_div, hipStream_t stream);
int64_t sieve_hdiag_slices(int64_t n);
hipError_t launch_sieve_hdiag(const void *x, int dt, int64_t n, int64_t K, float *partial, void *out, int ieee_div,
                              hipStream_t stream);
hipError_t launch_clock_stamp(uint64_t *dst, hipStream_t stream);
}  // namespace orth

using namespace orth;

namespace {

thread_local std::string t_error;
thread_local int t_last_kernel = KERNEL_NONE;

int policy_from_env() {
    const char *e = std::getenv("ORTH_KERNEL_POLICY");
    if (!e) return 0;
    if (!std::strcmp(e, "decode")) return 1;
    if (!std::strcmp(e, "prefill")) return 2;
    if (!std::strcmp(e, "general")) return 3;
    if (!std::strcmp(e, "skinny")) return 4;
    if (!std::strcmp(e, "mid")) return 5;
    if (!std::strcmp(e, "quarter")) return 6;
    if (!std::strcmp(e, "split")) return 7;
    if (!std::strcmp(e, "prefill_wide")) return 8;
    return 0;
}

std::atomic<int> g_policy{policy_from_env()};

int fail(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    t_error = buf;
    return status;
}

int fail_hip(hipError_t e, const char *what) {
    return fail(ORTH_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

bool valid_dtype(int32_t d) { return d == ORTH_DT_F16 || d == ORTH_DT_BF16 || d == ORTH_DT_F32; }
int64_t dtype_size(int32_t d) { return d == ORTH_DT_F32 ? 4 : 2; }

// Validates a layer (and, when check_io, the activations) and fills args.
int resolve(const orth_hip_layer_t *L, const void *input, void *output, int64_t batch,
            int32_t io_dtype, bool check_io, ForwardArgs &a) {
    if (!L) return fail(ORTH_ERR_INVALID_ARGUMENT, "layer is NULL");
    const orth_hip_base_t &b = L->base;
    const orth_hip_ortho_t &o = L->ortho;
    if (!b.q_weight) return fail(ORTH_ERR_INVALID_ARGUMENT, "base.q_weight is NULL");
    if (!b.q_scales) return fail(ORTH_ERR_INVALID_ARGUMENT, "base.q_scales is NULL");
    if (b.q_bits != 4)
        return fail(ORTH_ERR_UNSUPPORTED, "base.q_bits is %d; only 4-bit weights are supported", b.q_bits);
    if (b.in_features <= 0 || (b.in_features & 1))
        return fail(ORTH_ERR_INVALID_ARGUMENT, "in_features must be positive and even (got %lld)",
                    (long long)b.in_features);
    if (b.out_features <= 0)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "out_features must be positive (got %lld)",
                    (long long)b.out_features);
    if (b.in_features > ((int64_t)1 << 40) / b.out_features)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "in_features * out_features is too large");
    if (b.scale_groups < 1 || b.in_features % b.scale_groups != 0)
        return fail(ORTH_ERR_INVALID_ARGUMENT,
                    "scale_groups (%lld) must be >= 1 and divide in_features (%lld)",
                    (long long)b.scale_groups, (long long)b.in_features);
    if (b.scale_dtype != ORTH_DT_F16 && b.scale_dtype != ORTH_DT_F32)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or F32 (got %d)", b.scale_dtype);
    if (o.count < 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "ortho.count is negative");
    if (o.count >= ((int64_t)1 << 31))
        return fail(ORTH_ERR_UNSUPPORTED, "ortho.count exceeds the int32 CSR index range");
    if (o.count > 0) {
        if (!o.row_ptr || !o.col_indices || !o.values)
            return fail(ORTH_ERR_INVALID_ARGUMENT, "ortho has %lld entries but a NULL CSR buffer",
                        (long long)o.count);
        if (o.value_dtype != ORTH_DT_F16 && o.value_dtype != ORTH_DT_F32)
            return fail(ORTH_ERR_INVALID_ARGUMENT, "ortho.value_dtype must be F16 or F32 (got %d)",
                        o.value_dtype);
    }
    if (check_io) {
        if (batch < 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "batch_size is negative");
        if (!valid_dtype(io_dtype))
            return fail(ORTH_ERR_INVALID_ARGUMENT, "io_dtype must be F16, BF16 or F32 (got %d)", io_dtype);
        if (batch > 0 && (!input || !output))
            return fail(ORTH_ERR_INVALID_ARGUMENT, "input or output is NULL");
        if (batch > ((int64_t)1 << 40) / b.in_features || batch > ((int64_t)1 << 40) / b.out_features)
            return fail(ORTH_ERR_INVALID_ARGUMENT, "batch_size is too large");
    }
    a.q = static_cast<const uint8_t *>(b.q_weight);
    a.scales = b.q_scales;
    a.scale_dtype = b.scale_dtype;
    a.ngroups = b.scale_groups;
    a.G = b.in_features / b.scale_groups;
    a.row_ptr = o.row_ptr;
    a.col = o.col_indices;
    a.vals = o.values;
    a.val_dtype = o.value_dtype;
    a.nnz = o.count;
    a.x = input;
    a.y = output;
    a.io_dtype = io_dtype;
    a.M = batch;
    a.K = b.in_features;
    a.N = b.out_features;
    a.alpha = L->alpha;
    // the reference's gate: alpha > 0 && count > 0 (src/ortho.c:343); NaN -> off
    a.has_ortho = (L->alpha > 0.0f && o.count > 0) ? 1 : 0;
    t_error.clear();
    return ORTH_OK;
}

// Scratch memory of orth_layer_forward_hip_noalloc: one array per device
// (each GPU holds its own copy for the life of the process).  Host code
// never passes the array's name to a kernel: that is a host-side stand-in,
// not a device address.  Its device address is looked up once per device
// (hipGetSymbolAddress, in the device set-up below) and only that pointer
// is used.
static __device__ __align__(256) unsigned char scratch[ORTH_NOALLOC_SCRATCH_BYTES];

// Per-device check that the current device is a gfx950 (the only code object
// this library carries), one-time kernel attribute set-up, and the device
// address of the scratch array.
struct DeviceState {
    std::atomic<int> checked{0};  // 0 unknown, 1 ok, -1 not gfx950 (published after the fields below)
    int cus = 256;
    char arch[64] = {0};
    void *scratch = nullptr;      // device address of this device's scratch array
    // the last no-allocation call's completion on this device (recorded on
    // its stream), so that a call on another stream waits for it before it
    // touches the scratch array
    hipEvent_t noalloc_done = nullptr;
    hipStream_t noalloc_stream = nullptr;
    bool noalloc_recorded = false;
    std::mutex noalloc_mu;
};
std::mutex g_dev_mu;
DeviceState g_dev[64];

int current_device_ok(int *dev_out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(ORTH_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return fail(ORTH_ERR_NO_DEVICE, "device index %d out of range", dev);
    if (dev_out) *dev_out = dev;
    DeviceState &st = g_dev[dev];
    if (st.checked.load(std::memory_order_acquire) == 0) {
        std::lock_guard<std::mutex> lk(g_dev_mu);
        if (st.checked.load(std::memory_order_relaxed) == 0) {
            hipDeviceProp_t p;
            e = hipGetDeviceProperties(&p, dev);
            if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
            std::snprintf(st.arch, sizeof(st.arch), "%s", p.gcnArchName);
            st.cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
            const bool ok = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
            if (ok) {
                e = prefill_prepare_device();
                if (e == hipSuccess) e = plan_prepare_device();
                if (e != hipSuccess) return fail_hip(e, "kernel attribute set-up");
                void *ptr = nullptr;
                e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
                if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress (scratch)");
                st.scratch = ptr;
                e = hipEventCreateWithFlags(&st.noalloc_done, hipEventDisableTiming);
                if (e != hipSuccess) return fail_hip(e, "hipEventCreateWithFlags (no-allocation ordering)");
            }
            st.checked.store(ok ? 1 : -1, std::memory_order_release);
        }
    }
    if (st.checked.load(std::memory_order_acquire) < 0)
        return fail(ORTH_ERR_NO_DEVICE, "device %d is %s; this library carries gfx950 code only", dev,
                    st.arch);
    return ORTH_OK;
}

// Split-K workspace of the mid-batch kernels, one per (device, stream): the
// FP32 partials their reduction kernel sums.  Calls on one stream are
// ordered; calls on different streams use different workspaces.  Allocation
// happens on first use (and on growth), outside graph capture only.
//
// A captured call records no allocation: its partials (or the temporary
// plan of an unplanned prefill call) go to the device's scratch array when
// they fit it, else to the capturing stream's capture buffer, which eager
// calls on that stream size (allocated only for requests larger than the
// scratch array), else the call is refused.  Eager calls never touch either,
// so a graph replayed on any stream, beside eager calls on any stream, does
// not race with them; replays of graphs that overlap one another, or
// no-allocation calls, on the same GPU share that memory and must be
// ordered by the caller.
struct Workspace {
    void *buf = nullptr;
    int64_t part_bytes = 0;
    void *cap = nullptr;  // capture buffer
    int64_t cap_bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, void *>, Workspace> g_ws;
std::vector<void *> g_ws_retired;

int capturing(hipStream_t stream, bool *cap) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return fail_hip(e, "hipStreamIsCapturing");
    *cap = cs != hipStreamCaptureStatusNone;
    return ORTH_OK;
}

// Memory for a captured call (see above): *out, or ORTH_ERR_UNSUPPORTED.
int capture_memory(int dev, hipStream_t stream, int64_t bytes, const char *what, void **out) {
    if (bytes <= (int64_t)ORTH_NOALLOC_SCRATCH_BYTES) {
        *out = g_dev[dev].scratch;
        return ORTH_OK;
    }
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws.find({dev, static_cast<void *>(stream)});
    if (it != g_ws.end() && it->second.cap && it->second.cap_bytes >= bytes) {
        *out = it->second.cap;
        return ORTH_OK;
    }
    return fail(ORTH_ERR_UNSUPPORTED,
                "a captured call needs %lld bytes of %s, more than the %lld-byte scratch array; run the same call "
                "once outside capture on the capturing stream first (it sizes that stream's capture buffer)",
                (long long)bytes, what, (long long)ORTH_NOALLOC_SCRATCH_BYTES);
}

int workspace_for(int dev, hipStream_t stream, int64_t part_bytes, float **part) {
    bool cap = false;
    int rc = capturing(stream, &cap);
    if (rc != ORTH_OK) return rc;
    if (cap) {
        void *p = nullptr;
        rc = capture_memory(dev, stream, part_bytes, "split-K workspace", &p);
        *part = static_cast<float *>(p);
        return rc;
    }
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace &w = g_ws[{dev, static_cast<void *>(stream)}];
    hipError_t e = hipSuccess;
    if (part_bytes > (int64_t)ORTH_NOALLOC_SCRATCH_BYTES && w.cap_bytes < part_bytes) {
        // a capture of this call on this stream will find a buffer (an older,
        // smaller one is retired: graphs captured earlier may still use it)
        if (w.cap) g_ws_retired.push_back(w.cap);
        w.cap = nullptr;
        w.cap_bytes = 0;
        e = hipMalloc(&w.cap, (size_t)part_bytes);
        if (e != hipSuccess) return fail_hip(e, "hipMalloc (capture buffer)");
        w.cap_bytes = part_bytes;
    }
    if (w.buf && w.part_bytes >= part_bytes) {
        *part = static_cast<float *>(w.buf);
        return ORTH_OK;
    }
    if (w.buf) {
        // a smaller buffer is retired, not freed: in-flight work may still use it
        g_ws_retired.push_back(w.buf);
        w.buf = nullptr;
        w.part_bytes = 0;
    }
    e = hipMalloc(&w.buf, (size_t)part_bytes);
    if (e != hipSuccess) return fail_hip(e, "hipMalloc (mid-batch workspace)");
    w.part_bytes = part_bytes;
    *part = static_cast<float *>(w.buf);
    return ORTH_OK;
}

// The K split of a 256 x 128 prefill call: only with a plan or without an
// ortho term (an unplanned call's temporary plan would share the scratch
// array with the partials under capture and in no-allocation calls).
int prefill_split(const ForwardArgs &a, const void *plan, int cus) {
    return !a.has_ortho || plan ? prefill_ksplit(a, cus) : 1;
}

// The kernel a forward call takes under `policy` (orth_hip_set_kernel_policy).
int pick_kernel(const ForwardArgs &a, const void *plan, int policy, int cus, int *kernel) {
    const bool dec_ok = decode_supported(a) || decode_bf16_supported(a, a.has_ortho ? plan : nullptr);
    const bool pre_ok = prefill_supported(a);
    // the mid-batch kernel reads each row's ortho entries through the plan;
    // without one it filters whole rows by column, which still beats the
    // decode kernel from 9 tokens (c2: 26.5 against 29.2 us at 12 tokens,
    // 26.7 against 33.9 at 16) but not up to 8 (21.7 against 19.3-21.0)
    const bool sk_ok = skinny_supported(a);
    const bool sk_pref = sk_ok && (plan || !a.has_ortho || !dec_ok || a.M > 8);
    const bool mid_ok = mid_supported(a, a.has_ortho ? plan : nullptr);
    const bool qu_ok = quarter_supported(a, a.has_ortho ? plan : nullptr);
    const bool sp_ok = split_supported(a, a.has_ortho ? plan : nullptr);
    switch (policy) {
        case 1:
            if (!dec_ok) return fail(ORTH_ERR_UNSUPPORTED, "decode kernel forced but it cannot take this call");
            *kernel = KERNEL_DECODE;
            break;
        case 2:
            if (!pre_ok) return fail(ORTH_ERR_UNSUPPORTED, "prefill kernel forced but it cannot take this call");
            *kernel = KERNEL_PREFILL;
            break;
        case 3:
            *kernel = KERNEL_GENERAL;
            break;
        case 4:
            if (!sk_ok) return fail(ORTH_ERR_UNSUPPORTED, "mid-batch kernel forced but it cannot take this call");
            *kernel = KERNEL_SKINNY;
            break;
        case 5:
            if (!mid_ok) return fail(ORTH_ERR_UNSUPPORTED, "one-launch mid-batch kernel forced but it cannot take this call");
            *kernel = KERNEL_MID;
            break;
        case 6:
            if (!qu_ok) return fail(ORTH_ERR_UNSUPPORTED, "quarter-split kernel forced but it cannot take this call");
            *kernel = KERNEL_QUARTER;
            break;
        case 7:
            if (!sp_ok) return fail(ORTH_ERR_UNSUPPORTED, "slice-split kernel forced but it cannot take this call");
            *kernel = KERNEL_SPLIT;
            break;
        case 8:
            if (!prefill_wide_supported(a))
                return fail(ORTH_ERR_UNSUPPORTED, "wide-row prefill kernel forced but it cannot take this call");
            *kernel = KERNEL_PREFILL_WIDE;
            break;
        default:
            // the one-launch mid-batch kernel beats the split-K one on every
            // shape both take (c2 M=8 alpha=1 10.3 against 14.4 us, M=16
            // 13.6 against 16.6, 4096x4096 M=16 8.2 against 12.2)
            if (dec_ok && a.M <= 4) *kernel = KERNEL_DECODE;
            else if (mid_ok) *kernel = KERNEL_MID;
            else if (qu_ok) *kernel = KERNEL_QUARTER;
            // 17..32 tokens where the quarter-split kernel cannot go (K != 4096,
            // BF16 with 512-word records): c5 down_proj M=32 23.7 against
            // 35.5 us for the split-K kernel
            else if (sp_ok && a.M > 16) *kernel = KERNEL_SPLIT;
            // 33..64 tokens at K > 4096: the prefill kernel with K split
            // over the grid (c5 down_proj, K = 11008: 35-37 against 44-53
            // us on the split-K kernel at 33-64 tokens; at K = 4096 the
            // split-K kernel is level or ahead: c2 M=48 35.8 against 42.4)
            else if (pre_ok && a.M > 32 && a.K > 4096 && prefill_split(a, plan, cus) > 1) *kernel = KERNEL_PREFILL;
            else if (sk_pref) *kernel = KERNEL_SKINNY;
            else if (dec_ok) *kernel = KERNEL_DECODE;
            // (the 256 x 128 kernel where it splits K: c3 at 512 or 1024
            // tokens, where the tile grid alone leaves CUs idle)
            else if (pre_ok && a.M > 16)
                *kernel = prefill_split(a, plan, cus) == 1 && prefill_wide_preferred(a, cus) ? KERNEL_PREFILL_WIDE
                                                                                             : KERNEL_PREFILL;
            else *kernel = KERNEL_GENERAL;
    }
    return ORTH_OK;
}

int launch_kernel(const ForwardArgs &a, const void *plan, int kernel, int dev, hipStream_t stream, bool noalloc);

// noalloc: scratch from the device's scratch array instead of the stream's
// workspace or stream-ordered allocations (orth_layer_forward_hip_noalloc).
int forward_impl(const orth_hip_layer_t *layer, const void *plan, int64_t plan_bytes,
                 const void *input, void *output, int64_t batch, int32_t io_dtype, void *stream_v,
                 const void *bias = nullptr, int32_t bias_dtype = ORTH_DT_F32, bool noalloc = false) {
    ForwardArgs a;
    int rc = resolve(layer, input, output, batch, io_dtype, true, a);
    if (rc != ORTH_OK) return rc;
    if (bias && !valid_dtype(bias_dtype))
        return fail(ORTH_ERR_INVALID_ARGUMENT, "bias dtype %d is not F16, BF16 or F32", bias_dtype);
    a.bias = bias;
    a.bias_dtype = bias_dtype;
    if (plan && plan_bytes < plan_bytes_for(a.N, a.K, a.nnz))
        return fail(ORTH_ERR_INVALID_ARGUMENT, "plan_bytes %lld is smaller than the plan size %lld",
                    (long long)plan_bytes, (long long)plan_bytes_for(a.N, a.K, a.nnz));
    if (batch == 0) {
        t_last_kernel = KERNEL_NONE;
        return ORTH_OK;
    }
    int dev = 0;
    rc = current_device_ok(&dev);
    if (rc != ORTH_OK) return rc;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);

    int kernel = KERNEL_NONE;
    rc = pick_kernel(a, plan, g_policy.load(std::memory_order_relaxed), g_dev[dev].cus, &kernel);
    if (rc != ORTH_OK) return rc;

    // No-allocation calls share the device's scratch array: a call on a
    // stream other than the last one's first waits for that call (its
    // completion event), and records its own completion after its launches.
    // The lock keeps wait, launches and record of one call together when
    // several host threads call at once.  A stream under graph capture is not
    // ordered this way (a captured wait on an event recorded outside the
    // capture is not allowed): calls captured into graphs on one GPU must be
    // ordered by the caller.
    std::unique_lock<std::mutex> noalloc_lk;
    bool noalloc_order = false;
    if (noalloc) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t ce = hipStreamIsCapturing(stream, &cs);
        if (ce != hipSuccess) return fail_hip(ce, "hipStreamIsCapturing");
        noalloc_order = cs == hipStreamCaptureStatusNone;
        if (noalloc_order) {
            DeviceState &st = g_dev[dev];
            noalloc_lk = std::unique_lock<std::mutex>(st.noalloc_mu);
            if (st.noalloc_recorded && st.noalloc_stream != stream) {
                ce = hipStreamWaitEvent(stream, st.noalloc_done, 0);
                if (ce != hipSuccess) return fail_hip(ce, "hipStreamWaitEvent (no-allocation ordering)");
            }
        }
    }
    rc = launch_kernel(a, plan, kernel, dev, stream, noalloc);
    if (noalloc_order && rc == ORTH_OK) {
        DeviceState &st = g_dev[dev];
        hipError_t ce = hipEventRecord(st.noalloc_done, stream);
        if (ce != hipSuccess) return fail_hip(ce, "hipEventRecord (no-allocation ordering)");
        st.noalloc_stream = stream;
        st.noalloc_recorded = true;
    }
    if (rc != ORTH_OK) return rc;
    t_last_kernel = kernel;
    return ORTH_OK;
}

// The launches of one forward call with the kernel already chosen.
int launch_kernel(const ForwardArgs &a, const void *plan, int kernel, int dev, hipStream_t stream, bool noalloc) {
    int rc = ORTH_OK;
    hipError_t e = hipSuccess;
    if (kernel == KERNEL_DECODE) {
        e = launch_decode(a, plan, g_dev[dev].cus, stream);
    } else if (kernel == KERNEL_MID) {
        e = launch_mid(a, a.has_ortho ? plan : nullptr, g_dev[dev].cus, stream);
    } else if (kernel == KERNEL_SKINNY || kernel == KERNEL_QUARTER || kernel == KERNEL_SPLIT) {
        const int cus = g_dev[dev].cus;
        const bool qk = kernel == KERNEL_QUARTER, sk = kernel == KERNEL_SPLIT;
        const int64_t pbytes = qk ? quarter_workspace_bytes(a) : sk ? split_workspace_bytes(a) : skinny_workspace_bytes(a, cus);
        float *part = nullptr;
        if (pbytes > 0 && noalloc) {
            if (pbytes > (int64_t)ORTH_NOALLOC_SCRATCH_BYTES)
                return fail(ORTH_ERR_UNSUPPORTED,
                            "the %s kernel needs %lld bytes of scratch for this call; the no-allocation "
                            "entry point has %lld", qk ? "quarter-split" : sk ? "slice-split" : "mid-batch", (long long)pbytes,
                            (long long)ORTH_NOALLOC_SCRATCH_BYTES);
            part = static_cast<float *>(g_dev[dev].scratch);
        } else if (pbytes > 0) {
            rc = workspace_for(dev, stream, pbytes, &part);
            if (rc != ORTH_OK) return rc;
        }
        // without a plan the split-K kernel filters each row's CSR by column
        e = qk ? launch_quarter(a, a.has_ortho ? plan : nullptr, part, stream)
            : sk ? launch_split(a, a.has_ortho ? plan : nullptr, part, stream)
                 : launch_skinny(a, a.has_ortho ? plan : nullptr, cus, part, stream);
    } else if (kernel == KERNEL_PREFILL && prefill_split(a, plan, g_dev[dev].cus) > 1) {
        // K split: FP32 partials in the stream's workspace, or the scratch
        // array (prefill_ksplit keeps them within it)
        const int S = prefill_split(a, plan, g_dev[dev].cus);
        const int64_t pbytes = (int64_t)S * a.M * a.N * 4;
        float *part = nullptr;
        if (noalloc) {
            if (pbytes > (int64_t)ORTH_NOALLOC_SCRATCH_BYTES)
                return fail(ORTH_ERR_UNSUPPORTED, "prefill K split needs %lld bytes of scratch", (long long)pbytes);
            part = static_cast<float *>(g_dev[dev].scratch);
        } else {
            rc = workspace_for(dev, stream, pbytes, &part);
            if (rc != ORTH_OK) return rc;
        }
        e = launch_prefill(a, a.has_ortho ? plan : nullptr, stream, part, S);
    } else if (kernel == KERNEL_PREFILL || kernel == KERNEL_PREFILL_WIDE) {
        auto pf = [&](const void *p) {
            return kernel == KERNEL_PREFILL_WIDE ? launch_prefill_wide(a, p, stream, g_dev[dev].cus)
                                                 : launch_prefill(a, p, stream, nullptr, 1);
        };
        if (a.has_ortho && !plan && noalloc) {
            // the prefill part of a plan, built in the scratch array
            const int64_t pb = plan_prefill_bytes(a.N, a.K, a.nnz);
            if (pb > (int64_t)ORTH_NOALLOC_SCRATCH_BYTES)
                return fail(ORTH_ERR_UNSUPPORTED,
                            "the prefill kernel needs a %lld-byte ortho plan for this layer; the no-allocation "
                            "entry point has %lld bytes of scratch (pass a plan from orth_ortho_plan_build)",
                            (long long)pb, (long long)ORTH_NOALLOC_SCRATCH_BYTES);
            e = launch_plan_build_prefill(a, g_dev[dev].scratch, stream);
            if (e == hipSuccess) e = pf(g_dev[dev].scratch);
        } else if (a.has_ortho && !plan) {
            // temporary plan (its prefill part).  Under capture: in the
            // memory of captured calls (no allocation is recorded).  Else
            // stream-ordered: allocated, built, used and freed in stream
            // order, so the call stays asynchronous.
            const int64_t pb = plan_prefill_bytes(a.N, a.K, a.nnz);
            bool cap = false;
            rc = capturing(stream, &cap);
            if (rc != ORTH_OK) return rc;
            if (cap) {
                void *p = nullptr;
                rc = capture_memory(dev, stream, pb, "temporary ortho plan (pass a plan to capture this call)", &p);
                if (rc != ORTH_OK) return rc;
                e = launch_plan_build_prefill(a, p, stream);
                if (e == hipSuccess) e = pf(p);
                if (e != hipSuccess) return fail_hip(e, "kernel launch");
                return ORTH_OK;
            }
            void *tmp = nullptr;
            e = hipMallocAsync(&tmp, (size_t)pb, stream);
            if (e != hipSuccess) return fail_hip(e, "hipMallocAsync (temporary ortho plan)");
            e = launch_plan_build_prefill(a, tmp, stream);
            if (e == hipSuccess) e = pf(tmp);
            hipError_t f = hipFreeAsync(tmp, stream);
            if (e == hipSuccess) e = f;
        } else {
            e = pf(a.has_ortho ? plan : nullptr);
        }
    } else {
        e = launch_general(a, stream);
    }
    if (e != hipSuccess) return fail_hip(e, "kernel launch");
    return rc;
}

// Layers that read one input: a single decode launch when every layer takes
// the decode kernel and they share its instantiation (decode_group_ok),
// else one forward_impl call per layer.
int group_forward_impl(const orth_hip_layer_t *const *layers, const void *const *plans, const int64_t *plan_bytes,
                       const void *const *biases, const int32_t *bias_dtypes, int32_t count, const void *input,
                       void *const *outputs, int64_t batch, int32_t io_dtype, void *stream_v) {
    if (count < 1 || count > ORTH_GROUP_MAX)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "count %d is outside 1..%d", (int)count, (int)ORTH_GROUP_MAX);
    if (!layers || !outputs) return fail(ORTH_ERR_INVALID_ARGUMENT, "layers and outputs must not be NULL");
    ForwardArgs as[ORTH_GROUP_MAX];
    const void *pl[ORTH_GROUP_MAX];
    for (int l = 0; l < count; l++) {
        int rc = resolve(layers[l], input, outputs[l], batch, io_dtype, true, as[l]);
        if (rc != ORTH_OK) return rc;
        const void *bias = biases ? biases[l] : nullptr;
        const int32_t bdt = bias_dtypes ? bias_dtypes[l] : ORTH_DT_F32;
        if (bias && !valid_dtype(bdt))
            return fail(ORTH_ERR_INVALID_ARGUMENT, "bias %d dtype %d is not F16, BF16 or F32", l, (int)bdt);
        as[l].bias = bias;
        as[l].bias_dtype = bdt;
        pl[l] = plans ? plans[l] : nullptr;
        if (pl[l] && (!plan_bytes || plan_bytes[l] < plan_bytes_for(as[l].N, as[l].K, as[l].nnz)))
            return fail(ORTH_ERR_INVALID_ARGUMENT, "plan %d is smaller than the plan size %lld", l,
                        (long long)plan_bytes_for(as[l].N, as[l].K, as[l].nnz));
        // outputs written by one launch must not overlap each other
        const int64_t esz = dtype_size(io_dtype);
        const char *b0 = static_cast<const char *>(outputs[l]);
        for (int j = 0; j < l; j++) {
            const char *b1 = static_cast<const char *>(outputs[j]);
            if (batch > 0 && b0 < b1 + batch * as[j].N * esz && b1 < b0 + batch * as[l].N * esz)
                return fail(ORTH_ERR_INVALID_ARGUMENT, "outputs %d and %d overlap", j, l);
        }
    }
    if (batch == 0) {
        t_last_kernel = KERNEL_NONE;
        return ORTH_OK;
    }
    int dev = 0;
    int rc = current_device_ok(&dev);
    if (rc != ORTH_OK) return rc;
    bool grouped = count > 1;
    const int policy = g_policy.load(std::memory_order_relaxed);
    for (int l = 0; l < count && grouped; l++) {
        int kernel = KERNEL_NONE;
        rc = pick_kernel(as[l], pl[l], policy, g_dev[dev].cus, &kernel);
        if (rc != ORTH_OK) return rc;
        grouped = kernel == KERNEL_DECODE;
    }
    if (grouped && decode_group_ok(as, pl, count)) {
        hipError_t e = launch_decode_group(as, pl, count, g_dev[dev].cus, static_cast<hipStream_t>(stream_v));
        if (e != hipSuccess) return fail_hip(e, "kernel launch");
        t_last_kernel = KERNEL_DECODE_GROUP;
        return ORTH_OK;
    }
    // 17..32 tokens: one slice-split launch (and one reduction) for layers
    // that each take a kernel of that range, when they share the launch's
    // shape class (c5 q/k/v M=32: one launch instead of three)
    bool split_all = count > 1 && (policy == 0 || policy == 7) && as[0].M > 16;
    for (int l = 0; l < count && split_all; l++) {
        int kernel = KERNEL_NONE;
        rc = pick_kernel(as[l], pl[l], policy, g_dev[dev].cus, &kernel);
        if (rc != ORTH_OK) return rc;
        split_all = kernel == KERNEL_QUARTER || kernel == KERNEL_SPLIT;
    }
    if (split_all) {
        const void *spl[ORTH_GROUP_MAX];
        for (int l = 0; l < count; l++) spl[l] = as[l].has_ortho ? pl[l] : nullptr;
        if (split_group_ok(as, spl, count)) {
            hipStream_t stream = static_cast<hipStream_t>(stream_v);
            const int64_t pbytes = split_group_workspace_bytes(as, count);
            float *part = nullptr;
            if (pbytes > 0) {
                rc = workspace_for(dev, stream, pbytes, &part);
                if (rc != ORTH_OK) return rc;
            }
            hipError_t e = launch_split_group(as, spl, count, part, stream);
            if (e != hipSuccess) return fail_hip(e, "kernel launch");
            t_last_kernel = KERNEL_SPLIT_GROUP;
            return ORTH_OK;
        }
    }
    for (int l = 0; l < count; l++) {
        rc = forward_impl(layers[l], pl[l], pl[l] ? plan_bytes[l] : 0, input, outputs[l], batch, io_dtype, stream_v,
                          as[l].bias, as[l].bias_dtype);
        if (rc != ORTH_OK) return rc;
    }
    return ORTH_OK;
}

}  // namespace

extern "C" {

void orth_layer_hip_set_alpha(orth_hip_layer_t *layer, float alpha) {
    if (layer) layer->alpha = alpha;
}

int orth_layer_check_hip(const orth_hip_layer_t *layer, const void *input, void *output,
                         int64_t batch_size, int32_t io_dtype) {
    ForwardArgs a;
    return resolve(layer, input, output, batch_size, io_dtype, true, a);
}

int orth_layer_forward_hip(const orth_hip_layer_t *layer, const void *input, void *output,
                           int64_t batch_size, int32_t io_dtype, void *stream) {
    return forward_impl(layer, nullptr, 0, input, output, batch_size, io_dtype, stream);
}

int orth_layer_forward_hip_planned(const orth_hip_layer_t *layer, const void *plan,
                                   int64_t plan_bytes, const void *input, void *output,
                                   int64_t batch_size, int32_t io_dtype, void *stream) {
    return forward_impl(layer, plan, plan_bytes, input, output, batch_size, io_dtype, stream);
}

int orth_layer_forward_hip_ex(const orth_hip_layer_t *layer, const void *plan, int64_t plan_bytes,
                              const void *bias, int32_t bias_dtype, const void *input, void *output,
                              int64_t batch_size, int32_t io_dtype, void *stream) {
    return forward_impl(layer, plan, plan_bytes, input, output, batch_size, io_dtype, stream, bias,
                        bias_dtype);
}

int orth_layer_forward_hip_noalloc(const orth_hip_layer_t *layer, const void *plan, int64_t plan_bytes,
                                   const void *bias, int32_t bias_dtype, const void *input, void *output,
                                   int64_t batch_size, int32_t io_dtype, void *stream) {
    return forward_impl(layer, plan, plan_bytes, input, output, batch_size, io_dtype, stream, bias, bias_dtype,
                        true);
}

int64_t orth_noalloc_scratch_bytes(void) { return (int64_t)ORTH_NOALLOC_SCRATCH_BYTES; }

int orth_layers_forward_hip(const orth_hip_layer_t *const *layers, const void *const *plans,
                            const int64_t *plan_bytes, const void *const *biases, const int32_t *bias_dtypes,
                            int32_t count, const void *input, void *const *outputs, int64_t batch_size,
                            int32_t io_dtype, void *stream) {
    return group_forward_impl(layers, plans, plan_bytes, biases, bias_dtypes, count, input, outputs, batch_size,
                              io_dtype, stream);
}

int64_t orth_ortho_plan_bytes(const orth_hip_layer_t *layer) {
    ForwardArgs a;
    int rc = resolve(layer, nullptr, nullptr, 0, ORTH_DT_F16, false, a);
    if (rc != ORTH_OK) return -rc;
    if (a.nnz > 0 && !plan_supported(a))
        return -(int64_t)fail(ORTH_ERR_UNSUPPORTED,
                              "no ortho plan for in_features %lld (needs a multiple of 64, at most 12288)",
                              (long long)a.K);
    return plan_bytes_for(a.N, a.K, a.nnz);
}

int orth_ortho_plan_build(const orth_hip_layer_t *layer, void *plan, int64_t plan_bytes,
                          void *stream_v) {
    ForwardArgs a;
    int rc = resolve(layer, nullptr, nullptr, 0, ORTH_DT_F16, false, a);
    if (rc != ORTH_OK) return rc;
    if (a.nnz == 0) return ORTH_OK;
    if (!plan_supported(a))
        return fail(ORTH_ERR_UNSUPPORTED, "no ortho plan for in_features %lld", (long long)a.K);
    if (!plan) return fail(ORTH_ERR_INVALID_ARGUMENT, "plan is NULL");
    if (plan_bytes < plan_bytes_for(a.N, a.K, a.nnz))
        return fail(ORTH_ERR_INVALID_ARGUMENT, "plan_bytes %lld is smaller than the plan size %lld",
                    (long long)plan_bytes, (long long)plan_bytes_for(a.N, a.K, a.nnz));
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    hipError_t e = launch_plan_build(a, plan, stream);
    if (e != hipSuccess) return fail_hip(e, "plan build launch");
    uint32_t flags = 0;
    e = plan_read_flags(plan, stream, &flags);
    if (e != hipSuccess) return fail_hip(e, "plan build");
    if (flags & 2u)
        return fail(ORTH_ERR_INVALID_ARGUMENT,
                    "ortho.row_ptr is not monotone within [0, count] (malformed CSR)");
    return ORTH_OK;
}

int orth_base_dequant_hip(const orth_hip_layer_t *layer, float *out, void *stream) {
    ForwardArgs a;
    int rc = resolve(layer, nullptr, nullptr, 0, ORTH_DT_F16, false, a);
    if (rc != ORTH_OK) return rc;
    if (!out) return fail(ORTH_ERR_INVALID_ARGUMENT, "out is NULL");
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_dequant(a, out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "dequant launch");
    return ORTH_OK;
}

namespace {
int check_pack_dims(const void *w, int32_t w_dtype, int64_t N, int64_t K) {
    if (!w) return fail(ORTH_ERR_INVALID_ARGUMENT, "weights pointer is NULL");
    if (!valid_dtype(w_dtype)) return fail(ORTH_ERR_INVALID_ARGUMENT, "weight dtype %d is not F16, BF16 or F32", w_dtype);
    if (N <= 0 || K <= 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "out_features and in_features must be positive");
    if (K > ((int64_t)1 << 40) / N) return fail(ORTH_ERR_INVALID_ARGUMENT, "in_features * out_features is too large");
    return ORTH_OK;
}
}  // namespace

int orth_pack_base_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                       int64_t group_size, const void *scales_in, int32_t scales_in_dtype, void *q_out,
                       void *scales_out, void *stream) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return rc;
    const int64_t K = in_features;
    if (K & 1) return fail(ORTH_ERR_INVALID_ARGUMENT, "in_features must be even (got %lld)", (long long)K);
    const int64_t G = group_size <= 0 ? K : group_size;
    if ((G & 1) || K % G != 0)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "group_size (%lld) must be even and divide in_features (%lld)",
                    (long long)G, (long long)K);
    if (!q_out || !scales_out) return fail(ORTH_ERR_INVALID_ARGUMENT, "q_out or scales_out is NULL");
    if (scales_in && !valid_dtype(scales_in_dtype))
        return fail(ORTH_ERR_INVALID_ARGUMENT, "scales_in dtype %d is not F16, BF16 or F32", scales_in_dtype);
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_pack_base(w, w_dtype, out_features, K, G, scales_in, scales_in_dtype,
                                    static_cast<uint8_t *>(q_out), scales_out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "base packing launch");
    return ORTH_OK;
}

int orth_pack_base_path(const void *w, int32_t w_dtype, int64_t in_features, int64_t group_size,
                        const void *q_out) {
    const int64_t G = group_size <= 0 ? in_features : group_size;
    return pack_base_path(w, w_dtype, in_features, G, q_out);
}

int64_t orth_pack_csr_mask_bytes(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return -rc;
    return csr_mask_bytes(w, w_dtype, out_features, in_features);
}

namespace {
int check_mask(const void *w, int32_t w_dtype, int64_t N, int64_t K, const void *mask, int64_t mask_bytes) {
    if (!mask) return ORTH_OK;
    const int64_t need = csr_mask_bytes(w, w_dtype, N, K);
    if (need == 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "no nonzero mask for these weights (pass NULL)");
    if (mask_bytes < need)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "mask_bytes %lld is smaller than %lld", (long long)mask_bytes,
                    (long long)need);
    return ORTH_OK;
}
}  // namespace

int orth_pack_csr_rows_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                           int32_t *row_ptr, void *mask, int64_t mask_bytes, void *stream) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return rc;
    if (!row_ptr) return fail(ORTH_ERR_INVALID_ARGUMENT, "row_ptr is NULL");
    rc = check_mask(w, w_dtype, out_features, in_features, mask, mask_bytes);
    if (rc != ORTH_OK) return rc;
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_csr_rows(w, w_dtype, out_features, in_features, row_ptr, mask,
                                   static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "CSR row count launch");
    return ORTH_OK;
}

int orth_pack_csr_fill_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                           const int32_t *row_ptr, const void *mask, int64_t mask_bytes, int32_t *col_out,
                           void *values_out, int32_t value_dtype, void *stream) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return rc;
    if (!row_ptr) return fail(ORTH_ERR_INVALID_ARGUMENT, "row_ptr is NULL");
    rc = check_mask(w, w_dtype, out_features, in_features, mask, mask_bytes);
    if (rc != ORTH_OK) return rc;
    if (!valid_dtype(value_dtype)) return fail(ORTH_ERR_INVALID_ARGUMENT, "value dtype %d is not F16, BF16 or F32", value_dtype);
    if (!col_out || !values_out) return fail(ORTH_ERR_INVALID_ARGUMENT, "col_out or values_out is NULL");
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_csr_fill(w, w_dtype, out_features, in_features, row_ptr, mask, col_out, values_out,
                                   value_dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "CSR fill launch");
    return ORTH_OK;
}

static int check_sieve_flags(int32_t flags) {
    if (flags & ~ORTH_SIEVE_IEEE_DIV) return fail(ORTH_ERR_INVALID_ARGUMENT, "unknown sieve flags 0x%x", flags);
    return ORTH_OK;
}

int orth_sieve_quantize_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                            void *w_base, int32_t flags, void *stream) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return rc;
    rc = check_sieve_flags(flags);
    if (rc != ORTH_OK) return rc;
    if (!w_base) return fail(ORTH_ERR_INVALID_ARGUMENT, "w_base is NULL");
    if (out_features > INT32_MAX) return fail(ORTH_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_sieve_quantize(w, w_dtype, out_features, in_features, w_base,
                                         (flags & ORTH_SIEVE_IEEE_DIV) ? 1 : 0, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "sieve quantize launch");
    return ORTH_OK;
}

int64_t orth_sieve_select_bytes(void) { return 1040; }

int orth_sieve_split_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                         const void *h_inv, int32_t h_dtype, int64_t h_stride, int32_t score_dtype,
                         int32_t use_rank, int64_t rank, float threshold, void *w_base, void *w_ortho,
                         float *score, void *select_state, int32_t flags, void *stream) {
    int rc = check_pack_dims(w, w_dtype, out_features, in_features);
    if (rc != ORTH_OK) return rc;
    rc = check_sieve_flags(flags);
    if (rc != ORTH_OK) return rc;
    if (!h_inv || !valid_dtype(h_dtype)) return fail(ORTH_ERR_INVALID_ARGUMENT, "h_inv is NULL or of a bad dtype");
    if (!valid_dtype(score_dtype)) return fail(ORTH_ERR_INVALID_ARGUMENT, "score dtype %d is not F16, BF16 or F32", score_dtype);
    if (h_stride < 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "h_stride is negative");
    if (!w_base || !w_ortho || !score) return fail(ORTH_ERR_INVALID_ARGUMENT, "an output or the score buffer is NULL");
    if (use_rank && rank > 0 && !select_state) return fail(ORTH_ERR_INVALID_ARGUMENT, "select_state is NULL");
    if (rank < 0 || rank > out_features * in_features)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "rank %lld is outside [0, %lld]", (long long)rank,
                    (long long)(out_features * in_features));
    if (out_features > INT32_MAX || out_features * in_features > (int64_t)UINT32_MAX)
        return fail(ORTH_ERR_UNSUPPORTED, "the radix select counts in 32 bits: at most 2^32 - 1 weights");
    rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_sieve_split(w, w_dtype, out_features, in_features, h_inv, h_dtype, h_stride, score_dtype,
                                      use_rank, rank, threshold, w_base, w_ortho, score, select_state,
                                      (flags & ORTH_SIEVE_IEEE_DIV) ? 1 : 0, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "sieve split launch");
    return ORTH_OK;
}

int64_t orth_sieve_hdiag_workspace(int64_t rows, int64_t in_features) {
    if (rows <= 0 || in_features <= 0) return 0;
    return sieve_hdiag_slices(rows) * in_features;
}

int orth_sieve_hdiag_hip(const void *x, int32_t x_dtype, int64_t rows, int64_t in_features, float *workspace,
                         int64_t workspace_floats, void *out, int32_t flags, void *stream) {
    if (!x || !out || !workspace) return fail(ORTH_ERR_INVALID_ARGUMENT, "x, out or workspace is NULL");
    if (check_sieve_flags(flags) != ORTH_OK) return ORTH_ERR_INVALID_ARGUMENT;
    if (!valid_dtype(x_dtype)) return fail(ORTH_ERR_INVALID_ARGUMENT, "x dtype %d is not F16, BF16 or F32", x_dtype);
    if (rows <= 0 || in_features <= 0) return fail(ORTH_ERR_INVALID_ARGUMENT, "rows and in_features must be positive");
    if (workspace_floats < sieve_hdiag_slices(rows) * in_features)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "workspace holds %lld floats, %lld needed", (long long)workspace_floats,
                    (long long)(sieve_hdiag_slices(rows) * in_features));
    if (in_features > ((int64_t)1 << 40) / rows) return fail(ORTH_ERR_INVALID_ARGUMENT, "x is too large");
    int rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_sieve_hdiag(x, x_dtype, rows, in_features, workspace, out,
                                      (flags & ORTH_SIEVE_IEEE_DIV) ? 1 : 0, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "hessian diagonal launch");
    return ORTH_OK;
}

int orth_hip_device_info(int device, orth_hip_device_info_t *info) {
    if (!info) return fail(ORTH_ERR_INVALID_ARGUMENT, "info is NULL");
    std::memset(info, 0, sizeof(*info));
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return fail(ORTH_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return fail(ORTH_ERR_INVALID_ARGUMENT, "device %d out of range (count %d)", device, count);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
    std::snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
    info->is_gfx950 = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
    info->compute_units = p.multiProcessorCount;
    info->wavefront_size = p.warpSize;
    info->lds_bytes_per_block = (int32_t)p.sharedMemPerBlock;
    info->clock_khz = p.clockRate;
    info->memory_clock_khz = p.memoryClockRate;
    info->memory_bus_width = p.memoryBusWidth;
    info->l2_bytes = p.l2CacheSize;
    info->global_mem_bytes = (int64_t)p.totalGlobalMem;
    return ORTH_OK;
}

int orth_hip_set_kernel_policy(int policy) {
    if (policy < 0 || policy > 8) return fail(ORTH_ERR_INVALID_ARGUMENT, "policy must be 0..8");
    g_policy.store(policy);
    return ORTH_OK;
}

int orth_hip_get_kernel_policy(void) { return g_policy.load(); }

int orth_hip_last_kernel(void) { return t_last_kernel; }

const char *orth_hip_last_error(void) { return t_error.c_str(); }

int orth_hip_clock_stamp(uint64_t *dst, void *stream) {
    if (!dst) return fail(ORTH_ERR_INVALID_ARGUMENT, "dst is NULL");
    if (reinterpret_cast<uintptr_t>(dst) % 8) return fail(ORTH_ERR_INVALID_ARGUMENT, "dst is not 8-byte aligned");
    int rc = current_device_ok(nullptr);
    if (rc != ORTH_OK) return rc;
    hipError_t e = launch_clock_stamp(dst, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail_hip(e, "clock stamp launch");
    return ORTH_OK;
}

int orth_hip_abi_version(void) { return 103; }

}  // extern "C"
