/*
 * libortho_amd -- C ABI of the MI355X (gfx950) fused dual GEMM
 *
 *   y[m,n] = sum_k x[m,k] * q[n,k] * s[n, k/G]
 *          + [alpha > 0 && nnz > 0] * alpha * sum_{j in row n} v_j * x[m, c_j]
 *
 * A dense signed-INT4 "Base" (two nibbles per byte, FP16 scales per output
 * row or per group of G input columns) plus a sparse "Ortho" correction in
 * CSR form, in one launch.  All pointers are device pointers unless stated;
 * calls are asynchronous on the stream passed in (NULL = the null stream)
 * and never synchronise the device.  Plain C types only: no HIP or torch
 * types appear in the signatures (a stream is passed as void*).
 *
 * Replaces the reference's C ABI, /root/reference/include/ortho.h:22-159,
 * and its CUDA entry points, /root/reference/src/dual_gemm.cu:295-372 and
 * /root/reference/src/dual_gemm_tensor_core.cu:342-428.
 */
#ifndef ORTH_HIP_H
#define ORTH_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the buffers a layer points to. */
typedef enum {
    ORTH_DT_F16 = 0,
    ORTH_DT_BF16 = 1,
    ORTH_DT_F32 = 2
} orth_dtype_t;

/* Status codes.  Every entry point returns one; the message of the last
 * failure on the calling thread is in orth_hip_last_error().
 * Replaces the reference's 0 / -1 returns (src/dual_gemm.cu:301-303,361-371). */
typedef enum {
    ORTH_OK = 0,
    ORTH_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad shape, bad dtype     */
    ORTH_ERR_UNSUPPORTED = 2,      /* valid request this build cannot serve  */
    ORTH_ERR_HIP = 3,              /* a HIP runtime call failed              */
    ORTH_ERR_NO_DEVICE = 4         /* no usable gfx950 device                */
} orth_status_t;

/* The packed Base.  Mirrors orth_base_t, /root/reference/include/ortho.h:22-28,
 * with the scale element type and the number of scale groups made explicit.
 *   q_weight  uint8 [out_features, in_features/2]; element (n,k) is nibble
 *             n*K+k: byte (n*K+k)/2, low nibble for even k, two's complement
 *             (/root/reference/src/ortho.c:315-325)
 *   q_scales  [out_features, scale_groups] of scale_dtype (F16 or F32);
 *             G = in_features / scale_groups; scale_groups == 1 is the
 *             reference's per-row scale (/root/reference/torch_bind/ortho_linear.py:60) */
typedef struct {
    const void *q_weight;
    const void *q_scales;
    int32_t q_bits;          /* must be 4 */
    int32_t scale_dtype;     /* orth_dtype_t: ORTH_DT_F16 or ORTH_DT_F32 */
    int64_t scale_groups;    /* K / G, >= 1, divides in_features */
    int64_t in_features;     /* K, even, > 0 */
    int64_t out_features;    /* N, > 0 */
} orth_hip_base_t;

/* The sparse Ortho in CSR form.  Mirrors the CSR half of orth_ortho_t,
 * /root/reference/include/ortho.h:41-53 (the deprecated uint16 COO index is
 * not supported), as packed by /root/reference/tools/sieve.py:119-152.
 *   row_ptr      int32 [out_features + 1]; may be NULL when count == 0
 *   col_indices  int32 [count]; entries with col < 0 or col >= K are skipped
 *                (the reference's guard, /root/reference/src/dual_gemm.cu:124)
 *   values       [count] of value_dtype (F16 or F32) */
typedef struct {
    const int32_t *row_ptr;
    const int32_t *col_indices;
    const void *values;
    int32_t value_dtype;     /* orth_dtype_t: ORTH_DT_F16 or ORTH_DT_F32 */
    int32_t reserved;
    int64_t count;           /* nnz */
} orth_hip_ortho_t;

/* The dual-manifold layer.  Mirrors orth_layer_t,
 * /root/reference/include/ortho.h:63-71: the ortho term is applied iff
 * alpha > 0 and count > 0 (/root/reference/src/ortho.c:343), so a zero or
 * negative alpha gives the Base alone. */
typedef struct {
    orth_hip_base_t base;
    orth_hip_ortho_t ortho;
    float alpha;
} orth_hip_layer_t;

/* Sets layer->alpha.  Replaces orth_layer_set_alpha,
 * /root/reference/include/ortho.h:91 (/root/reference/src/ortho.c:111-115). */
void orth_layer_hip_set_alpha(orth_hip_layer_t *layer, float alpha);

/* Host-side validation of a forward call, with no device access: returns
 * ORTH_OK or the status orth_layer_forward_hip would return for these
 * arguments before launching anything.  No reference counterpart (the
 * reference validates nothing, /root/reference/torch_bind/bindings.cpp:19-43). */
int orth_layer_check_hip(const orth_hip_layer_t *layer, const void *input, void *output,
                         int64_t batch_size, int32_t io_dtype);

/* Forward pass y = Base(x) + alpha * Ortho(x).
 *   input   [batch_size, in_features] of io_dtype (F16, BF16 or F32), row-major
 *   output  [batch_size, out_features] of io_dtype, written in full
 * Picks, for FP16 I/O and the supported shapes, the decode kernel (batch <=
 * 4), the one-launch mid-batch kernel (5..16, K = 4096, a plan or no ortho
 * term), the quarter-split kernel (17..32, K = 4096, a plan or no ortho
 * term), the slice-split kernel (17..32 at the other K % 128 == 0, a plan
 * or no ortho term), the split-K mid-batch kernel (other batches up to 64;
 * 33..64 at K > 4096 with a plan or no ortho term: the prefill kernel with
 * K split over the grid),
 * the MFMA prefill kernels above (256 x 128 tiles with K split over the
 * grid and a reduction launch where the tiles alone leave CUs idle and a
 * plan or no ortho term is given; else the wide kernel where its 256 x 352
 * tile per workgroup needs fewer rounds of the grid than 256 x 128 tiles,
 * as at 4096 -> 11008 with 2048 tokens, or from 1024 tokens with 256 x
 * 128 tiles in 64-column steps; else 256 x 128 tiles), and a general kernel for shapes and
 * dtypes the fast kernels do not take (orth_hip_last_kernel() names the
 * choice).  BF16 I/O
 * takes the decode kernel for 1..4 tokens and the one-launch mid-batch
 * kernel for 5..16 (both K = 4096 with a plan or no ortho term), the
 * slice-split kernel for 17..32 (K % 128 == 0, a plan or no ortho term),
 * the split-K mid-batch kernel for the other batches up to 64
 * (K % 128 == 0), the prefill kernel above; FP32 I/O the general kernel.  Kernels
 * that need scratch memory (split-K partials, a prefill plan when none is
 * given) take it from a per-stream workspace or stream-ordered allocations.
 * Replaces orth_layer_forward_cuda, /root/reference/include/ortho.h:141-144
 * (/root/reference/src/dual_gemm.cu:295-372), the body of the torch binding
 * /root/reference/torch_bind/bindings.cpp:9-44, and the CPU entry
 * orth_layer_forward, /root/reference/include/ortho.h:132-135. */
int orth_layer_forward_hip(const orth_hip_layer_t *layer, const void *input, void *output,
                           int64_t batch_size, int32_t io_dtype, void *stream);

/* Same, with a prebuilt ortho plan (orth_ortho_plan_build) for the prefill
 * kernel; plan may be NULL.  The plan must have been built from this layer's
 * current CSR buffers.  No reference counterpart: the plan is a derived
 * layout of the CSR of /root/reference/tools/sieve.py:119-152. */
int orth_layer_forward_hip_planned(const orth_hip_layer_t *layer, const void *plan,
                                   int64_t plan_bytes, const void *input, void *output,
                                   int64_t batch_size, int32_t io_dtype, void *stream);

/* Same, with the bias of OrthoLinear.forward fused into the output store:
 * bias [out_features] (F16, BF16 or F32; NULL for none) is added as
 * `output += bias` does after the kernel, /root/reference/torch_bind/
 * ortho_linear.py:165-166: y = round(float(round(acc)) + bias[n]) in the
 * output dtype, so the result has the same bits as the unfused add. */
int orth_layer_forward_hip_ex(const orth_hip_layer_t *layer, const void *plan, int64_t plan_bytes,
                              const void *bias, int32_t bias_dtype, const void *input, void *output,
                              int64_t batch_size, int32_t io_dtype, void *stream);

/* Same as orth_layer_forward_hip_ex, but it allocates nothing: no
 * hipMalloc, hipFree or stream-ordered allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it).  No counterpart in the reference.  The scratch memory the
 * kernels need (the mid-batch kernels' split-K, quarter and slice partials,
 * the prefill K split's partials, the prefill part of an ortho plan when
 * the caller passes none) comes from a static device array of
 * ORTH_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call
 * that would need more returns ORTH_ERR_UNSUPPORTED before launching
 * anything.  Every call on one GPU shares that GPU's array: an eager call on
 * a stream other than the previous call's first waits for that call (an
 * event the library records), so eager calls on several streams or threads
 * do not race; calls captured into graphs, and their replays, are not
 * ordered that way and must be ordered by the caller.  Each call writes all
 * the scratch it reads, so nothing carries over from an earlier call. */
#define ORTH_NOALLOC_SCRATCH_BYTES (32u << 20)
int orth_layer_forward_hip_noalloc(const orth_hip_layer_t *layer, const void *plan, int64_t plan_bytes,
                                   const void *bias, int32_t bias_dtype, const void *input, void *output,
                                   int64_t batch_size, int32_t io_dtype, void *stream);

/* ORTH_NOALLOC_SCRATCH_BYTES, for bindings that cannot read the macro. */
int64_t orth_noalloc_scratch_bytes(void);

/* Forward of `count` (1..ORTH_GROUP_MAX) layers that read the same input,
 * outputs[l] = layers[l](input) as orth_layer_forward_hip_ex computes it
 * (plans, plan_bytes, biases and bias_dtypes: arrays of `count` entries, or
 * NULL for none; a NULL entry is no plan / no bias).  When every layer takes
 * the decode kernel with the same instantiation (the same in_features,
 * scale layout, ortho mode and plan record size) the layers share one
 * launch, each layer's output rows dealt to their own workgroups
 * (orth_hip_last_kernel() then returns 5); at 17..32 tokens, when every
 * layer takes the quarter- or slice-split kernel and the layers share K,
 * scale layout, ortho class and record size, one slice-split launch and one
 * reduction take them all (returns 9; each output then has the bits of
 * that layer's slice-split call, kernel policy 7, which at K = 4096 differs
 * from the default quarter-split call in FP32 summation order only);
 * otherwise each layer is its own forward call.  Outputs must not overlap.
 * No counterpart in the
 * reference, which calls its forward once per projection
 * (OrthoLinear.forward, /root/reference/torch_bind/ortho_linear.py:130-168, per module): for the
 * projections of one block that read one activation (q/k/v, gate/up) it
 * saves the launch gaps between them. */
#define ORTH_GROUP_MAX 4
int orth_layers_forward_hip(const orth_hip_layer_t *const *layers, const void *const *plans,
                            const int64_t *plan_bytes, const void *const *biases, const int32_t *bias_dtypes,
                            int32_t count, const void *input, void *const *outputs, int64_t batch_size,
                            int32_t io_dtype, void *stream);

/* Size in bytes of the ortho plan for this layer (0 when count == 0), or a
 * negative orth_status_t on invalid arguments. */
int64_t orth_ortho_plan_bytes(const orth_hip_layer_t *layer);

/* Builds the ortho plan into caller-owned device memory and waits for it
 * (load-time call: it synchronises the stream to report CSR errors).
 * Returns ORTH_ERR_INVALID_ARGUMENT for a row_ptr that is not monotone or
 * does not end at count.  Derived layout of the CSR of
 * /root/reference/tools/sieve.py:119-152; no reference counterpart. */
int orth_ortho_plan_build(const orth_hip_layer_t *layer, void *plan, int64_t plan_bytes,
                          void *stream);

/* Writes the dequantised Base, out[n*K+k] = float(q[n,k]) * float(s[n,k/G]),
 * as FP32 [out_features, in_features] (exact: |q| <= 8 times an FP16 scale
 * fits in 24 bits).  Debug/parity entry; replaces the per-element
 * "(float)unpack_int4(...) * scale" of /root/reference/src/ortho.c:360-363
 * and unpack_int4 of /root/reference/src/dual_gemm.cu:30-40. */
int orth_base_dequant_hip(const orth_hip_layer_t *layer, float *out, void *stream);

/* Packing on the device (load time).  All pointers are device memory; the
 * calls are asynchronous on `stream`.
 *
 * orth_pack_base_hip quantises dense weights w [out_features, in_features]
 * (F16, BF16 or F32, row-major) to the packed INT4 layout of
 * orth_hip_base_t: q_out uint8 [out_features, in_features / 2] (low nibble =
 * even index) and scales_out FP16 [out_features, in_features / group_size]
 * (group_size <= 0: one scale per row).  Without scales_in the scales are
 * max|w| / 7 per row or group, clamped at 1e-6; with scales_in (dtype
 * scales_in_dtype, same shape) those are used.  q = clamp(round(w / s), -8,
 * 7) with s as computed or given, not its FP16 copy.  Replaces the torch
 * ops of load_from_weights, /root/reference/torch_bind/ortho_linear.py:89-120,
 * with their results on a GPU tensor (see orth_pack.hip for the arithmetic).
 * group_size must be even and divide in_features (even). */
int orth_pack_base_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                       int64_t group_size, const void *scales_in, int32_t scales_in_dtype, void *q_out,
                       void *scales_out, void *stream);

/* Which kernel orth_pack_base_hip takes for these arguments: 1 one wave per
 * (row, group) for group sizes 128, 256, 512, 1024 and 2048 (16-byte
 * aligned w and q_out), 2 one workgroup per row for one scale per row up to
 * 16384 columns, 3 the per-group fallback.  No counterpart in the
 * reference (testing and measurement). */
int orth_pack_base_path(const void *w, int32_t w_dtype, int64_t in_features, int64_t group_size,
                        const void *q_out);

/* CSR of the nonzeros (w != 0: -0 dropped, NaN kept) of dense w
 * [out_features, in_features], in two steps as
 * pack_ortho_sparse(w, "csr"), /root/reference/tools/sieve.py:119-152:
 * orth_pack_csr_rows_hip writes row_ptr int32 [out_features + 1] (0, then
 * the running counts; -1 from the first row where the count passes
 * 2^31 - 1); the caller reads nnz = row_ptr[out_features] and allocates;
 * orth_pack_csr_fill_hip writes col_out int32 [nnz] (ascending within a
 * row) and values_out [nnz] in value_dtype (bit copies when it is w's dtype,
 * else rounded to nearest even).  mask: optional device workspace of
 * orth_pack_csr_mask_bytes bytes (0: none for these weights, pass NULL)
 * where the first step records each element's nonzero bit, so that the
 * second reads only the nonzero elements of w instead of all of it; the
 * same mask must be passed to both steps (or NULL to both).  No reference
 * counterpart for the mask. */
int64_t orth_pack_csr_mask_bytes(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features);
int orth_pack_csr_rows_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                           int32_t *row_ptr, void *mask, int64_t mask_bytes, void *stream);
int orth_pack_csr_fill_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                           const int32_t *row_ptr, const void *mask, int64_t mask_bytes, int32_t *col_out,
                           void *values_out, int32_t value_dtype, void *stream);

/* The offline Base/Ortho sieve on the device (a one-off step before
 * packing; all pointers device memory, calls asynchronous on `stream`).
 * Each replaces torch ops of /root/reference/tools/sieve.py with the same
 * arithmetic on a GPU tensor (every intermediate rounded to the dtype the
 * torch op returns).  `flags`: 0, or ORTH_SIEVE_IEEE_DIV to divide by the
 * host scalars (7 and the row count) as torch does on a CPU tensor (IEEE
 * division) instead of as on a GPU tensor (a product with the FP32
 * reciprocal); any other bit is an error.
 *
 * orth_sieve_quantize_hip: w_base [out_features, in_features] (w's dtype) =
 * quantize_int4(w), /root/reference/tools/sieve.py:13-23: per-row scale
 * clamp(max|w|, 1e-8) / 7, clamp(round(w / s), -8, 7) * s, non-finite -> 0. */
#define ORTH_SIEVE_IEEE_DIV 1
int orth_sieve_quantize_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                            void *w_base, int32_t flags, void *stream);

/* orth_sieve_split_hip: hessian_sieve, /root/reference/tools/sieve.py:25-76.
 * Writes w_base as above and w_ortho = residual * (score > t) (w's dtype),
 * with residual = w - w_base and score = residual^2 / (h + 1e-6) (written to
 * `score`, FP32 [out_features * in_features], holding values of score_dtype,
 * the promotion of w's and h's dtypes).  h: element k at h_inv[k * h_stride]
 * (the diagonal of a matrix H_inv: its two strides summed; a vector: 1).
 * use_rank: t = the rank-th largest score (torch.topk(...).values[-1], NaN
 * largest; rank 0 keeps nothing), found by a radix select in select_state
 * (orth_sieve_select_bytes() bytes of device memory); else t = threshold. */
int64_t orth_sieve_select_bytes(void);
int orth_sieve_split_hip(const void *w, int32_t w_dtype, int64_t out_features, int64_t in_features,
                         const void *h_inv, int32_t h_dtype, int64_t h_stride, int32_t score_dtype,
                         int32_t use_rank, int64_t rank, float threshold, void *w_base, void *w_ortho,
                         float *score, void *select_state, int32_t flags, void *stream);

/* orth_sieve_hdiag_hip: out [in_features] (x's dtype) = diag(x^T x) / rows +
 * 1e-6 for x [rows, in_features], /root/reference/tools/sieve.py:79-95 (the
 * diagonal only: FP32 column sums of squares over row slices, then the
 * division and the add of the torch ops).  workspace: FP32 device memory of
 * orth_sieve_hdiag_workspace(rows, in_features) elements. */
int64_t orth_sieve_hdiag_workspace(int64_t rows, int64_t in_features);
int orth_sieve_hdiag_hip(const void *x, int32_t x_dtype, int64_t rows, int64_t in_features, float *workspace,
                         int64_t workspace_floats, void *out, int32_t flags, void *stream);

/* Device facts.  Replaces check_tensor_core_support,
 * /root/reference/src/dual_gemm_tensor_core.cu:342-350. */
typedef struct {
    char arch[64];            /* e.g. "gfx950:sramecc+:xnack-" */
    int32_t is_gfx950;        /* 1 when the fast kernels can run */
    int32_t compute_units;
    int32_t wavefront_size;
    int32_t lds_bytes_per_block;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int32_t l2_bytes;
    int64_t global_mem_bytes;
} orth_hip_device_info_t;

int orth_hip_device_info(int device, orth_hip_device_info_t *info);

/* Kernel choice override for benchmarking and tests: 0 = automatic (the
 * default), 1 = decode, 2 = prefill, 3 = general, 4 = split-K mid-batch
 * (5..64 tokens), 5 = one-launch mid-batch (5..16 tokens), 6 = K quarters
 * over the grid (17..32 tokens, K = 4096), 7 = 1024-column slices over the
 * grid (1..32 tokens), 8 = the wide prefill kernel (any batch; its 256 x
 * 352 tile where that needs fewer rounds of the grid than 256 x 128 tiles
 * at 512 tokens or more, else 256 x 128 tiles in 64-column steps).  A
 * forced kernel that cannot take a call returns
 * ORTH_ERR_UNSUPPORTED.  Process-wide. */
int orth_hip_set_kernel_policy(int policy);
int orth_hip_get_kernel_policy(void);

/* The kernel the calling thread's last successful forward launched:
 * 1 decode, 2 prefill, 3 general, 4 split-K mid-batch, 5 decode for a
 * group of layers in one launch (orth_layers_forward_hip), 6 one-launch
 * mid-batch, 7 K quarters over the grid, 8 1024-column slices over the
 * grid, 9 the same for a group of layers in one launch, 10 the wide
 * prefill kernel (256 x 352 or 256 x 128 tiles), 0 none. */
int orth_hip_last_kernel(void);

/* Device clock stamp for timing stream-ordered work (benchmarks; no
 * counterpart in the reference): launches ORTH_CLOCK_GROUPS workgroups on
 * `stream`; workgroup i writes dst[2i] = the 100 MHz constant device clock
 * (s_memrealtime) read as it starts and dst[2i + 1] = the id of the XCD it
 * ran on.  dst: device memory of 2 * ORTH_CLOCK_GROUPS uint64_t.  Two
 * stamps around K launches, differenced per XCD, time the K launches plus
 * one launch gap. */
#define ORTH_CLOCK_GROUPS 8
#define ORTH_CLOCK_HZ 100000000
int orth_hip_clock_stamp(uint64_t *dst, void *stream);

/* Message of the calling thread's last failure ("" if none). */
const char *orth_hip_last_error(void);

/* ABI version of this header (major * 100 + minor). */
int orth_hip_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ORTH_HIP_H */
