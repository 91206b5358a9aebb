// Device-side building blocks shared by the gfx950 dual-GEMM kernels.
//
// Packed Base layout (the API layout, /root/reference/src/ortho.c:315-325 and
// /root/reference/torch_bind/ortho_linear.py:107-120): element (n, k) of the
// [N, K] INT4 matrix is nibble n*K+k, stored in byte (n*K+k)/2, low nibble for
// even k, two's complement.  One 32-bit word therefore holds 8 consecutive k
// of one row: nibble i of the word (bits 4i..4i+3) is k0+i.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "orth_hip.h"

namespace orth {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Which kernel served a forward call (orth_hip_last_kernel()).
enum KernelId {
    KERNEL_NONE = 0,
    KERNEL_DECODE = 1,
    KERNEL_PREFILL = 2,
    KERNEL_GENERAL = 3,
    KERNEL_SKINNY = 4,
    KERNEL_DECODE_GROUP = 5,  // one decode launch for several layers
    KERNEL_MID = 6,           // one-launch mid-batch kernel (5..16 tokens)
    KERNEL_QUARTER = 7,       // K quarters over the grid (17..32 tokens)
    KERNEL_SPLIT = 8,         // 1024-column slices over the grid (17..32 tokens)
    KERNEL_SPLIT_GROUP = 9,   // the same for a group of layers in one launch
    KERNEL_PREFILL_WIDE = 10  // the wide prefill kernel (256 x 352 or 256 x 128 tiles)
};

// Everything a forward launch needs, resolved on the host.
struct ForwardArgs {
    const uint8_t *q;        // [N, K/2]
    const void *scales;      // [N, ngroups]
    int scale_dtype;
    int64_t ngroups;
    int64_t G;               // K / ngroups
    const int32_t *row_ptr;  // [N+1]
    const int32_t *col;      // [nnz]
    const void *vals;        // [nnz]
    int val_dtype;
    int64_t nnz;
    const void *x;           // [M, K]
    void *y;                 // [M, N]
    int io_dtype;
    int64_t M, K, N;
    float alpha;
    int has_ortho;           // alpha > 0 && nnz > 0 (/root/reference/src/ortho.c:343)
    const void *bias = nullptr;  // [N] added to y after rounding, or null
    int bias_dtype = 0;
};

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    // round to nearest even; NaN stays NaN
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Load element i of a buffer of the given orth_dtype_t as float.
__device__ __forceinline__ float load_as_f32(const void *p, int dtype, int64_t i) {
    if (dtype == ORTH_DT_F16) return (float)((const f16 *)p)[i];
    if (dtype == ORTH_DT_BF16) return bf16_bits_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

__device__ __forceinline__ void store_from_f32(void *p, int dtype, int64_t i, float v) {
    if (dtype == ORTH_DT_F16) ((f16 *)p)[i] = (f16)v;
    else if (dtype == ORTH_DT_BF16) ((uint16_t *)p)[i] = f32_to_bf16_bits(v);
    else ((float *)p)[i] = v;
}

// v rounded to the precision of an orth_dtype_t (nearest even), as float.
__device__ __forceinline__ float round_as(int dtype, float v) {
    if (dtype == ORTH_DT_F16) return (float)(f16)v;
    if (dtype == ORTH_DT_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    return v;
}

// An FP16 output with the optional bias: y = fp16(float(fp16(v)) + bias[n]),
// the bits of the kernel's FP16 output followed by `y += bias` in torch
// (/root/reference/torch_bind/ortho_linear.py:165-166: the sum in FP32,
// rounded to y's dtype).
__device__ __forceinline__ f16 out_f16(float v, const void *bias, int bias_dtype, int64_t n) {
    f16 r = (f16)v;
    if (bias) r = (f16)((float)r + load_as_f32(bias, bias_dtype, n));
    return r;
}

// The same for a BF16 output (round to nearest even): y = bf16(float(bf16(v)) + bias[n]).
__device__ __forceinline__ uint16_t out_bf16(float v, const void *bias, int bias_dtype, int64_t n) {
    uint16_t r = f32_to_bf16_bits(v);
    if (bias) r = f32_to_bf16_bits(bf16_bits_to_f32(r) + load_as_f32(bias, bias_dtype, n));
    return r;
}

// A 16-bit activation (FP16, or BF16 when XB) as float.
template <bool XB>
__device__ __forceinline__ float x16_to_f32(f16 h) {
    if constexpr (XB) return bf16_bits_to_f32(__builtin_bit_cast(uint16_t, h));
    else return (float)h;
}

// Sign-extend a 4-bit two's complement nibble.
__device__ __forceinline__ int sext4(uint32_t nib) { return (int)(nib ^ 8u) - 8; }

// Ortho plan cell records (built in orth_prefill.hip): for a 16-row group g
// and a column cell c (the decode kernel's K quarters, the mid-batch
// kernel's 1024-column slices), `words` words at an address that needs no
// other load.  Header: [0] tag, [1] the number of the cell's entries that
// did not fit (the kernel then reads the CSR), [2 + r] row 16 g + r's
// entries as start | end << 16 (entry indices), [18], [19] zero.  Entries
// from word 20: column - the cell's first column | fp16 value bits << 16,
// rows in order, each row's entries in CSR order; unused slots 0xffff.
constexpr int kCellHdrWords = 20;
constexpr uint32_t kCellQuarter = 0x51524543u;  // decode K quarters
constexpr uint32_t kCellSlice = 0x53524543u;    // mid-batch 1024-column slices

// Tag of a cell record: ties it to its kind, the layer shape, the record
// size and its place, so that a plan of another layer is not read as this one.
__host__ __device__ inline uint32_t plan_cell_tag(uint32_t kind, int64_t N, int64_t K, int64_t nnz, int words,
                                                  int64_t g, int c) {
    return kind ^ (uint32_t)nnz ^ ((uint32_t)N * 0x9E3779B1u) ^ ((uint32_t)K << 13) ^
           ((uint32_t)words * 0xC2B2AE3Du) ^ ((uint32_t)g * 0x85EBCA77u) ^ ((uint32_t)c * 0x27D4EB2Fu);
}

// Chunks (128 columns) per wave of the decode kernel: the K quarter of wave
// w is chunks [w c, min((w + 1) c, K / 128)), c even.
__host__ __device__ inline int decode_chunks_per_wave(int64_t K) {
    const int64_t nchunks = K / 128;
    const int64_t c = (nchunks + 3) / 4;
    return (int)((c + 1) & ~int64_t(1));
}

// CSR row range [rs, re), clamped into [0, nnz] so a malformed row_ptr can
// never address outside the index arrays.
__device__ __forceinline__ void csr_row_range(const int32_t *row_ptr, int64_t n, int64_t nnz,
                                              int32_t &rs, int32_t &re) {
    int64_t a = row_ptr[n], b = row_ptr[n + 1];
    a = a < 0 ? 0 : (a > nnz ? nnz : a);
    b = b < a ? a : (b > nnz ? nnz : b);
    rs = (int32_t)a;
    re = (int32_t)b;
}

// ------------------------------------------------------ INT4 -> FP16 words
//
// Magic-number conversion: a 4-bit value u placed in mantissa bits 0..3 of
// binary16 1024.0 (0x6400) reads as exactly 1024 + u; placed in bits 4..7 of
// binary16 64.0 (0x5400) it reads as exactly 64 + u (the unit in the last
// place of 64 is 1/16).  With u = n ^ 8 = q + 8 for the two's complement
// nibble n, q = (1024 + u) - 1032 = (64 + u) - 72 exactly.  The XOR by 8 is
// folded into the constant: (w & M) ^ (C | 0x8<<shift) == ((w ^ 0x88888888) & M) | C
// because the masked bits and C's bits do not overlap.

// "Interleaved" order: from one packed word produce four f16x2 words holding
// k-pairs (0,4) (1,5) (2,6) (3,7).  One shift, four and-xor (v_bitop3) and
// four exact packed-half subtracts for 8 weights; the activation operand
// must use the same order (see permute_x8).
__device__ __forceinline__ void int4x8_to_f16_interleaved(uint32_t w, uint32_t out[4]) {
    const uint32_t t = w >> 8;
    const uint32_t p0 = (w & 0x000F000Fu) ^ 0x64086408u;  // 1024+u0 | 1024+u4
    const uint32_t p1 = (w & 0x00F000F0u) ^ 0x54805480u;  //   64+u1 |   64+u5
    const uint32_t p2 = (t & 0x000F000Fu) ^ 0x64086408u;  // 1024+u2 | 1024+u6
    const uint32_t p3 = (t & 0x00F000F0u) ^ 0x54805480u;  //   64+u3 |   64+u7
    const f16x2 b1032 = {(f16)-1032.0f, (f16)-1032.0f};
    const f16x2 b72 = {(f16)-72.0f, (f16)-72.0f};
    out[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, p0) + b1032);
    out[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, p1) + b72);
    out[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, p2) + b1032);
    out[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, p3) + b72);
}

// Same words without the bias: halves read 1024+u (k-pairs (0,4), (2,6))
// and 64+u (k-pairs (1,5), (3,7)).  An MFMA over them yields
// sum_k x_k q_k + 1032 * sum_{k even} x_k + 72 * sum_{k odd} x_k, and the two
// activation sums are removed afterwards: five ops for 8 weights.
__device__ __forceinline__ void int4x8_to_f16_biased(uint32_t w, uint32_t out[4]) {
    const uint32_t t = w >> 8;
    out[0] = (w & 0x000F000Fu) ^ 0x64086408u;
    out[1] = (w & 0x00F000F0u) ^ 0x54805480u;
    out[2] = (t & 0x000F000Fu) ^ 0x64086408u;
    out[3] = (t & 0x00F000F0u) ^ 0x54805480u;
}

// BF16 words in the same interleaved order, biased: a 4-bit value u in
// mantissa bits 0..3 of bfloat16 128.0 (0x4300, whose unit in the last
// place is 1) reads as exactly 128 + u, so with u = n ^ 8 = q + 8 every half
// is q + 136.  An MFMA over them yields sum_k x_k q_k + 136 * sum_k x_k.
__device__ __forceinline__ void int4x8_to_bf16_biased(uint32_t w, uint32_t out[4]) {
    out[0] = (w & 0x000F000Fu) ^ 0x43084308u;          // k-pair (0,4)
    out[1] = ((w >> 4) & 0x000F000Fu) ^ 0x43084308u;   // (1,5)
    out[2] = ((w >> 8) & 0x000F000Fu) ^ 0x43084308u;   // (2,6)
    out[3] = ((w >> 12) & 0x000F000Fu) ^ 0x43084308u;  // (3,7)
}

// Reorder 8 consecutive fp16 (as 4 words (0,1)(2,3)(4,5)(6,7)) into the
// interleaved order (0,4)(1,5)(2,6)(3,7) used by int4x8_to_f16_interleaved.
__device__ __forceinline__ u32x4 permute_x8(u32x4 d) {
    u32x4 r;
    r.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);  // lo halves of d0, d2
    r.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);  // hi halves of d0, d2
    r.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
    r.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
    return r;
}

// Position of element r (0..7) of an 8-chunk in the interleaved order.
__device__ __forceinline__ int interleaved_pos(int r) { return ((r & 3) << 1) | (r >> 2); }

// ------------------------------------------------------------ reductions

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// v of the lane `ctrl` names (a DPP pattern within rows of 16 lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
// Groups of 16 are the DPP rows: rotations by 8, 4, 2, 1 lanes within the
// row (register moves, no LDS round trip) leave every lane with its row's
// sum (each lane adds in its own order, so callers take one fixed lane).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (WIDTH == 16) {
        v += dpp_f32<0x128>(v);  // row_ror:8
        v += dpp_f32<0x124>(v);  // row_ror:4
        v += dpp_f32<0x122>(v);  // row_ror:2
        v += dpp_f32<0x121>(v);  // row_ror:1
        return v;
    } else {
#pragma unroll
        for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        return v;
    }
}

}  // namespace orth
