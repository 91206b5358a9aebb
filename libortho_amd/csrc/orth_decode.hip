// Decode dual GEMM (batch M <= 16) for gfx950.
//
// Computes what /root/reference/src/dual_gemm.cu:176-225 computes (the
// reference launches one 32-thread block per 32 output rows and walks K
// serially per thread, one byte load per nibble); the work here is laid out
// for CDNA4 instead:
//
//  * A workgroup of W waves owns RT = 16*R consecutive output rows.  K is cut
//    into 128-wide chunks dealt round-robin to the waves (split-K inside the
//    workgroup, reduced through LDS: deterministic, no atomics).
//  * Per chunk and 16-row block every lane issues ONE 16-byte load: lane
//    (row r = lane%16, quarter g = lane/16) takes bytes [64c + 16g, +16) of
//    row r, so the 4 lanes of a row read its 64 contiguous bytes of the
//    chunk.  All of a wave's chunk loads are issued before any are consumed.
//  * Each 32-bit word (8 nibbles) becomes 8 exact FP16 integers in registers
//    (int4x8_to_f16_interleaved) and feeds v_mfma_f32_16x16x32_f16 as the B
//    operand; the activations (tokens padded to 16 with zeros) are the A
//    operand, staged once per workgroup in LDS in the matching interleaved
//    k order.  One MFMA consumes 8 nibbles per lane, so the tensor core does
//    the K reduction and no cross-lane shuffles are needed for the base term.
//  * Group scales (G a multiple of 128) are applied to FP32 partial sums per
//    chunk: q stays exact in FP16 and q*s is never rounded.
//  * Epilogue: the CSR rows of the workgroup's RT output rows are contiguous
//    in col/values; 16-lane groups per row walk them with x from LDS, reduce
//    with lane shuffles and add alpha*sum after the base term, as
//    /root/reference/src/dual_gemm.cu:212-221 does.  alpha <= 0 skips it on a
//    uniform branch without touching the CSR arrays.
#include "orth_common.h"

namespace orth {

struct DecodeArgs {
    const uint8_t *q;
    const f16 *scales;
    int64_t ngroups;
    int64_t G;
    const int32_t *row_ptr;
    const int32_t *col;
    const f16 *vals;
    int64_t nnz;
    const f16 *x;
    f16 *y;
    int M;
    int nchunks;   // K / 128
    int64_t K, N;
    int xstride;   // LDS row stride of the staged activations, in halves
    float alpha;
    int has_ortho;
};

template <int MT, bool GROUPED, bool XLDS, int W, int R, int PF>
__global__ void __launch_bounds__(64 * W) decode_kernel(DecodeArgs a) {
    constexpr int NT = 64 * W;
    constexpr int RT = 16 * R;
    constexpr int TPR = NT / RT;  // threads per output row in the sparse epilogue
    static_assert(TPR >= 1 && TPR <= 64 && (TPR & (TPR - 1)) == 0, "bad epilogue split");

    extern __shared__ __align__(16) unsigned char smem[];
    float *red = reinterpret_cast<float *>(smem);           // [W][R][16][16]
    float *sp = red + W * R * 256;                           // [MT][RT]
    f16 *ss = reinterpret_cast<f16 *>(sp + MT * RT);         // [RT][ngroups] (GROUPED)
    f16 *xs = ss + (GROUPED ? RT * a.ngroups : 0);           // [MT][xstride] (XLDS)
    xs = reinterpret_cast<f16 *>((reinterpret_cast<uintptr_t>(xs) + 15) & ~uintptr_t(15));

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int nl = lane & 15;  // B column (weight row) and A row (token) of this lane
    const int g = lane >> 4;   // which 32-k quarter of a chunk
    const int64_t n0 = (int64_t)blockIdx.x * RT;
    const int64_t K = a.K;

    // ---- issue this wave's first weight loads before anything else
    const int nci = (a.nchunks - wave + W - 1) / W;  // chunks of this wave
    const uint8_t *qrow[R];
#pragma unroll
    for (int rb = 0; rb < R; rb++) {
        int64_t n = n0 + rb * 16 + nl;
        n = n < a.N ? n : a.N - 1;
        qrow[rb] = a.q + n * (K >> 1) + g * 16;
    }
    u32x4 wbuf[PF][R];
    u32x4 abuf[XLDS ? 1 : PF][4];
    const bool tok_ok = nl < a.M;  // rows of A beyond M are zero
    const f16 *xrow = a.x + (int64_t)(tok_ok ? nl : 0) * K + g * 32;
#pragma unroll
    for (int p = 0; p < PF; p++) {
        if (p < nci) {
            const int c = wave + W * p;
#pragma unroll
            for (int rb = 0; rb < R; rb++)
                wbuf[p][rb] = *reinterpret_cast<const u32x4 *>(qrow[rb] + c * 64);
            if (!XLDS) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    abuf[p][j] = tok_ok ? *reinterpret_cast<const u32x4 *>(xrow + c * 128 + 8 * j)
                                        : u32x4{0, 0, 0, 0};
            }
        }
    }

    // ---- stage activations (interleaved k order) and group scales in LDS
    if (XLDS) {
        const int k8 = (int)(K >> 3);
        for (int idx = tid; idx < MT * k8; idx += NT) {
            const int m = idx / k8, c8 = idx - m * k8;
            u32x4 v = {0, 0, 0, 0};
            if (m < a.M) v = permute_x8(*reinterpret_cast<const u32x4 *>(a.x + (int64_t)m * K + c8 * 8));
            *reinterpret_cast<u32x4 *>(xs + m * a.xstride + c8 * 8) = v;
        }
    }
    if (GROUPED) {
        const int total = RT * (int)a.ngroups;
        for (int idx = tid; idx < total; idx += NT) {
            const int r = idx / (int)a.ngroups, gg = idx - r * (int)a.ngroups;
            int64_t n = n0 + r;
            n = n < a.N ? n : a.N - 1;
            ss[idx] = a.scales[n * a.ngroups + gg];
        }
    }
    __syncthreads();

    // ---- main loop over this wave's chunks
    f32x4 acc[R];
#pragma unroll
    for (int rb = 0; rb < R; rb++) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int base = 0; base < nci; base += PF) {
        u32x4 cur[PF][R];
        u32x4 acur[XLDS ? 1 : PF][4];
#pragma unroll
        for (int p = 0; p < PF; p++) {
#pragma unroll
            for (int rb = 0; rb < R; rb++) cur[p][rb] = wbuf[p][rb];
            if (!XLDS) {
#pragma unroll
                for (int j = 0; j < 4; j++) acur[p][j] = abuf[p][j];
            }
        }
        // prefetch the next batch
#pragma unroll
        for (int p = 0; p < PF; p++) {
            if (base + PF + p < nci) {
                const int c = wave + W * (base + PF + p);
#pragma unroll
                for (int rb = 0; rb < R; rb++)
                    wbuf[p][rb] = *reinterpret_cast<const u32x4 *>(qrow[rb] + c * 64);
                if (!XLDS) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        abuf[p][j] = tok_ok ? *reinterpret_cast<const u32x4 *>(xrow + c * 128 + 8 * j)
                                            : u32x4{0, 0, 0, 0};
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PF; p++) {
            if (base + p < nci) {
                const int c = wave + W * (base + p);
                f16x8 afr[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    u32x4 av;
                    if (XLDS) {
                        av = (nl < MT) ? *reinterpret_cast<const u32x4 *>(xs + nl * a.xstride + c * 128 + g * 32 + 8 * j)
                                       : u32x4{0, 0, 0, 0};
                    } else {
                        av = permute_x8(acur[p][j]);
                    }
                    afr[j] = __builtin_bit_cast(f16x8, av);
                }
#pragma unroll
                for (int rb = 0; rb < R; rb++) {
                    const u32x4 wv = cur[p][rb];
                    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
                    f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        uint32_t b[4];
                        int4x8_to_f16_interleaved(words[j], b);
                        const f16x8 bfr = __builtin_bit_cast(f16x8, u32x4{b[0], b[1], b[2], b[3]});
                        if (GROUPED)
                            part = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[j], bfr, part, 0, 0, 0);
                        else
                            acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[j], bfr, acc[rb], 0, 0, 0);
                    }
                    if (GROUPED) {
                        const float s = (float)ss[(rb * 16 + nl) * a.ngroups + ((int64_t)c * 128) / a.G];
                        acc[rb] += s * part;
                    }
                }
            }
        }
    }

    // ---- split-K partials to LDS: lane holds D[token 4g+i][row nl]
#pragma unroll
    for (int rb = 0; rb < R; rb++) {
#pragma unroll
        for (int i = 0; i < 4; i++) red[((wave * R + rb) * 16 + (4 * g + i)) * 16 + nl] = acc[rb][i];
    }

    // ---- sparse ortho term: TPR lanes per output row
    if (a.has_ortho) {
        const int rl = tid / TPR, sub = tid - rl * TPR;
        const int64_t n = n0 + rl;
        float sacc[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) sacc[m] = 0.f;
        if (n < a.N) {
            int32_t rs, re;
            csr_row_range(a.row_ptr, n, a.nnz, rs, re);
            for (int32_t j = rs + sub; j < re; j += TPR) {
                const int32_t c = a.col[j];
                if (c >= 0 && c < K) {
                    const float v = (float)a.vals[j];
#pragma unroll
                    for (int m = 0; m < MT; m++) {
                        if (m < a.M) {
                            float xv;
                            if (XLDS) xv = (float)xs[m * a.xstride + (c & ~7) + interleaved_pos(c & 7)];
                            else xv = (float)a.x[(int64_t)m * K + c];
                            sacc[m] += v * xv;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float s = group_sum<TPR>(sacc[m]);
            if (sub == 0) sp[m * RT + rl] = s;
        }
    }
    __syncthreads();

    // ---- combine split-K partials, scale, add alpha * sparse, store
    for (int idx = tid; idx < MT * RT; idx += NT) {
        const int m = idx / RT, rl = idx - m * RT;
        const int64_t n = n0 + rl;
        if (m < a.M && n < a.N) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < W; w++) v += red[((w * R + (rl >> 4)) * 16 + m) * 16 + (rl & 15)];
            if (!GROUPED) v *= (float)a.scales[n];
            if (a.has_ortho) v += a.alpha * sp[m * RT + rl];
            a.y[(int64_t)m * a.N + n] = (f16)v;
        }
    }
}

// ------------------------------------------------------------------ host

template <int MT, bool GROUPED, bool XLDS>
static hipError_t launch_decode_t(const DecodeArgs &d, int64_t lds_bytes, hipStream_t stream) {
    constexpr int W = 4, R = 1;
    constexpr int PF = XLDS ? 8 : 4;
    auto kern = decode_kernel<MT, GROUPED, XLDS, W, R, PF>;
    const unsigned blocks = (unsigned)((d.N + 16 * R - 1) / (16 * R));
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * W), (uint32_t)lds_bytes, stream, d);
    return hipGetLastError();
}

template <bool GROUPED, bool XLDS>
static hipError_t launch_decode_mt(int mt, const DecodeArgs &d, int64_t lds, hipStream_t s) {
    switch (mt) {
        case 1: return launch_decode_t<1, GROUPED, XLDS>(d, lds, s);
        case 2: return launch_decode_t<2, GROUPED, XLDS>(d, lds, s);
        case 4: return launch_decode_t<4, GROUPED, XLDS>(d, lds, s);
        case 8: return launch_decode_t<8, GROUPED, XLDS>(d, lds, s);
        default: return launch_decode_t<16, GROUPED, XLDS>(d, lds, s);
    }
}

// Largest activation block staged in LDS; above it the A operand is read
// straight from global memory (L2-resident) with a register prefetch.
static const int64_t kDecodeXLdsMax = 40 * 1024;

bool decode_supported(const ForwardArgs &a) {
    if (a.M < 1 || a.M > 16) return false;
    if (a.io_dtype != ORTH_DT_F16 || a.scale_dtype != ORTH_DT_F16) return false;
    if (a.has_ortho && a.val_dtype != ORTH_DT_F16) return false;
    if (a.K % 128 != 0) return false;
    if (a.ngroups != 1 && (a.G % 128 != 0)) return false;
    if (a.K > (int64_t)1 << 24 || a.N > ((int64_t)1 << 31)) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.x)) & 15) return false;
    return true;
}

hipError_t launch_decode(const ForwardArgs &a, hipStream_t stream) {
    DecodeArgs d;
    d.q = a.q;
    d.scales = static_cast<const f16 *>(a.scales);
    d.ngroups = a.ngroups;
    d.G = a.G;
    d.row_ptr = a.row_ptr;
    d.col = a.col;
    d.vals = static_cast<const f16 *>(a.vals);
    d.nnz = a.nnz;
    d.x = static_cast<const f16 *>(a.x);
    d.y = static_cast<f16 *>(a.y);
    d.M = (int)a.M;
    d.nchunks = (int)(a.K / 128);
    d.K = a.K;
    d.N = a.N;
    d.xstride = (int)(a.K + 8);  // +16 bytes: rows start in different LDS banks
    d.alpha = a.alpha;
    d.has_ortho = a.has_ortho;

    int mt = 1;
    while (mt < a.M) mt <<= 1;
    const bool grouped = a.ngroups != 1;
    const int W = 4, R = 1;
    int64_t lds = (int64_t)W * R * 256 * 4 + (int64_t)mt * 16 * R * 4;
    if (grouped) lds += (int64_t)16 * R * a.ngroups * 2;
    lds = (lds + 15) & ~int64_t(15);
    const int64_t xbytes = (int64_t)mt * d.xstride * 2;
    const bool xlds = xbytes <= kDecodeXLdsMax;
    if (xlds) lds += xbytes + 16;
    if (lds > 64 * 1024) return hipErrorInvalidValue;

    if (grouped) {
        return xlds ? launch_decode_mt<true, true>(mt, d, lds, stream)
                    : launch_decode_mt<true, false>(mt, d, lds, stream);
    }
    return xlds ? launch_decode_mt<false, true>(mt, d, lds, stream)
                : launch_decode_mt<false, false>(mt, d, lds, stream);
}

}  // namespace orth
