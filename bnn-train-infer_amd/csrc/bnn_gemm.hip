// Multi-row jobs (GEMM, GEMM_F32, DOT_GROUPS with rows >= kMfmaMinRows) on the
// gfx950 matrix cores: v_mfma_i32_16x16x64_i8.
//
// The weights of a matrix are expanded once, on its first multi-row job, from
// sign bits to int8 +1/-1 rows (wbytes[n_pad][K], 8x the bit form: HBM capacity
// traded for VALU work, freed with the matrix).  Per 128-weight group g -- the
// unit of the numeric contract (reference bnn-accelerator.h:133-149,
// soft-bnn-accelerator.c:219-276):
//   * two MFMAs per 16x16 output subtile accumulate D = sum_k Q[m][k] * W[n][k]
//     (exact) onto an accumulator initialised to 0x4B400000, so the integer result
//     is 0x4B400000 + D; read as a float that bit pattern is exactly 12582912 + D
//     (|D| <= 16256 < 2^22);
//   * fma(scale, 12582912 + D, -scale * 12582912) is the correctly rounded product
//     scale * D: the constant is exact in binary32 (11 + 2 significant bits), so the
//     fused operation rounds the exact value scale * D once;
//   * the product is added to the FP32 accumulator of (m, n) -- groups in
//     increasing order, one rounding per add.  A zero product comes out as +0
//     where the reference may form -0; the accumulator starts at +0 and never
//     becomes -0 (x + -x == +0 in round-to-nearest), so the sums agree bit for bit.
// DOT_GROUPS initialises the accumulator to 0 and stores D as int16.
// Each group's A (Q rows) and B (weight rows) blocks are staged in LDS, double
// buffered: group g+1 is written while group g is computed, and group g+2 is
// already being loaded into registers.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "bnn_internal.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMagicBits = 0x4B400000;     // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicValue = 12582912.0f;
constexpr int kPitch = 144;                // LDS bytes per staged row: 128 + 16 (bank spread)

__device__ __forceinline__ u32x4 gload16(const void* p) {
    return *(const __attribute__((address_space(1))) u32x4*)p;
}

// 4 sign bits -> 4 bytes of +1 (bit 1) or -1 (bit 0): the multiply places copies of
// the nibble at bit offsets 0, 7, 14, 21 (disjoint), the mask keeps bit i in byte i,
// then 1 -> ~0xFE = 0x01 and 0 -> ~0x00 = 0xFF per byte (no carries).
__device__ __forceinline__ uint32_t pm1_nibble(uint32_t nib) {
    return ~(((nib * 0x204081u) & 0x01010101u) * 0xFEu);
}

__global__ __launch_bounds__(256) void k_expand(const uint4* __restrict__ wbits, uint32_t tiles, uint32_t groups,
                                                uint32_t n_pad, int8_t* __restrict__ wbytes) {
    const uint64_t total = (uint64_t)n_pad * groups;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint32_t n = (uint32_t)(i / groups), g = (uint32_t)(i - (uint64_t)n * groups);
        uint4 b = make_uint4(0u, 0u, 0u, 0u);
        if (n < tiles * kTile)
            b = wbits[((size_t)(n >> 6) * groups + g) * kTile + (n & 63u)];
        const uint32_t w[4] = {b.x, b.y, b.z, b.w};
        u32x4* dst = reinterpret_cast<u32x4*>(wbytes + (size_t)n * groups * kGroup + (size_t)g * kGroup);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 lo, hi;
            lo.x = pm1_nibble(w[q] & 15u);
            lo.y = pm1_nibble((w[q] >> 4) & 15u);
            lo.z = pm1_nibble((w[q] >> 8) & 15u);
            lo.w = pm1_nibble((w[q] >> 12) & 15u);
            hi.x = pm1_nibble((w[q] >> 16) & 15u);
            hi.y = pm1_nibble((w[q] >> 20) & 15u);
            hi.z = pm1_nibble((w[q] >> 24) & 15u);
            hi.w = pm1_nibble(w[q] >> 28);
            dst[2 * q] = lo;
            dst[2 * q + 1] = hi;
        }
    }
}

// Workgroup tile TM x TN = (32*MS) x (32*NS); 4 waves in a 2 x 2 grid, each 16*MS x 16*NS.
template <int MS, int NS, bool DOT>
__global__ __launch_bounds__(256) void k_gemm(GemmJob j, uint32_t mtiles, uint64_t seq,
                                              const uint64_t* __restrict__ flag) {
    constexpr int TM = 32 * MS, TN = 32 * NS;
    constexpr int A_CH = TM * 8 / 256;  // 16-byte chunks per thread and group
    constexpr int B_CH = TN * 8 / 256;
    __shared__ __attribute__((aligned(16))) unsigned char lds_a[2][TM * kPitch];
    __shared__ __attribute__((aligned(16))) unsigned char lds_b[2][TN * kPitch];
    if (*flag == seq)
        return;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    const uint32_t groups = j.groups;
    const uint32_t n_scaled = j.tiles * kTile;  // features covered by the scale layout
    const uint32_t lane_n0 = n0 + wn * 16u * NS + (lane & 15u);

    u32x4 a_reg[A_CH], b_reg[B_CH];
    uint32_t sc_reg[NS];
    auto load_group = [&](uint32_t g) {
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const uint32_t c = tid + 256u * i, row = c >> 3, col = c & 7u;
            const uint32_t m = m0 + row;
            a_reg[i] = m < j.rows ? gload16(j.q + (size_t)m * j.k + (size_t)g * kGroup + col * 16u)
                                  : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const uint32_t c = tid + 256u * i, row = c >> 3, col = c & 7u;
            b_reg[i] = gload16(j.wbytes + (size_t)(n0 + row) * j.k + (size_t)g * kGroup + col * 16u);
        }
        if constexpr (!DOT) {
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                const uint32_t n = lane_n0 + 16u * ni;
                sc_reg[ni] = n < n_scaled ? *(const __attribute__((address_space(1))) uint16_t*)(
                                                j.wscale + ((size_t)(n >> 6) * groups + g) * kTile + (n & 63u))
                                          : 0u;
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const uint32_t c = tid + 256u * i;
            *reinterpret_cast<u32x4*>(lds_a[buf] + (c >> 3) * kPitch + (c & 7u) * 16u) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const uint32_t c = tid + 256u * i;
            *reinterpret_cast<u32x4*>(lds_b[buf] + (c >> 3) * kPitch + (c & 7u) * 16u) = b_reg[i];
        }
    };

    float acc[MS][NS][4];
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
    float sc[NS], cneg[NS];
    auto take_scales = [&]() {
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            sc[ni] = __half2float(__ushort_as_half((uint16_t)sc_reg[ni]));
            cneg[ni] = sc[ni] * -kMagicValue;  // exact
        }
    };

    load_group(0);
    stage(0);
    if (!DOT)
        take_scales();
    if (groups > 1u)
        load_group(1);
    __syncthreads();

    const uint32_t koff = 16u * (lane >> 4);
    const v4i c_init = {DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits};
    for (uint32_t g = 0; g < groups; ++g) {
        const int buf = g & 1u;
        v4i bop[NS][2];
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            const uint32_t brow = wn * 16u * NS + ni * 16u + (lane & 15u);
            bop[ni][0] = *reinterpret_cast<const v4i*>(lds_b[buf] + brow * kPitch + koff);
            bop[ni][1] = *reinterpret_cast<const v4i*>(lds_b[buf] + brow * kPitch + 64u + koff);
        }
#pragma unroll
        for (int mi = 0; mi < MS; ++mi) {
            const uint32_t arow = wm * 16u * MS + mi * 16u + (lane & 15u);
            const v4i a0 = *reinterpret_cast<const v4i*>(lds_a[buf] + arow * kPitch + koff);
            const v4i a1 = *reinterpret_cast<const v4i*>(lds_a[buf] + arow * kPitch + 64u + koff);
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bop[ni][0], c_init, 0, 0, 0);
                d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bop[ni][1], d, 0, 0, 0);
                if constexpr (DOT) {
                    const uint32_t n = lane_n0 + 16u * ni;
                    const uint32_t mrow = m0 + wm * 16u * MS + mi * 16u + 4u * (lane >> 4);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (mrow + r < j.rows && n < j.n)
                            reinterpret_cast<int16_t*>(j.out + (size_t)(mrow + r) * j.out_stride)[(size_t)n * groups + g] =
                                (int16_t)d[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc[ni], __int_as_float(d[r]), cneg[ni]);
                }
            }
        }
        if (g + 1u < groups) {
            stage(buf ^ 1);  // group g+1 (registers loaded one group ago)
            if (!DOT)
                take_scales();
            if (g + 2u < groups)
                load_group(g + 2u);
        }
        __syncthreads();
    }
    if constexpr (DOT)
        return;
    // ---- store Z (or Z * s) ----
#pragma unroll
    for (int mi = 0; mi < MS; ++mi) {
        const uint32_t mrow = m0 + wm * 16u * MS + mi * 16u + 4u * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = mrow + r;
            if (m >= j.rows)
                continue;
            const float s = j.mode == MODE_SUM_SCALED ? j.rscale[m] : 1.0f;
            float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                const uint32_t n = lane_n0 + 16u * ni;
                if (n < j.n)
                    orow[n] = j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * s : acc[mi][ni][r];
            }
        }
    }
}

template <int MS, int NS>
hipError_t launch_t(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + 32u * MS - 1u) / (32u * MS);
    const uint32_t ntiles = (job.n + 32u * NS - 1u) / (32u * NS);
    if (job.mode == MODE_DOT_I16)
        hipLaunchKernelGGL((k_gemm<MS, NS, true>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq,
                           flag);
    else
        hipLaunchKernelGGL((k_gemm<MS, NS, false>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq,
                           flag);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_expand(hipStream_t stream, const uint4* wbits, uint32_t tiles, uint32_t groups, uint32_t n_pad,
                         int8_t* wbytes) {
    const uint64_t total = (uint64_t)n_pad * groups;
    uint64_t blocks = (total + 255u) / 256u;
    if (blocks > 4096u)
        blocks = 4096u;
    hipLaunchKernelGGL(k_expand, dim3((uint32_t)blocks), dim3(256), 0, stream, wbits, tiles, groups, n_pad, wbytes);
    return hipGetLastError();
}

// Largest workgroup tile that still gives every CU a workgroup; else the smallest tile.
#ifndef BNN_GEMM_TILE
#define BNN_GEMM_TILE 0  // 0: choose by size; 44 / 24 / 22: force MS x NS
#endif
hipError_t launch_gemm(hipStream_t stream, const GemmJob& job, uint32_t cu_count, uint64_t seq,
                       const uint64_t* flag) {
    const uint64_t cus = cu_count ? cu_count : 256u;
    auto blocks = [&](uint32_t tm, uint32_t tn) {
        return (uint64_t)((job.rows + tm - 1u) / tm) * ((job.n + tn - 1u) / tn);
    };
    if (BNN_GEMM_TILE == 44 || (BNN_GEMM_TILE == 0 && blocks(128, 128) >= cus))
        return launch_t<4, 4>(stream, job, seq, flag);
    if (BNN_GEMM_TILE == 24 || (BNN_GEMM_TILE == 0 && blocks(64, 128) >= cus))
        return launch_t<2, 4>(stream, job, seq, flag);
    return launch_t<2, 2>(stream, job, seq, flag);
}

}  // namespace bnnhip
