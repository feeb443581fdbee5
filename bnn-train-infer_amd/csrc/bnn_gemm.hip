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

// Output elements as nontemporal stores: written once, not kept dirty in the L2s for
// the end-of-kernel release to write back.
__device__ __forceinline__ void store_out(float* p, float v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) float*)p);
}

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
                    store_out(orow + n, j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * s : acc[mi][ni][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_gemm_big: F32-accumulating jobs large enough to give every CU a 128 x 128 tile.
// Workgroup tile 128 x 128 (4 waves, 2 x 2, 64 x 64 each = 4 x 4 MFMA subtiles).
// Per group g (one iteration, one barrier):
//   * the group's A (Q rows) and B (+-1 weight rows) blocks, 16 KB each, and each
//     wave's 64 column scales (128 B) go straight from global memory into LDS
//     (global_load_lds, 16 bytes per lane, no registers), double buffered: group
//     g+1 is issued right after the barrier of iteration g;
//   * every wave issues the same loads (8, plus 1 for the scales), so "my part of
//     group g has landed" is vmcnt(0) before the barrier, and after it the whole
//     group is in LDS;
//   * the epilogue of group g-1 (RN(scale * D) added to the FP32 accumulators) is
//     interleaved subtile by subtile with the first-half MFMAs of group g, which
//     restart that subtile's integer accumulator: VALU and matrix pipes overlap
//     without a second set of accumulator registers.
// LDS layout of a block: 16-byte chunk c (0..7) of row r at r*128 + 16*(c ^ ((r >> 1) & 7)):
// the 16 lanes reading one fragment (rows r0..r0+15, one chunk) hit 16 distinct
// 16-byte bank groups.
// ---------------------------------------------------------------------------
constexpr uint32_t kBigTile = 128;
constexpr uint32_t kBlock = kBigTile * kGroup;  // bytes per operand per group

__device__ __forceinline__ uint32_t swz128(uint32_t r, uint32_t c) { return r * 128u + 16u * (c ^ ((r >> 1) & 7u)); }

// The bijective workgroup remap that keeps consecutive tiles (the M tiles of one
// N tile, which share B) on one XCD and its L2.
__device__ __forceinline__ uint32_t gemm_tile_of_block(uint32_t b, uint32_t grid) {
    const uint32_t x = b % 8u, i = b / 8u, q = grid / 8u, r = grid % 8u;
    return (x < r ? x * (q + 1u) : r * (q + 1u) + (x - r) * q) + i;
}

// 16 bytes per lane from global memory into LDS at lds_addr + 16 * lane (the wave's
// LDS base goes in M0).  Issued as inline assembly so that the compiler's own wait
// insertion does not add a wait for every LDS DMA before each later LDS read: the
// kernel bounds the outstanding loads itself.  The s_nop covers the one wait state
// between writing M0 and the LDS DMA reading it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_addr) : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_big(
    GemmJob j, uint32_t mtiles, uint64_t seq, const uint64_t* __restrict__ flag) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2][2][kBlock];  // [buffer][A/B]
    __shared__ __attribute__((aligned(16))) unsigned char lds_sc[2][4][128];   // [buffer][wave]
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t tile = gemm_tile_of_block(blockIdx.x, gridDim.x);
    const uint32_t mt = tile % mtiles, nt = tile / mtiles;
    const uint32_t m0 = mt * kBigTile, n0 = nt * kBigTile;
    const uint32_t groups = j.groups;

    // this lane's chunks of a block: instruction i of wave w fills positions
    // (4w + i) * 64 + lane, i.e. row r = (4w + i) * 8 + lane / 8, slot lane % 8
    const uint8_t* a_src[4];
    const uint8_t* b_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = (4u * wave + i) * 8u + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ ((r >> 1) & 7u);
        const uint32_t m = min(m0 + r, j.rows - 1u);
        a_src[i] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)m * j.k + 16u * c;
        b_src[i] = reinterpret_cast<const uint8_t*>(j.wbytes) + (size_t)(n0 + r) * j.k + 16u * c;
    }
    // scales of this wave's 64 columns: one 64-feature tile of the scale layout
    // (clamped into the array for columns past the last tile; those are never stored)
    const uint32_t stile = min((n0 + wn * 64u) >> 6, j.tiles - 1u);
    const uint8_t* sc_src = reinterpret_cast<const uint8_t*>(j.wscale) + ((size_t)stile * groups) * 128u + 16u * (lane & 7u);
    const uint32_t lds0 = lds_offset(lds);
    const uint32_t lds_sc0 = lds_offset(lds_sc) + wave * 128u;
    auto issue_group = [&](uint32_t g) {
        const uint32_t koff = g * kGroup;
        const uint32_t buf = lds0 + (g & 1u) * (2u * kBlock);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dma16(a_src[i] + koff, buf + (4u * wave + i) * 1024u);
            dma16(b_src[i] + koff, buf + kBlock + (4u * wave + i) * 1024u);
        }
        if (lane < 8u)
            dma16(sc_src + (size_t)g * 128u, lds_sc0 + (g & 1u) * 512u);
    };

    float acc[4][4][4];
    v4i d[4][4];
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            d[mi][ni] = c_init;  // with scale 0 the first epilogue adds +0
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
        }
    float sc_prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    issue_group(0);

    const uint32_t arow0 = wm * 64u + (lane & 15u), brow0 = wn * 64u + (lane & 15u);
    const uint32_t chunk = lane >> 4;
    for (uint32_t g = 0; g < groups; ++g) {
        // only group g is outstanding; after the barrier every wave's part of it is
        // in LDS, and every wave has finished reading the other buffer (group g-1:
        // its MFMAs consumed those registers)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (g + 1u < groups)
            issue_group(g + 1u);
        const unsigned char* blk = lds[g & 1u][0];
        const uint16_t* scl = reinterpret_cast<const uint16_t*>(lds_sc[g & 1u][wave]);
        float sc_cur[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            sc_cur[ni] = __half2float(__ushort_as_half(scl[16u * ni + (lane & 15u)]));
        v4i a[4], b[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(blk + swz128(arow0 + 16u * mi, chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(blk + kBlock + swz128(brow0 + 16u * ni, chunk));
        // first half: epilogue of group g-1 on each subtile, then restart it
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const float sc = sc_prev[ni];
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], c_init, 0, 0, 0);
            }
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(blk + swz128(arow0 + 16u * mi, 4u + chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(blk + kBlock + swz128(brow0 + 16u * ni, 4u + chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], d[mi][ni], 0, 0, 0);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            sc_prev[ni] = sc_cur[ni];
        // issue order: the 12 LDS reads of the scales and first half, then per
        // subtile its 8 epilogue VALU ops and its restarting MFMA (the matrix pipe
        // runs while the next subtile's VALU ops issue), the second-half LDS reads
        // spread among them, then the 16 second-half MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i >= 4 && i < 12)
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
    }
    // epilogue of the last group, then store Z (or Z * s)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const float sc = sc_prev[ni];
        const float cneg = sc * -kMagicValue;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
    }
    const uint32_t ncol0 = n0 + wn * 64u + (lane & 15u);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + wm * 64u + 16u * mi + 4u * (lane >> 4) + r;
            if (m >= j.rows)
                continue;
            const float s = j.mode == MODE_SUM_SCALED ? j.rscale[m] : 1.0f;
            float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const uint32_t n = ncol0 + 16u * ni;
                if (n < j.n)
                    store_out(orow + n, j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * s : acc[mi][ni][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_gemm_pipe<MI>: F32-accumulating jobs on (32*MI) x 128 workgroup tiles (4 waves,
// 2 x 2, each (16*MI) x 64 = MI x 4 MFMA subtiles).  K streams through LDS in
// stages of half a group (64 bytes of every A and B row: one MFMA step), with four
// LDS slots: stage h+3 is issued right after the barrier of stage h, so three
// stages in flight (about 1.5 groups of compute) cover the global->LDS latency.
//   * every wave issues the same DMAs per stage (its share of the A and B blocks,
//     plus, for the first half of a group, its 64 columns' scales), so the wait for
//     stage h is a fixed count of younger DMAs (vmcnt), then one barrier;
//   * the DMA source is a uniform 64-bit base in SGPRs (advanced by K per stage)
//     plus a per-lane offset fixed for the whole loop: no VALU work per DMA;
//   * the epilogue of group g-1 (RN(scale * D) added in group order, as in
//     k_gemm_big) is interleaved subtile by subtile with the first-half MFMAs of
//     group g, which restart that subtile's integer accumulator.
// LDS layout of a stage block: 16-byte chunk c (0..3) of row r at r*64 + 16*(c ^ ((r >> 1) & 3)):
// the 16 lanes reading one fragment (16 rows, one chunk) are spread over the banks.
// ---------------------------------------------------------------------------
constexpr uint32_t kPipeSlots = 4;
constexpr uint32_t kHalf = 64;  // K bytes per stage

__device__ __forceinline__ uint32_t swz64(uint32_t r, uint32_t c) { return r * 64u + 16u * (c ^ ((r >> 1) & 3u)); }

// 16 bytes per lane from sbase + voff into LDS at lds_addr + 16 * lane (see dma16)
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

// vmcnt(N) and lgkmcnt(0): at most N of this wave's DMAs still in flight, and its LDS
// reads done -- before a barrier after which other waves refill the slot it read
template <int N>
__device__ __forceinline__ void wait_stage() {
    static_assert(N >= 0 && N < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0070 | N);
}

template <int MI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_pipe(
    GemmJob j, uint32_t mtiles, uint64_t seq, const uint64_t* __restrict__ flag) {
    constexpr uint32_t TM = 32u * MI, TN = 128u;
    constexpr uint32_t A_BYTES = TM * kHalf, B_BYTES = TN * kHalf, SLOT = A_BYTES + B_BYTES;
    constexpr uint32_t A_INS = A_BYTES / 1024u / 4u, B_INS = B_BYTES / 1024u / 4u;  // DMAs per wave and stage
    constexpr int P = (int)(A_INS + B_INS);
    static_assert(A_INS >= 1 && 2 * P + 1 < 16, "stage DMAs");
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kPipeSlots][SLOT];
    __shared__ __attribute__((aligned(16))) unsigned char lds_sc[4][4][128];  // [group % 4][wave]
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t tile = gemm_tile_of_block(blockIdx.x, gridDim.x);
    const uint32_t mt = tile % mtiles, nt = tile / mtiles;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    const uint32_t groups = j.groups, stages = 2u * groups;

    // DMA instruction i of wave w fills block positions p = (w * INS + i) * 64 + lane:
    // row p / 4, stored chunk p % 4 = logical chunk ^ ((row >> 1) & 3); A rows past
    // the job are clamped (never stored), B rows stay below n_pad
    uint32_t a_off[A_INS], b_off[B_INS];
#pragma unroll
    for (uint32_t i = 0; i < A_INS; ++i) {
        const uint32_t p = (wave * A_INS + i) * 64u + lane, r = p >> 2;
        const uint32_t c = (p & 3u) ^ ((r >> 1) & 3u);
        a_off[i] = (min(m0 + r, j.rows - 1u) - m0) * j.k + 16u * c;
    }
#pragma unroll
    for (uint32_t i = 0; i < B_INS; ++i) {
        const uint32_t p = (wave * B_INS + i) * 64u + lane, r = p >> 2;
        const uint32_t c = (p & 3u) ^ ((r >> 1) & 3u);
        b_off[i] = r * j.k + 16u * c;
    }
    const uint8_t* a_base = reinterpret_cast<const uint8_t*>(j.q) + (size_t)m0 * j.k;
    const uint8_t* b_base = reinterpret_cast<const uint8_t*>(j.wbytes) + (size_t)n0 * j.k;
    // this wave's 64 columns' scales: one 64-feature tile of the scale layout (clamped
    // into the array for columns past the last tile; those are never stored)
    const uint32_t stile = min((n0 + wn * 64u) >> 6, j.tiles - 1u);
    const uint8_t* sc_base = reinterpret_cast<const uint8_t*>(j.wscale) + (size_t)stile * groups * 128u;
    const uint32_t lds0 = lds_offset(lds);
    const uint32_t lds_sc0 = lds_offset(lds_sc) + wave * 128u;
    // stage h (h past the last stage reloads the last one into a free slot: every
    // stage issues the same DMAs, so the wait counts are the same throughout)
    auto issue = [&](uint32_t h, bool first_half) {
        const uint32_t hs = min(h, stages - 1u);
        const uint32_t koff = (hs >> 1) * kGroup + (hs & 1u) * kHalf;
        const uint32_t slot = lds0 + (h % kPipeSlots) * SLOT;
#pragma unroll
        for (uint32_t i = 0; i < A_INS; ++i)
            dma16s(a_base + koff, a_off[i], slot + (wave * A_INS + i) * 1024u);
#pragma unroll
        for (uint32_t i = 0; i < B_INS; ++i)
            dma16s(b_base + koff, b_off[i], slot + A_BYTES + (wave * B_INS + i) * 1024u);
        if (first_half && lane < 8u)
            dma16s(sc_base + (size_t)(hs >> 1) * 128u, 16u * lane, lds_sc0 + ((h >> 1) & 3u) * 512u);
    };

    float acc[MI][4][4];
    v4i d[MI][4];
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            d[mi][ni] = c_init;  // with scale 0 the first epilogue adds +0
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
        }
    float sc_prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    issue(0, true);
    issue(1, false);
    issue(2, true);

    const uint32_t arow0 = wm * 16u * MI + (lane & 15u), brow0 = wn * 64u + (lane & 15u);
    const uint32_t chunk = lane >> 4;
    for (uint32_t g = 0; g < groups; ++g) {
        // ---- first half of group g (stage 2g): stages 2g+1 and 2g+2 stay in flight
        wait_stage<2 * P + 1>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(2u * g + 3u, false);
        const unsigned char* blk = lds[(2u * g) % kPipeSlots];
        const uint16_t* scl = reinterpret_cast<const uint16_t*>(lds_sc[g & 3u][wave]);
        float sc_cur[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            sc_cur[ni] = __half2float(__ushort_as_half(scl[16u * ni + (lane & 15u)]));
        v4i a[MI], b[4];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(blk + swz64(arow0 + 16u * mi, chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(blk + A_BYTES + swz64(brow0 + 16u * ni, chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const float sc = sc_prev[ni];
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], c_init, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, MI + 8, 0);
#pragma unroll
        for (int i = 0; i < 4 * MI; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        // ---- second half (stage 2g+1): stages 2g+2 and 2g+3 stay in flight
        wait_stage<2 * P + 1>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(2u * g + 4u, true);
        blk = lds[(2u * g + 1u) % kPipeSlots];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(blk + swz64(arow0 + 16u * mi, chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(blk + A_BYTES + swz64(brow0 + 16u * ni, chunk));
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], d[mi][ni], 0, 0, 0);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            sc_prev[ni] = sc_cur[ni];
    }
    // no DMA may still be writing this workgroup's LDS when it ends
    wait_stage<0>();
    // epilogue of the last group, then store Z (or Z * s)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const float sc = sc_prev[ni];
        const float cneg = sc * -kMagicValue;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
    }
    const uint32_t ncol0 = n0 + wn * 64u + (lane & 15u);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + wm * 16u * MI + 16u * mi + 4u * (lane >> 4) + r;
            if (m >= j.rows)
                continue;
            const float s = j.mode == MODE_SUM_SCALED ? j.rscale[m] : 1.0f;
            float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const uint32_t n = ncol0 + 16u * ni;
                if (n < j.n)
                    store_out(orow + n, j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * s : acc[mi][ni][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_gemm_ks: F32-accumulating jobs too small to give every CU a 128 x 128 tile.
// Workgroup tile (16*TMS) x (16*TNS); the W waves split the K dimension instead of
// the tile: wave w computes groups w, w+W, w+2W, ... for the whole tile, with its
// operands loaded straight into registers DEPTH-1 rounds ahead.  Per round of W
// groups each wave turns its integer results into the exact products
// RN(scale * D) (the same magic-bias FMA as above) and writes them to LDS; then the
// threads add the W products of their outputs to their FP32 accumulators in group
// order -- the order of the sums is the reference's, only the integer work ran in
// parallel.
// ---------------------------------------------------------------------------
__device__ __forceinline__ v4i gload_v4i(const void* p) {
    return *(const __attribute__((address_space(1))) v4i*)p;
}

template <int TMS, int TNS>
struct KsOps {
    v4i a[TMS][2];
    v4i b[TNS][2];
    uint16_t s[TNS];
};

template <int TMS, int TNS, int W, int DEPTH>
__global__ __launch_bounds__(64 * W) void k_gemm_ks(GemmJob j, uint32_t mtiles, uint64_t seq,
                                                   const uint64_t* __restrict__ flag) {
    constexpr uint32_t TM = 16u * TMS, TN = 16u * TNS, SUBS = TMS * TNS, NT = 64u * W;
    constexpr uint32_t BLOCKS = SUBS * 64u;              // 16-byte blocks of products per wave
    constexpr uint32_t PER_THREAD = (BLOCKS + NT - 1u) / NT;
    static_assert(DEPTH >= 2, "at least one round in flight");
    __shared__ __attribute__((aligned(16))) float prod[W][BLOCKS * 4u];  // [wave][subtile][lane][4]
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tile = gemm_tile_of_block(blockIdx.x, gridDim.x);
    const uint32_t mt = tile % mtiles, nt = tile / mtiles;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    const uint32_t groups = j.groups;

    // lane l supplies row (or column) l % 16 of a subtile and bytes 16*(l/16) .. +16 of
    // each 64-byte half group; rows past the end are clamped (never stored), columns
    // stay below n_pad (TN divides 128) and their scale tile is clamped into the array
    const uint8_t* a_ptr[TMS];
    const uint8_t* b_ptr[TNS];
    const uint16_t* s_ptr[TNS];
#pragma unroll
    for (int mi = 0; mi < TMS; ++mi) {
        const uint32_t m = min(m0 + 16u * mi + (lane & 15u), j.rows - 1u);
        a_ptr[mi] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)m * j.k + 16u * (lane >> 4);
    }
#pragma unroll
    for (int ni = 0; ni < TNS; ++ni) {
        const uint32_t n = n0 + 16u * ni + (lane & 15u);
        b_ptr[ni] = reinterpret_cast<const uint8_t*>(j.wbytes) + (size_t)n * j.k + 16u * (lane >> 4);
        const uint32_t st = min(n >> 6, j.tiles - 1u);
        s_ptr[ni] = reinterpret_cast<const uint16_t*>(j.wscale) + (size_t)st * groups * kTile + (n & 63u);
    }
    // loads are unconditional (group clamped into range) so that every path has the
    // same loads in flight and the wait for a round's operands leaves the later
    // rounds' loads outstanding
    auto load = [&](KsOps<TMS, TNS>& o, uint32_t round) {
        const uint32_t g = min(W * round + wave, groups - 1u);
#pragma unroll
        for (int mi = 0; mi < TMS; ++mi)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                o.a[mi][h] = gload_v4i(a_ptr[mi] + (size_t)g * kGroup + 64u * h);
#pragma unroll
        for (int ni = 0; ni < TNS; ++ni)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                o.b[ni][h] = gload_v4i(b_ptr[ni] + (size_t)g * kGroup + 64u * h);
#pragma unroll
        for (int ni = 0; ni < TNS; ++ni)
            o.s[ni] = s_ptr[ni][(size_t)g * kTile];
    };

    float acc[PER_THREAD][4];
#pragma unroll
    for (int i = 0; i < (int)PER_THREAD; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[i][r] = 0.0f;
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};

    auto round = [&](const KsOps<TMS, TNS>& cur, KsOps<TMS, TNS>& nxt, uint32_t r) {
        load(nxt, r + DEPTH - 1u);
        const uint32_t g = W * r + wave;
        float4 p[TMS][TNS];
        if (g < groups) {
#pragma unroll
            for (int ni = 0; ni < TNS; ++ni) {
                const float sc = __half2float(__ushort_as_half(cur.s[ni]));
                const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
                for (int mi = 0; mi < TMS; ++mi) {
                    v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][0], cur.b[ni][0], c_init, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][1], cur.b[ni][1], d, 0, 0, 0);
                    p[mi][ni].x = __builtin_fmaf(sc, __int_as_float(d[0]), cneg);
                    p[mi][ni].y = __builtin_fmaf(sc, __int_as_float(d[1]), cneg);
                    p[mi][ni].z = __builtin_fmaf(sc, __int_as_float(d[2]), cneg);
                    p[mi][ni].w = __builtin_fmaf(sc, __int_as_float(d[3]), cneg);
                }
            }
        }
        // the previous round's reads of prod are done (their sums consumed them)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (g < groups) {
#pragma unroll
            for (int mi = 0; mi < TMS; ++mi)
#pragma unroll
                for (int ni = 0; ni < TNS; ++ni)
                    *reinterpret_cast<float4*>(&prod[wave][((mi * TNS + ni) * 64u + lane) * 4u]) = p[mi][ni];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int w = 0; w < W; ++w) {
            if (W * r + w < groups) {
#pragma unroll
                for (int i = 0; i < (int)PER_THREAD; ++i) {
                    const uint32_t blk = NT * i + tid;
                    if (BLOCKS % NT == 0 || blk < BLOCKS) {
                        const float4 v = *reinterpret_cast<const float4*>(&prod[w][blk * 4u]);
                        acc[i][0] = acc[i][0] + v.x;
                        acc[i][1] = acc[i][1] + v.y;
                        acc[i][2] = acc[i][2] + v.z;
                        acc[i][3] = acc[i][3] + v.w;
                    }
                }
            }
        }
    };

    KsOps<TMS, TNS> o[DEPTH];
#pragma unroll
    for (int d = 0; d + 1 < DEPTH; ++d)
        load(o[d], d);
    const uint32_t rounds = (groups + W - 1u) / W;
    // the round count is padded to a multiple of DEPTH with rounds of no groups
    for (uint32_t r = 0; r < rounds; r += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            round(o[d], o[(d + DEPTH - 1) % DEPTH], r + d);
    }
    // block NT*i + tid is subtile W*i + wave, lane `lane`
#pragma unroll
    for (int i = 0; i < (int)PER_THREAD; ++i) {
        const uint32_t sub = W * i + wave;
        if (sub >= SUBS)
            continue;
        const uint32_t mi = sub / TNS, ni = sub % TNS;
        const uint32_t n = n0 + 16u * ni + (lane & 15u);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + 16u * mi + 4u * (lane >> 4) + r;
            if (m >= j.rows || n >= j.n)
                continue;
            float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
            store_out(orow + n, j.mode == MODE_SUM_SCALED ? acc[i][r] * j.rscale[m] : acc[i][r]);
        }
    }
}

template <int TMS, int TNS, int W, int DEPTH>
hipError_t launch_ks(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + 16u * TMS - 1u) / (16u * TMS);
    const uint32_t ntiles = (job.n + 16u * TNS - 1u) / (16u * TNS);
    launch_kernel((k_gemm_ks<TMS, TNS, W, DEPTH>), dim3(mtiles * ntiles), dim3(64 * W), 0, stream, job, mtiles,
                       seq, flag);
    return hipGetLastError();
}

template <int MS, int NS>
hipError_t launch_t(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + 32u * MS - 1u) / (32u * MS);
    const uint32_t ntiles = (job.n + 32u * NS - 1u) / (32u * NS);
    if (job.mode == MODE_DOT_I16)
        launch_kernel((k_gemm<MS, NS, true>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq,
                           flag);
    else
        launch_kernel((k_gemm<MS, NS, false>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq,
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
    launch_kernel(k_expand, dim3((uint32_t)blocks), dim3(256), 0, stream, wbits, tiles, groups, n_pad, wbytes);
    return hipGetLastError();
}

// Largest workgroup tile that still gives every CU a workgroup; else the smallest tile.
#ifndef BNN_GEMM_TILE
#define BNN_GEMM_TILE 0  // 0: choose by size; 44 / 24 / 22: force MS x NS
#endif
#ifndef BNN_GEMM_KS
#define BNN_GEMM_KS 0  // tuning: TMS TNS W DEPTH (four digits) forces k_gemm_ks with that shape
#endif
#ifndef BNN_GEMM_PIPE
#define BNN_GEMM_PIPE 1  // k_gemm_pipe for F32-accumulating jobs with enough 128 x 128 or 64 x 128 tiles
#endif
#ifndef BNN_GEMM_BIG
#define BNN_GEMM_BIG 1  // k_gemm_big for F32-accumulating jobs with a 128 x 128 tile per CU
#endif
hipError_t launch_gemm(hipStream_t stream, const GemmJob& job, uint32_t cu_count, uint64_t seq,
                       const uint64_t* flag) {
    const uint64_t cus = cu_count ? cu_count : 256u;
    auto blocks = [&](uint32_t tm, uint32_t tn) {
        return (uint64_t)((job.rows + tm - 1u) / tm) * ((job.n + tn - 1u) / tn);
    };
#if BNN_GEMM_PIPE
    // 128 x 128 tiles for every CU: k_gemm_big (measured 30.9 vs 32.5 us for k_gemm_pipe<4>
    // at 1024 x 2048 x 6144); fewer: the pipelined kernel on 64 x 128 tiles when those
    // give most CUs one (6144 -> 2048 at 1024 rows: 35 vs 62 us for 64 x 128 k_gemm)
    if (job.mode != MODE_DOT_I16 && blocks(128, 128) < cus && blocks(64, 128) >= cus * 3u / 4u) {
        const uint32_t mtiles = (job.rows + 63u) / 64u, ntiles = (job.n + 127u) / 128u;
        launch_kernel(k_gemm_pipe<2>, dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq, flag);
        return hipGetLastError();
    }
#endif
    if (BNN_GEMM_BIG && job.mode != MODE_DOT_I16 && blocks(kBigTile, kBigTile) >= cus) {
        const uint32_t mtiles = (job.rows + kBigTile - 1u) / kBigTile;
        const uint32_t ntiles = (job.n + kBigTile - 1u) / kBigTile;
        launch_kernel(k_gemm_big, dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq, flag);
        return hipGetLastError();
    }
#if BNN_GEMM_KS
    if (job.mode != MODE_DOT_I16) {
        // tuning: BNN_GEMM_KS = TMS TNS W DEPTH as four digits
        constexpr int v = BNN_GEMM_KS;
        return launch_ks<v / 1000, (v / 100) % 10, (v / 10) % 10, v % 10>(stream, job, seq, flag);
    }
#else
    // too few 64 x 64 tiles to occupy the CUs: split K across 8 waves per tile, with
    // the largest tile that still yields about a workgroup per CU (measured on the
    // 64/256-row 2048x6144 and 6144x2048 shapes)
    if (BNN_GEMM_TILE == 0 && job.mode != MODE_DOT_I16 && blocks(64, 64) < cus) {
        const uint64_t enough = cus * 3u / 4u;
        if (blocks(64, 32) >= enough)
            return launch_ks<4, 2, 8, 2>(stream, job, seq, flag);
        if (blocks(32, 32) >= enough)
            return launch_ks<2, 2, 8, 2>(stream, job, seq, flag);
        return launch_ks<2, 1, 8, 3>(stream, job, seq, flag);
    }
#endif
    if (BNN_GEMM_TILE == 44 || (BNN_GEMM_TILE == 0 && blocks(128, 128) >= cus))
        return launch_t<4, 4>(stream, job, seq, flag);
    if (BNN_GEMM_TILE == 24 || (BNN_GEMM_TILE == 0 && blocks(64, 128) >= cus))
        return launch_t<2, 4>(stream, job, seq, flag);
    return launch_t<2, 2>(stream, job, seq, flag);
}

}  // namespace bnnhip
