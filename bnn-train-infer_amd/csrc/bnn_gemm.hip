// Multi-row jobs (GEMM, GEMM_F32, DOT_GROUPS with rows >= kMfmaMinRows) on the
// gfx950 matrix cores (v_mfma_i32_16x16x64_i8), fed from the matrix's resident
// 1.125-bit layout: the sign bits of each 128-weight group are unpacked to +1/-1
// bytes in LDS, per workgroup tile and group, right before the MFMAs use them.
//
// Numeric contract (reference bnn-accelerator.h:133-149, soft-bnn-accelerator.c:219-276),
// per 128-weight group g:
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
// DOT_GROUPS restarts the accumulator at 0 and stores D itself as int16.
//
// k_gemm_bits<TM, TN>: workgroup tile TM x TN, 4 waves (2 x 2) of (TM/2) x (TN/2).
// Everything a group needs reaches LDS by DMA (global_load_lds, 16 bytes per lane,
// no registers): the TM rows' 128 quantised bytes, the TN features' 16-byte sign-bit
// chunks (1 KiB per 64-feature tile of the matrix layout) and each wave's column
// scales.  Iteration g, after one wait and one barrier:
//   * issue the DMAs of group g+1's rows, group g+3's bits and group g+2's scales;
//   * unpack group g+1's bits into its +1/-1 tile: every thread turns 4 or 8 bytes
//     of bits into 32 or 64 bytes with one 8-byte lookup per byte in a 256-entry
//     table (2 KiB, built at start), i.e. ~0.25 VALU op per weight;
//   * group g's MFMAs, interleaved subtile by subtile with group g-1's epilogue.
// The bits run three groups ahead of the MFMAs (they come from HBM), the rows one
// (they are shared by every column tile and come from the L2).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "bnn_internal.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMagicBits = 0x4B400000;  // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicValue = 12582912.0f;

// Output elements as nontemporal stores: written once, not kept dirty in the L2s for
// the end-of-kernel release to write back.
__device__ __forceinline__ void store_out(float* p, float v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) float*)p);
}

// 4 sign bits -> 4 bytes of +1 (bit 1) or -1 (bit 0): the multiply places copies of
// the nibble at bit offsets 0, 7, 14, 21 (disjoint), the mask keeps bit i in byte i,
// then 1 -> ~0xFE = 0x01 and 0 -> ~0x00 = 0xFF per byte (no carries).
__device__ __forceinline__ uint32_t pm1_nibble(uint32_t nib) {
    return ~(((nib * 0x204081u) & 0x01010101u) * 0xFEu);
}

// A 128-byte LDS row holds 8 chunks of 16 bytes; chunk c of row r sits at
// r*128 + 16*(c ^ ((r >> 1) & 7)): the 16 lanes reading one MFMA fragment (16 rows,
// one chunk) hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ uint32_t swz128(uint32_t r, uint32_t c) { return r * 128u + 16u * (c ^ ((r >> 1) & 7u)); }

// The bijective workgroup remap that keeps consecutive tiles (the M tiles of one
// N tile, which share the weights) on one XCD and its L2.
__device__ __forceinline__ uint32_t gemm_tile_of_block(uint32_t b, uint32_t grid) {
    const uint32_t x = b % 8u, i = b / 8u, q = grid / 8u, r = grid % 8u;
    return (x < r ? x * (q + 1u) : r * (q + 1u) + (x - r) * q) + i;
}

// 16 bytes per active lane from global memory into LDS at lds_addr + 16 * lane (the
// wave's LDS base goes in M0).  Inline assembly, so that the compiler's own wait
// insertion does not add a wait for every LDS DMA before each later LDS read: the
// kernel bounds the outstanding loads itself.  The s_nop covers the one wait state
// between writing M0 and the LDS DMA reading it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_addr) : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// vmcnt(N) and lgkmcnt(0): at most N of this wave's DMAs in flight, its LDS reads and
// writes done
template <int N>
__device__ __forceinline__ void wait_dma() {
    static_assert(N >= 0 && N < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0070 | N);
}

template <int TM, int TN, bool DOT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_bits(
    GemmJob j, uint32_t mtiles, uint64_t seq, const uint64_t* __restrict__ flag) {
    constexpr int MS = TM / 32, NS = TN / 32;  // 16 x 16 subtiles per wave
    constexpr uint32_t A_INS = TM / 32;        // row DMAs per wave and group
    constexpr uint32_t BIT_LANES = TN / 4;     // lanes of a wave carrying bits (TN * 16 B per group)
    constexpr uint32_t SC_LANES = TN / 16;     // lanes carrying a wave's TN/2 column scales
    constexpr uint32_t BPT = TN / 16;          // bytes of bits each thread unpacks per group
    static_assert(MS >= 1 && (TN == 64 || TN == 128), "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char lds_a[2][TM * 128];
    __shared__ __attribute__((aligned(1024))) unsigned char lds_b[2][TN * 128];
    __shared__ __attribute__((aligned(16))) unsigned char lds_bits[4][TN * 16];
    __shared__ __attribute__((aligned(16))) unsigned char lds_sc[4][4][TN];  // [slot][wave][TN/2 fp16]
    __shared__ uint2 lut[256];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t tile = gemm_tile_of_block(blockIdx.x, gridDim.x);
    const uint32_t mt = tile % mtiles, nt = tile / mtiles;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    const uint32_t groups = j.groups;

    // byte b of sign bits -> 8 bytes of +1/-1 (bit i -> byte i)
    lut[tid] = make_uint2(pm1_nibble(tid & 15u), pm1_nibble(tid >> 4));

    // this lane's DMA sources (without the group offset)
    const uint8_t* a_src[A_INS];
#pragma unroll
    for (uint32_t i = 0; i < A_INS; ++i) {
        const uint32_t p = (wave * A_INS + i) * 64u + lane, r = p >> 3;
        const uint32_t c = (p & 7u) ^ ((r >> 1) & 7u);
        a_src[i] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)min(m0 + r, j.rows - 1u) * j.k + 16u * c;
    }
    // bits: feature f = BIT_LANES * wave + lane of the tile; its 64-feature matrix tile
    // is clamped into the array (features past the last tile are never stored)
    const uint32_t f = BIT_LANES * wave + lane;
    const uint32_t bit_tile = min((n0 + f) >> 6, j.tiles - 1u);
    const uint8_t* bit_src = reinterpret_cast<const uint8_t*>(j.wbits) + ((size_t)bit_tile * groups * kTile + (f & 63u)) * 16u;
    // scales of this wave's TN/2 columns: part of one 64-feature tile
    const uint32_t col0 = n0 + wn * (TN / 2u);
    const uint32_t sc_tile = min(col0 >> 6, j.tiles - 1u);
    const uint8_t* sc_src = reinterpret_cast<const uint8_t*>(j.wscale) +
                            ((size_t)sc_tile * groups * kTile + (col0 & 63u)) * 2u + 16u * lane;
    const uint32_t la0 = lds_offset(lds_a), lbits0 = lds_offset(lds_bits), lsc0 = lds_offset(lds_sc);
    const size_t bit_step = (size_t)kTile * 16u, sc_step = (size_t)kTile * 2u;  // bytes per group
    auto issue_rows = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
#pragma unroll
        for (uint32_t i = 0; i < A_INS; ++i)
            dma16(a_src[i] + (size_t)gg * kGroup, la0 + (g & 1u) * (TM * 128u) + (wave * A_INS + i) * 1024u);
    };
    auto issue_bits = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        if (lane < BIT_LANES)
            dma16(bit_src + gg * bit_step, lbits0 + (g & 3u) * (TN * 16u) + wave * (BIT_LANES * 16u));
    };
    auto issue_scales = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        if (lane < SC_LANES)
            dma16(sc_src + gg * sc_step, lsc0 + (g & 3u) * (4u * TN) + wave * TN);
    };
    // unpacks group g's bits (slot g % 4) into the +1/-1 tile lds_b[g % 2]
    auto unpack = [&](uint32_t g) {
        constexpr uint32_t PER_ROW = 16u / BPT;  // threads per feature
        const uint32_t row = tid / PER_ROW, part = tid % PER_ROW;
        const unsigned char* src = lds_bits[g & 3u] + row * 16u + part * BPT;
        uint32_t w[BPT / 4];
#pragma unroll
        for (uint32_t i = 0; i < BPT / 4; ++i)
            w[i] = reinterpret_cast<const uint32_t*>(src)[i];
#pragma unroll
        for (uint32_t c = 0; c < BPT / 2; ++c) {  // 16 expanded bytes = 2 bytes of bits per chunk
            const uint32_t word = w[c / 2], sh = 16u * (c & 1u);
            const uint2 lo = lut[(word >> sh) & 0xffu], hi = lut[(word >> (sh + 8u)) & 0xffu];
            *reinterpret_cast<uint4*>(lds_b[g & 1u] + swz128(row, part * (BPT / 2) + c)) =
                make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
    };

    float acc[MS][NS][4];
    v4i d[MS][NS];
    const v4i c_init = {DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits, DOT ? 0 : kMagicBits};
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            d[mi][ni] = c_init;  // with scale 0 the first epilogue adds +0
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
        }

    issue_bits(0);
    issue_scales(0);
    issue_bits(1);
    issue_scales(1);
    issue_bits(2);
    issue_rows(0);
    wait_dma<0>();
    __builtin_amdgcn_s_barrier();  // the table and group 0's bits are in LDS
    asm volatile("" ::: "memory");
    unpack(0);

    const uint32_t arow0 = wm * (TM / 2u) + (lane & 15u), brow0 = wn * (TN / 2u) + (lane & 15u);
    const uint32_t chunk = lane >> 4;
    const uint32_t row_base = m0 + wm * (TM / 2u) + 4u * (lane >> 4);
    const uint32_t col_base = n0 + wn * (TN / 2u) + (lane & 15u);
    float sc_prev[NS];
#pragma unroll
    for (int ni = 0; ni < NS; ++ni)
        sc_prev[ni] = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) {
        // group g's rows have landed (only the bits and scales issued one iteration ago
        // may be in flight), every wave's unpacked tile of group g is written, and every
        // wave has finished reading the buffers of group g-1
        wait_dma<2>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_rows(g + 1u);
        issue_bits(g + 3u);
        issue_scales(g + 2u);
        if (g + 1u < groups)
            unpack(g + 1u);
        const unsigned char* la = lds_a[g & 1u];
        const unsigned char* lb = lds_b[g & 1u];
        const uint16_t* scl = reinterpret_cast<const uint16_t*>(lds_sc[g & 3u][wave]);
        float sc_cur[NS];
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_cur[ni] = DOT ? 0.0f : __half2float(__ushort_as_half(scl[16u * ni + (lane & 15u)]));
        v4i a[MS], b[NS];
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(la + swz128(arow0 + 16u * mi, chunk));
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(lb + swz128(brow0 + 16u * ni, chunk));
        // first half: the epilogue of group g-1 on each subtile, then restart it
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            const float sc = sc_prev[ni];
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (int mi = 0; mi < MS; ++mi) {
                if constexpr (DOT) {
                    // D of group g-1 as int16 at [m][n][g-1]
                    const uint32_t n = col_base + 16u * ni;
                    if (g > 0 && n < j.n) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t m = row_base + 16u * mi + r;
                            if (m < j.rows)
                                reinterpret_cast<int16_t*>(j.out + (size_t)m * j.out_stride)[(size_t)n * groups + g - 1u] =
                                    (int16_t)d[mi][ni][r];
                        }
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
                }
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], c_init, 0, 0, 0);
            }
        }
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(la + swz128(arow0 + 16u * mi, 4u + chunk));
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(lb + swz128(brow0 + 16u * ni, 4u + chunk));
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int mi = 0; mi < MS; ++mi)
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b[ni], d[mi][ni], 0, 0, 0);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_prev[ni] = sc_cur[ni];
        if constexpr (!DOT) {
            // issue order: the LDS reads of the scales and first half, then per subtile
            // its 8 epilogue VALU ops and its restarting MFMA (the matrix pipe runs while
            // the next subtile's VALU ops issue), then the second-half MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, MS + 2 * NS, 0);
#pragma unroll
            for (int i = 0; i < MS * NS; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, MS * NS, 0);
        }
    }
    // no DMA may still be writing this workgroup's LDS when it ends
    wait_dma<0>();
    if constexpr (DOT) {
        // D of the last group
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                const uint32_t n = col_base + 16u * ni;
                if (n >= j.n)
                    continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t m = row_base + 16u * mi + r;
                    if (m < j.rows)
                        reinterpret_cast<int16_t*>(j.out + (size_t)m * j.out_stride)[(size_t)n * groups + groups - 1u] =
                            (int16_t)d[mi][ni][r];
                }
            }
        return;
    }
    // epilogue of the last group, then store Z (or Z * s)
#pragma unroll
    for (int ni = 0; ni < NS; ++ni) {
        const float sc = sc_prev[ni];
        const float cneg = sc * -kMagicValue;
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
    }
#pragma unroll
    for (int mi = 0; mi < MS; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = row_base + 16u * mi + r;
            if (m >= j.rows)
                continue;
            const float s = j.mode == MODE_SUM_SCALED ? j.rscale[m] : 1.0f;
            float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                const uint32_t n = col_base + 16u * ni;
                if (n < j.n)
                    store_out(orow + n, j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * s : acc[mi][ni][r]);
            }
        }
    }
}

template <int TM, int TN>
hipError_t launch_bits(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + TM - 1u) / TM, ntiles = (job.n + TN - 1u) / TN;
    if (job.mode == MODE_DOT_I16)
        launch_kernel((k_gemm_bits<TM, TN, true>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq, flag);
    else
        launch_kernel((k_gemm_bits<TM, TN, false>), dim3(mtiles * ntiles), dim3(256), 0, stream, job, mtiles, seq,
                      flag);
    return hipGetLastError();
}

}  // namespace

// The largest workgroup tile that still gives every CU a workgroup, else the tile
// with the most workgroups.
hipError_t launch_gemm(hipStream_t stream, const GemmJob& job, uint32_t cu_count, uint64_t seq,
                       const uint64_t* flag) {
    const uint64_t cus = cu_count ? cu_count : 256u;
    auto blocks = [&](uint32_t tm, uint32_t tn) {
        return (uint64_t)((job.rows + tm - 1u) / tm) * ((job.n + tn - 1u) / tn);
    };
    if (blocks(128, 128) >= cus)
        return launch_bits<128, 128>(stream, job, seq, flag);
    if (blocks(64, 128) >= cus)
        return launch_bits<64, 128>(stream, job, seq, flag);
    if (blocks(64, 64) >= cus)
        return launch_bits<64, 64>(stream, job, seq, flag);
    return launch_bits<32, 64>(stream, job, seq, flag);
}

}  // namespace bnnhip
