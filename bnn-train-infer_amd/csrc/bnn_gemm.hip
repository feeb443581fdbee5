// Multi-row jobs (GEMM, GEMM_F32, DOT_GROUPS with rows >= kMfmaMinRows) on the
// gfx950 matrix cores (v_mfma_i32_16x16x64_i8), fed from the matrix's resident
// 1.125-bit layout: the sign bits of each 128-weight group are unpacked to +1/-1
// bytes in LDS, per workgroup tile and group, two groups before the MFMAs use them.
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
// k_gemm_bits<TM, TN, WGM, WGN>: workgroup tile TM x TN, WGM x WGN waves of
// (TM/WGM) x (TN/WGN).  Everything a group needs reaches LDS by DMA
// (global_load_lds, 16 bytes per lane, no registers): the TM rows' 128 quantised
// bytes, the TN features' 16-byte sign-bit chunks (1 KiB per 64-feature tile of the
// matrix layout) and their column scales.  One barrier per group; iteration g:
//   * issue the DMAs of group g+3's rows, group g+5's bits and group g+2's scales
//     (each has two iterations to land);
//   * look up group g+2's bits (read into registers one iteration ago) in a
//     256-entry table (2 KiB, built at start): one 8-byte lookup turns a byte of
//     bits into 8 bytes of +1/-1;
//   * read group g+3's bits, and group g+1's MFMA operands into the second
//     register set (the loop is unrolled by two, so the two sets alternate without
//     copies);
//   * group g's first-half MFMAs (operands read one iteration ago), each subtile
//     interleaved with group g-1's epilogue on it;
//   * store group g+2's +1/-1 tile; group g's second-half MFMAs.
// At the end every wave writes its accumulators into LDS and the workgroup stores
// the tile row by row, 16 bytes per lane.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>
#include <hip/hip_fp16.h>

#include "bnn_internal.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kMagicBits = 0x4B400000;  // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicValue = 12582912.0f;

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

// Output tiles in bands of `band` M tiles, M tile fastest within a band (the last
// band may be narrower), and workgroups remapped so that consecutive tiles run on one
// XCD: each XCD's share of the grid is then a rectangle of about band M tiles by
// (tiles / 8 / band) N tiles, whose rows and weights stay in that XCD's L2.  The host
// picks `band` so that the rows (re-read once per XCD that covers an M tile) and the
// weights (once per band) cost the least traffic.
struct TileRC {
    uint32_t mt, nt;
};
__device__ __forceinline__ TileRC gemm_tile_of_block(uint32_t b, uint32_t grid, uint32_t mtiles, uint32_t ntiles,
                                                     uint32_t band) {
    const uint32_t x = b % 8u, i = b / 8u, q = grid / 8u, r = grid % 8u;
    const uint32_t t = (x < r ? x * (q + 1u) : r * (q + 1u) + (x - r) * q) + i;
    const uint32_t bi = t / (band * ntiles), rest = t % (band * ntiles);
    const uint32_t width = min(band, mtiles - bi * band);
    return TileRC{bi * band + rest % width, rest / width};
}

// 16 bytes per active lane from global memory into LDS at lds_addr + 16 * lane (the
// wave's LDS base goes in M0).  Inline assembly, so that the compiler's own wait
// insertion does not add a wait for every LDS DMA before each later LDS read: the
// kernel bounds the outstanding loads itself.  The s_nop covers the one wait state
// between writing M0 and the LDS DMA reading it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_addr) : "memory");
}

// The same for the lanes of a constant mask only: the mask goes into exec inside the
// assembly (and exec is restored there), so that the caller needs no branch around
// the load -- a branch would split the loop body into blocks across which the
// compiler moves the arithmetic of one group into the next.
template <uint64_t LANES>
__device__ __forceinline__ void dma16_lanes(const void* gptr, uint32_t lds_addr) {
    if constexpr (LANES == ~0ull) {
        dma16(gptr, lds_addr);
    } else {
        uint64_t saved;
        asm volatile(
            "s_mov_b64 %0, exec\n\ts_mov_b64 exec, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
            "s_mov_b64 exec, %0"
            : "=&s"(saved)
            : "v"(gptr), "{m0}"(lds_addr), "s"(LANES)
            : "memory");
    }
}

// The same with the address as a wave-uniform base (SGPRs) plus a 32-bit per-lane
// offset: no 64-bit per-lane address arithmetic per DMA.
__device__ __forceinline__ void dma16_s(uint32_t voff, const void* sbase, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

template <uint32_t N>
constexpr uint64_t lane_mask() {
    return N >= 64 ? ~0ull : (1ull << (N % 64u)) - 1ull;
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

// A job's row scale through the global address space (a flat load would also count on the
// LDS counter that the kernels' LDS waits use).
__device__ __forceinline__ float row_scale(const GemmJob& j, uint32_t m) {
    return *(const __attribute__((address_space(1))) float*)(j.rscale + m);
}

__device__ __forceinline__ void barrier() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access moves across it
}

template <int TM, int TN, int WGM, int WGN, int ASLOTS = 4>
struct Tiling {
    static constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
    static constexpr int WTM = TM / WGM, WTN = TN / WGN, MS = WTM / 16, NS = WTN / 16;
    // DMA work per wave and group: every wave issues exactly A_INS + 2 DMAs, each
    // with at least one active lane, so that the vmcnt bookkeeping is uniform
    static constexpr uint32_t A_CHUNKS = TM * 8 / WAVES;  // 16-byte row chunks
    static constexpr uint32_t A_INS = A_CHUNKS >= 64 ? A_CHUNKS / 64 : 1;
    static constexpr uint32_t A_LANES = A_CHUNKS >= 64 ? 64 : A_CHUNKS;
    static constexpr uint32_t BIT_LANES = TN / WAVES;     // one 16-byte chunk per feature
    static constexpr uint32_t SC_CHUNKS = TN / 8;         // 8 fp16 scales per chunk
    static constexpr uint32_t SC_CPW = SC_CHUNKS >= (uint32_t)WAVES ? SC_CHUNKS / WAVES : 1;
    // LDS carve-up (bytes)
    static constexpr uint32_t A_SLOT = TM * 128, B_SLOT = TN * 128, BITS_SLOT = TN * 16, SC_SLOT = TN * 2;
    static constexpr uint32_t OFF_B = ASLOTS * A_SLOT, OFF_BITS = OFF_B + 2 * B_SLOT, OFF_SC = OFF_BITS + 4 * BITS_SLOT,
                              OFF_LUT = (OFF_SC + 4 * SC_SLOT + 15u) & ~15u, LOOP_BYTES = OFF_LUT + 2048;
    static constexpr uint32_t OUT_STRIDE = TN + 16;  // floats per staged output row
    static constexpr uint32_t OUT_BYTES = TM * OUT_STRIDE * 4;
    static constexpr uint32_t SMEM = LOOP_BYTES > OUT_BYTES ? LOOP_BYTES : OUT_BYTES;
    static_assert(TM % (16 * WGM) == 0 && TN % (16 * WGN) == 0, "wave tiles of 16 x 16 subtiles");
    static_assert(A_CHUNKS % 64 == 0 || A_CHUNKS < 64, "row DMA split");
    static_assert(TN % WAVES == 0 && BIT_LANES <= 64, "bits DMA split");
    static_assert(SC_CHUNKS < (uint32_t)WAVES || SC_CHUNKS % WAVES == 0, "scales DMA split");
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(TM * TN / 4 % THREADS == 0, "output chunks per thread");
};

template <int TM, int TN, int WGM, int WGN, bool DOT>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_bits(GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band,
                                                              uint64_t seq, const uint64_t* __restrict__ flag) {
    using T = Tiling<TM, TN, WGM, WGN>;
    constexpr int MS = T::MS, NS = T::NS, THREADS = T::THREADS;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t mt = tile.mt, nt = tile.nt;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    const uint32_t groups = j.groups;
    unsigned char* const lds_a = smem;
    unsigned char* const lds_b = smem + T::OFF_B;
    unsigned char* const lds_bits = smem + T::OFF_BITS;
    unsigned char* const lds_sc = smem + T::OFF_SC;
    uint2* const lut = reinterpret_cast<uint2*>(smem + T::OFF_LUT);

    // byte b of sign bits -> 8 bytes of +1/-1 (bit i -> byte i)
    if (tid < 256u)
        lut[tid] = make_uint2(pm1_nibble(tid & 15u), pm1_nibble(tid >> 4));

    // this lane's DMA sources (without the group offset)
    const uint8_t* a_src[T::A_INS];
#pragma unroll
    for (uint32_t i = 0; i < T::A_INS; ++i) {
        const uint32_t p = wave * T::A_CHUNKS + i * 64u + lane, r = p >> 3;
        const uint32_t c = (p & 7u) ^ ((r >> 1) & 7u);
        a_src[i] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)min(m0 + min(r, TM - 1u), j.rows - 1u) * j.k +
                   16u * c;
    }
    // bits: feature f of the tile; its 64-feature matrix tile is clamped into the
    // array (features past the last tile are never stored)
    const uint32_t f = T::BIT_LANES * wave + min(lane, T::BIT_LANES - 1u);
    const uint8_t* bit_src = reinterpret_cast<const uint8_t*>(j.wbits) +
                             ((size_t)min((n0 + f) >> 6, j.tiles - 1u) * groups * kTile + ((n0 + f) & 63u)) * 16u;
    // scales: chunks of 8 columns, SC_CPW consecutive ones per wave (with fewer
    // chunks than waves, the waves past the last chunk repeat one, writing the same
    // bytes)
    const uint32_t sc_first = (wave * T::SC_CPW) % T::SC_CHUNKS;
    const uint32_t sc_col = n0 + 8u * (sc_first + min(lane, T::SC_CPW - 1u));
    const uint8_t* sc_src = reinterpret_cast<const uint8_t*>(j.wscale) +
                            ((size_t)min(sc_col >> 6, j.tiles - 1u) * groups * kTile + (sc_col & 63u)) * 2u;
    const uint32_t la0 = lds_offset(lds_a), lbits0 = lds_offset(lds_bits), lsc0 = lds_offset(lds_sc);
    const size_t bit_step = (size_t)kTile * 16u, sc_step = (size_t)kTile * 2u;  // bytes per group
    auto issue_rows = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
#pragma unroll
        for (uint32_t i = 0; i < T::A_INS; ++i)
            dma16_lanes<lane_mask<T::A_LANES>()>(a_src[i] + (size_t)gg * kGroup,
                                                 la0 + (g & 3u) * T::A_SLOT + (wave * T::A_CHUNKS + i * 64u) * 16u);
    };
    auto issue_bits = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        dma16_lanes<lane_mask<T::BIT_LANES>()>(bit_src + gg * bit_step,
                                               lbits0 + (g & 3u) * T::BITS_SLOT + wave * (T::BIT_LANES * 16u));
    };
    auto issue_scales = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        dma16_lanes<lane_mask<T::SC_CPW>()>(sc_src + gg * sc_step, lsc0 + (g & 3u) * T::SC_SLOT + 16u * sc_first);
    };
    // unpacks group g's bits (slot g % 4) into the +1/-1 tile lds_b[g % 2], in two
    // parts so that the read of the bits can be issued long before its use: unit u =
    // feature u / 4, bytes 4 * (u % 4) .. +3 of its 16 bytes of bits -> chunks
    // 2 * (u % 4) and 2 * (u % 4) + 1 of its 128-byte row
    constexpr uint32_t UNITS = TN * 4u, UPT = (UNITS + THREADS - 1u) / THREADS;  // units per thread
    // a thread's i-th unit; past the last unit a thread repeats one (same bytes to the
    // same place), so that no branch splits the loop body
    auto unit = [&](uint32_t i) {
        const uint32_t u = i * THREADS + tid;
        return UNITS % THREADS == 0 || u < UNITS ? u : u - THREADS;
    };
    auto unpack_read = [&](uint32_t (&w)[UPT], uint32_t g) {
        const unsigned char* bits = lds_bits + (g & 3u) * T::BITS_SLOT;
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i) {
            const uint32_t u = unit(i);
            w[i] = *reinterpret_cast<const uint32_t*>(bits + (u >> 2) * 16u + (u & 3u) * 4u);
        }
    };
    auto unpack_lut = [&](uint2 (&e)[UPT][4], const uint32_t (&w)[UPT]) {
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i) {
#pragma unroll
            for (uint32_t b = 0; b < 4; ++b)
                e[i][b] = lut[(w[i] >> (8u * b)) & 0xffu];
        }
    };
    auto unpack_store = [&](const uint2 (&e)[UPT][4], uint32_t g) {
        unsigned char* dst = lds_b + (g & 1u) * T::B_SLOT;
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i) {
            const uint32_t u = unit(i), row = u >> 2, part = u & 3u;
            *reinterpret_cast<uint4*>(dst + swz128(row, 2u * part)) =
                make_uint4(e[i][0].x, e[i][0].y, e[i][1].x, e[i][1].y);
            *reinterpret_cast<uint4*>(dst + swz128(row, 2u * part + 1u)) =
                make_uint4(e[i][2].x, e[i][2].y, e[i][3].x, e[i][3].y);
        }
    };
    auto unpack = [&](uint32_t g) {
        uint32_t w[UPT];
        uint2 e[UPT][4];
        unpack_read(w, g);
        unpack_lut(e, w);
        unpack_store(e, g);
    };

    const uint32_t arow0 = wm * T::WTM + (lane & 15u), brow0 = wn * T::WTN + (lane & 15u);
    const uint32_t chunk = lane >> 4;
    // MFMA operands of group g: [half][subtile]
    auto load_frags = [&](v4i (&a)[2][MS], v4i (&b)[2][NS], uint32_t g) {
        const unsigned char* la = lds_a + (g & 3u) * T::A_SLOT;
        const unsigned char* lb = lds_b + (g & 1u) * T::B_SLOT;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mi = 0; mi < MS; ++mi)
                a[h][mi] = *reinterpret_cast<const v4i*>(la + swz128(arow0 + 16u * mi, 4u * h + chunk));
#pragma unroll
            for (int ni = 0; ni < NS; ++ni)
                b[h][ni] = *reinterpret_cast<const v4i*>(lb + swz128(brow0 + 16u * ni, 4u * h + chunk));
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
    const uint32_t row_base = m0 + wm * T::WTM + 4u * (lane >> 4);
    const uint32_t col_base = n0 + wn * T::WTN + (lane & 15u);
    float sc_prev[NS];
#pragma unroll
    for (int ni = 0; ni < NS; ++ni)
        sc_prev[ni] = 0.0f;

    // One group: see the header.  At entry (after the barrier) LDS holds group g+1's
    // rows and +1/-1 tile, group g+3's bits and group g's scales (the DMAs of the
    // previous step may still be landing); ubits holds group g+2's bits, read in the
    // previous step.
    uint32_t ubits[UPT];
    auto step = [&](uint32_t g, v4i (&ca)[2][MS], v4i (&cb)[2][NS], v4i (&na)[2][MS], v4i (&nb)[2][NS]) {
        // this wave's DMAs but the previous step's have landed, its LDS accesses are
        // done; after the barrier the same holds for every wave
        wait_dma<T::A_INS + 2>();
        barrier();
        issue_rows(g + 3u);
        issue_bits(g + 5u);
        issue_scales(g + 2u);
        // LDS reads in this order: the table lookups of group g+2 (first, so that the
        // unpack does not queue behind the operand reads), group g+3's bits, group
        // g+1's operands, group g's scales
        uint2 ex[UPT][4];
        unpack_lut(ex, ubits);
        __builtin_amdgcn_sched_barrier(0);
        unpack_read(ubits, g + 3u);
        load_frags(na, nb, g + 1u);
        float sc_cur[NS];
        const uint16_t* scl = reinterpret_cast<const uint16_t*>(lds_sc + (g & 3u) * T::SC_SLOT);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_cur[ni] = DOT ? 0.0f : __half2float(__ushort_as_half(scl[wn * T::WTN + 16u * ni + (lane & 15u)]));
        __builtin_amdgcn_sched_barrier(0);
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
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ca[0][mi], cb[0][ni], c_init, 0, 0, 0);
            }
        }
        if constexpr (!DOT) {
            // per subtile its 8 epilogue VALU ops, then its restarting MFMA: the matrix
            // pipe runs while the next subtile's VALU ops issue
#pragma unroll
            for (int i = 0; i < MS * NS; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        unpack_store(ex, g + 2u);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int mi = 0; mi < MS; ++mi)
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ca[1][mi], cb[1][ni], d[mi][ni], 0, 0, 0);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_prev[ni] = sc_cur[ni];
        __builtin_amdgcn_sched_barrier(0);  // nothing moves across steps
    };

    // prologue: groups 0..3's bits, 0..2's rows, 0..1's scales; groups 0 and 1 unpacked,
    // group 2's bits in registers; group 4's bits issued once group 0's have been
    // read (they share a slot); group 0's operands in registers
#pragma unroll
    for (uint32_t b = 0; b < 4; ++b)
        issue_bits(b);
    issue_scales(0);
    issue_scales(1);
    issue_rows(0);
    issue_rows(1);
    issue_rows(2);
    wait_dma<0>();
    barrier();  // the table and the first DMAs are in LDS
    unpack(0);
    unpack(1);
    unpack_read(ubits, 2);
    wait_dma<0>();
    barrier();
    issue_bits(4);
    v4i xa[2][MS], xb[2][NS], ya[2][MS], yb[2][NS];
    load_frags(xa, xb, 0);
    uint32_t g = 0;
    for (; g + 1u < groups; g += 2u) {
        step(g, xa, xb, ya, yb);
        step(g + 1u, ya, yb, xa, xb);
    }
    if (g < groups)
        step(g, xa, xb, ya, yb);

    // no DMA may still be writing LDS when it is reused or the workgroup ends
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
    // epilogue of the last group
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
    // stage the tile in LDS, then store it row by row (16 bytes per lane where the
    // output rows allow it); Z * s for GEMM_F32
    barrier();
    float* const so = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                so[(wm * T::WTM + 16u * mi + 4u * (lane >> 4) + r) * T::OUT_STRIDE + wn * T::WTN + 16u * ni +
                   (lane & 15u)] = acc[mi][ni][r];
    wait_dma<0>();
    barrier();
    const bool vec = ((j.out_stride | (uint64_t)(uintptr_t)j.out) & 15u) == 0;
    const bool scaled = j.mode == MODE_SUM_SCALED;
#pragma unroll
    for (uint32_t c0 = 0; c0 < TM * TN / 4u; c0 += THREADS) {
        const uint32_t c = c0 + tid, row = c / (TN / 4u), col = 4u * (c % (TN / 4u));
        const uint32_t m = m0 + row, n = n0 + col;
        if (m >= j.rows || n >= j.n)
            continue;
        float4 v = *reinterpret_cast<const float4*>(so + row * T::OUT_STRIDE + col);
        if (scaled) {
            const float s = row_scale(j, m);
            v.x = v.x * s;
            v.y = v.y * s;
            v.z = v.z * s;
            v.w = v.w * s;
        }
        float* dst = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride) + n;
        if (vec && n + 4u <= j.n) {
            const v4f w = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(w, reinterpret_cast<v4f*>(dst));
        } else {
            dst[0] = v.x;
            if (n + 1u < j.n)
                dst[1] = v.y;
            if (n + 2u < j.n)
                dst[2] = v.z;
            if (n + 3u < j.n)
                dst[3] = v.w;
        }
    }
}

// k_gemm_co<TM, TN, WGM, WGN>: GEMM / GEMM_F32 with two workgroups per CU.  The
// same per-group work as k_gemm_bits with a shorter pipeline, so that a 128 x 128
// tile fits in 75 KB of LDS and 4 waves of at most 256 VGPRs: the rows' DMA runs one
// group ahead (two slots), the unpack one, and each group's MFMA operands are read
// right after its barrier; the other workgroup on the CU covers the latency.
// Iteration g, after one wait and one barrier:
//   * issue the DMAs of group g+1's rows, group g+4's bits and group g+2's scales;
//   * look up group g+1's bits (read one iteration ago), read group g+2's bits, group
//     g's operands and scales;
//   * group g's first-half MFMAs interleaved with group g-1's epilogue;
//   * store group g+1's +1/-1 tile; group g's second-half MFMAs.
template <int TM, int TN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_co(
    GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band, uint64_t seq, const uint64_t* __restrict__ flag) {
    using T = Tiling<TM, TN, WGM, WGN, 2>;
    constexpr int MS = T::MS, NS = T::NS, THREADS = T::THREADS;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t m0 = tile.mt * TM, n0 = tile.nt * TN;
    const uint32_t groups = j.groups;
    unsigned char* const lds_a = smem;
    unsigned char* const lds_b = smem + T::OFF_B;
    unsigned char* const lds_bits = smem + T::OFF_BITS;
    unsigned char* const lds_sc = smem + T::OFF_SC;
    uint2* const lut = reinterpret_cast<uint2*>(smem + T::OFF_LUT);
    if (tid < 256u)
        lut[tid] = make_uint2(pm1_nibble(tid & 15u), pm1_nibble(tid >> 4));

    const uint8_t* a_src[T::A_INS];
#pragma unroll
    for (uint32_t i = 0; i < T::A_INS; ++i) {
        const uint32_t p = wave * T::A_CHUNKS + i * 64u + lane, r = min(p >> 3, TM - 1u);
        const uint32_t c = (p & 7u) ^ ((r >> 1) & 7u);
        a_src[i] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)min(m0 + r, j.rows - 1u) * j.k + 16u * c;
    }
    const uint32_t f = T::BIT_LANES * wave + min(lane, T::BIT_LANES - 1u);
    const uint8_t* bit_src = reinterpret_cast<const uint8_t*>(j.wbits) +
                             ((size_t)min((n0 + f) >> 6, j.tiles - 1u) * groups * kTile + ((n0 + f) & 63u)) * 16u;
    const uint32_t sc_first = (wave * T::SC_CPW) % T::SC_CHUNKS;
    const uint32_t sc_col = n0 + 8u * (sc_first + min(lane, T::SC_CPW - 1u));
    const uint8_t* sc_src = reinterpret_cast<const uint8_t*>(j.wscale) +
                            ((size_t)min(sc_col >> 6, j.tiles - 1u) * groups * kTile + (sc_col & 63u)) * 2u;
    const uint32_t la0 = lds_offset(lds_a), lbits0 = lds_offset(lds_bits), lsc0 = lds_offset(lds_sc);
    const size_t bit_step = (size_t)kTile * 16u, sc_step = (size_t)kTile * 2u;
    auto issue_rows = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
#pragma unroll
        for (uint32_t i = 0; i < T::A_INS; ++i)
            dma16_lanes<lane_mask<T::A_LANES>()>(a_src[i] + (size_t)gg * kGroup,
                                                 la0 + (g & 1u) * T::A_SLOT + (wave * T::A_CHUNKS + i * 64u) * 16u);
    };
    auto issue_bits = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        dma16_lanes<lane_mask<T::BIT_LANES>()>(bit_src + gg * bit_step,
                                               lbits0 + (g & 3u) * T::BITS_SLOT + wave * (T::BIT_LANES * 16u));
    };
    auto issue_scales = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        dma16_lanes<lane_mask<T::SC_CPW>()>(sc_src + gg * sc_step, lsc0 + (g & 3u) * T::SC_SLOT + 16u * sc_first);
    };
    constexpr uint32_t UNITS = TN * 4u, UPT = (UNITS + THREADS - 1u) / THREADS;
    static_assert(UNITS % THREADS == 0, "whole units per thread");
    auto unpack_read = [&](uint32_t (&w)[UPT], uint32_t g) {
        const unsigned char* bits = lds_bits + (g & 3u) * T::BITS_SLOT;
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i) {
            const uint32_t u = i * THREADS + tid;
            w[i] = *reinterpret_cast<const uint32_t*>(bits + (u >> 2) * 16u + (u & 3u) * 4u);
        }
    };
    auto unpack_lut = [&](uint2 (&e)[UPT][4], const uint32_t (&w)[UPT]) {
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i)
#pragma unroll
            for (uint32_t b = 0; b < 4; ++b)
                e[i][b] = lut[(w[i] >> (8u * b)) & 0xffu];
    };
    auto unpack_store = [&](const uint2 (&e)[UPT][4], uint32_t g) {
        unsigned char* dst = lds_b + (g & 1u) * T::B_SLOT;
#pragma unroll
        for (uint32_t i = 0; i < UPT; ++i) {
            const uint32_t u = i * THREADS + tid, row = u >> 2, part = u & 3u;
            *reinterpret_cast<uint4*>(dst + swz128(row, 2u * part)) =
                make_uint4(e[i][0].x, e[i][0].y, e[i][1].x, e[i][1].y);
            *reinterpret_cast<uint4*>(dst + swz128(row, 2u * part + 1u)) =
                make_uint4(e[i][2].x, e[i][2].y, e[i][3].x, e[i][3].y);
        }
    };
    const uint32_t arow0 = wm * T::WTM + (lane & 15u), brow0 = wn * T::WTN + (lane & 15u);
    const uint32_t chunk = lane >> 4;
    // half h of group g's MFMA operands (one register set, reused by the two halves)
    auto load_half = [&](v4i (&a)[MS], v4i (&b)[NS], uint32_t g, uint32_t h) {
        const unsigned char* la = lds_a + (g & 1u) * T::A_SLOT;
        const unsigned char* lb = lds_b + (g & 1u) * T::B_SLOT;
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
            a[mi] = *reinterpret_cast<const v4i*>(la + swz128(arow0 + 16u * mi, 4u * h + chunk));
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            b[ni] = *reinterpret_cast<const v4i*>(lb + swz128(brow0 + 16u * ni, 4u * h + chunk));
    };

    float acc[MS][NS][4];
    v4i d[MS][NS];
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            d[mi][ni] = c_init;  // with scale 0 the first epilogue adds +0
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
        }
    float sc_prev[NS];
#pragma unroll
    for (int ni = 0; ni < NS; ++ni)
        sc_prev[ni] = 0.0f;

    // prologue: groups 0..3's bits, 0..1's scales, group 0's rows; group 0 unpacked,
    // group 1's bits in registers
#pragma unroll
    for (uint32_t b = 0; b < 4; ++b)
        issue_bits(b);
    issue_scales(0);
    issue_scales(1);
    issue_rows(0);
    wait_dma<0>();
    barrier();
    uint32_t ubits[UPT];
    {
        uint2 e0[UPT][4];
        unpack_read(ubits, 0);
        unpack_lut(e0, ubits);
        unpack_store(e0, 0);
    }
    unpack_read(ubits, 1);
    wait_dma<0>();

    for (uint32_t g = 0; g < groups; ++g) {
        // this wave's DMAs but the last two have landed (group g's rows among them),
        // its LDS accesses are done; after the barrier the same holds for every wave
        wait_dma<2>();
        barrier();
        issue_rows(g + 1u);
        issue_bits(g + 4u);
        issue_scales(g + 2u);
        uint2 ex[UPT][4];
        unpack_lut(ex, ubits);
        __builtin_amdgcn_sched_barrier(0);
        unpack_read(ubits, g + 2u);
        v4i ca[MS], cb[NS];
        load_half(ca, cb, g, 0);
        float sc_cur[NS];
        const uint16_t* scl = reinterpret_cast<const uint16_t*>(lds_sc + (g & 3u) * T::SC_SLOT);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_cur[ni] = __half2float(__ushort_as_half(scl[wn * T::WTN + 16u * ni + (lane & 15u)]));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            const float sc = sc_prev[ni];
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (int mi = 0; mi < MS; ++mi) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ca[mi], cb[ni], c_init, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < MS * NS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        unpack_store(ex, g + 1u);
        load_half(ca, cb, g, 1);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int mi = 0; mi < MS; ++mi)
                d[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ca[mi], cb[ni], d[mi][ni], 0, 0, 0);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_prev[ni] = sc_cur[ni];
        __builtin_amdgcn_sched_barrier(0);
    }
    wait_dma<0>();
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
    barrier();
    float* const so = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                so[(wm * T::WTM + 16u * mi + 4u * (lane >> 4) + r) * T::OUT_STRIDE + wn * T::WTN + 16u * ni +
                   (lane & 15u)] = acc[mi][ni][r];
    wait_dma<0>();
    barrier();
    const bool vec = ((j.out_stride | (uint64_t)(uintptr_t)j.out) & 15u) == 0;
    const bool scaled = j.mode == MODE_SUM_SCALED;
#pragma unroll
    for (uint32_t c0 = 0; c0 < TM * TN / 4u; c0 += THREADS) {
        const uint32_t c = c0 + tid, row = c / (TN / 4u), col = 4u * (c % (TN / 4u));
        const uint32_t m = m0 + row, n = n0 + col;
        if (m >= j.rows || n >= j.n)
            continue;
        float4 v = *reinterpret_cast<const float4*>(so + row * T::OUT_STRIDE + col);
        if (scaled) {
            const float s = row_scale(j, m);
            v.x = v.x * s;
            v.y = v.y * s;
            v.z = v.z * s;
            v.w = v.w * s;
        }
        float* dst = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride) + n;
        if (vec && n + 4u <= j.n) {
            const v4f w = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(w, reinterpret_cast<v4f*>(dst));
        } else {
            dst[0] = v.x;
            if (n + 1u < j.n)
                dst[1] = v.y;
            if (n + 2u < j.n)
                dst[2] = v.z;
            if (n + 3u < j.n)
                dst[3] = v.w;
        }
    }
}

uint32_t gemm_band(const GemmJob& job, uint32_t mtiles);

template <int TM, int TN, int WGM, int WGN>
hipError_t launch_co(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + TM - 1u) / TM, ntiles = (job.n + TN - 1u) / TN;
    launch_kernel((k_gemm_co<TM, TN, WGM, WGN>), dim3(mtiles * ntiles), dim3(64 * WGM * WGN), 0, stream, job, mtiles,
                  ntiles, gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

// k_gemm_ks: F32-accumulating jobs with too few tiles to give every CU a workgroup.
// Workgroup tile (16*TMS) x (16*TNS); the W waves split K instead of the tile: wave w
// computes groups w, w+W, w+2W, ... for the whole tile, its operands loaded from
// global memory straight into registers DEPTH-1 rounds ahead.  The K order inside a
// group is permuted so that a lane's share of a column's sign bits is 4 contiguous
// bytes: lane chunk c (lane / 16) covers weights 32c .. 32c+31, MFMA half h the 16
// starting at 32c + 16h, in the rows and the weights alike.  The bits of the next
// round become +1/-1 operands through the byte table while this round's MFMAs run.
// Per round each wave writes the exact products RN(scale * D) of its group to LDS;
// then every thread adds the W products of its outputs to its FP32 accumulators in
// group order -- the order of the sums is the reference's, only the integer work ran
// in parallel.
template <int TMS, int TNS>
struct KsOps {
    v4i a[TMS][2];
    uint32_t bits[TNS];
    uint16_t s[TNS];
    v4i b[TNS][2];  // the +1/-1 operands, from bits
};

__device__ __forceinline__ v4i gload_v4i(const void* p) {
    return *(const __attribute__((address_space(1))) v4i*)p;
}

template <int TMS, int TNS, int W, int DEPTH>
__global__ __launch_bounds__(64 * W) void k_gemm_ks(GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band,
    uint64_t seq,
                                                   const uint64_t* __restrict__ flag) {
    constexpr uint32_t TM = 16u * TMS, TN = 16u * TNS, SUBS = TMS * TNS, NT = 64u * W;
    constexpr uint32_t BLOCKS = SUBS * 64u;  // 16-byte blocks of products per wave
    constexpr uint32_t PER_THREAD = (BLOCKS + NT - 1u) / NT;
    static_assert(DEPTH >= 3, "the next round's bits loaded a round before their expansion");
    static_assert(TN <= 64, "a tile's columns lie in one 64-feature tile of the matrix layout");
    __shared__ __attribute__((aligned(16))) float prod[W][BLOCKS * 4u];  // [wave][subtile][lane][4]
    __shared__ uint2 lut[256];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t mt = tile.mt, nt = tile.nt;
    const uint32_t m0 = mt * TM, n0 = nt * TN;
    // the row scales of this thread's outputs (F32 jobs), requested now (see k_gemm_kr)
    float rs[PER_THREAD][4];
#pragma unroll
    for (int i = 0; i < (int)PER_THREAD; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + 16u * ((W * i + wave) / TNS) + 4u * (lane >> 4) + r;
            rs[i][r] = j.mode == MODE_SUM_SCALED && W * i + wave < SUBS && m < j.rows ? row_scale(j, m) : 1.0f;
        }
    const uint32_t groups = j.groups;
    for (uint32_t i = tid; i < 256u; i += NT)
        lut[i] = make_uint2(pm1_nibble(i & 15u), pm1_nibble(i >> 4));

    // rows past the end are clamped (never stored); so is the matrix tile of columns
    // past the last tile
    const uint32_t chunk = lane >> 4;
    const uint8_t* a_ptr[TMS];
    const uint8_t* b_ptr[TNS];
    const uint16_t* s_ptr[TNS];
#pragma unroll
    for (int mi = 0; mi < TMS; ++mi) {
        const uint32_t m = min(m0 + 16u * mi + (lane & 15u), j.rows - 1u);
        a_ptr[mi] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)m * j.k + 32u * chunk;
    }
#pragma unroll
    for (int ni = 0; ni < TNS; ++ni) {
        const uint32_t n = n0 + 16u * ni + (lane & 15u), st = min(n >> 6, j.tiles - 1u);
        b_ptr[ni] = reinterpret_cast<const uint8_t*>(j.wbits) + ((size_t)st * groups * kTile + (n & 63u)) * 16u +
                    4u * chunk;
        s_ptr[ni] = j.wscale + (size_t)st * groups * kTile + (n & 63u);
    }
    // loads are unconditional (group clamped into range) so that every path has the
    // same loads in flight
    auto load = [&](KsOps<TMS, TNS>& o, uint32_t round) {
        const uint32_t g = min(W * round + wave, groups - 1u);
#pragma unroll
        for (int mi = 0; mi < TMS; ++mi)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                o.a[mi][h] = gload_v4i(a_ptr[mi] + (size_t)g * kGroup + 16u * h);
#pragma unroll
        for (int ni = 0; ni < TNS; ++ni) {
            o.bits[ni] = *reinterpret_cast<const uint32_t*>(b_ptr[ni] + (size_t)g * kTile * 16u);
            o.s[ni] = s_ptr[ni][(size_t)g * kTile];
        }
    };
    auto expand = [&](KsOps<TMS, TNS>& o) {
#pragma unroll
        for (int ni = 0; ni < TNS; ++ni)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint2 lo = lut[(o.bits[ni] >> (16u * h)) & 0xffu];
                const uint2 hi = lut[(o.bits[ni] >> (16u * h + 8u)) & 0xffu];
                o.b[ni][h] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
    };

    float acc[PER_THREAD][4];
#pragma unroll
    for (int i = 0; i < (int)PER_THREAD; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[i][r] = 0.0f;
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
    KsOps<TMS, TNS> o[DEPTH];

    // round r with its operands in o[d] (d = r % DEPTH)
    auto round = [&](int d, uint32_t r) {
        KsOps<TMS, TNS>& cur = o[d];
        load(o[(d + DEPTH - 1) % DEPTH], r + DEPTH - 1u);
        const uint32_t g = W * r + wave;
        float4 p[TMS][TNS];
        if (g < groups) {
#pragma unroll
            for (int ni = 0; ni < TNS; ++ni) {
                const float sc = __half2float(__ushort_as_half(cur.s[ni]));
                const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
                for (int mi = 0; mi < TMS; ++mi) {
                    v4i dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][0], cur.b[ni][0], c_init, 0, 0, 0);
                    dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][1], cur.b[ni][1], dd, 0, 0, 0);
                    p[mi][ni].x = __builtin_fmaf(sc, __int_as_float(dd[0]), cneg);
                    p[mi][ni].y = __builtin_fmaf(sc, __int_as_float(dd[1]), cneg);
                    p[mi][ni].z = __builtin_fmaf(sc, __int_as_float(dd[2]), cneg);
                    p[mi][ni].w = __builtin_fmaf(sc, __int_as_float(dd[3]), cneg);
                }
            }
        }
        expand(o[(d + 1) % DEPTH]);  // round r+1's operands, loaded one round ago
        // the previous round's reads of prod are done (their sums consumed them)
        barrier();
        if (g < groups) {
#pragma unroll
            for (int mi = 0; mi < TMS; ++mi)
#pragma unroll
                for (int ni = 0; ni < TNS; ++ni)
                    *reinterpret_cast<float4*>(&prod[wave][((mi * TNS + ni) * 64u + lane) * 4u]) = p[mi][ni];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
        barrier();
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

#pragma unroll
    for (int d = 0; d + 1 < DEPTH; ++d)
        load(o[d], d);
    barrier();  // the table is in LDS
    expand(o[0]);
    const uint32_t rounds = (groups + W - 1u) / W;
    // the round count is padded to a multiple of DEPTH with rounds of no groups
    for (uint32_t r = 0; r < rounds; r += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            round(d, r + d);
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
            __builtin_nontemporal_store(j.mode == MODE_SUM_SCALED ? acc[i][r] * rs[i][r] : acc[i][r], orow + n);
        }
    }
}

// k_gemm_wv: F32-accumulating jobs with few rows.  Every wave computes a (16*MS) x
// (16*NS) block of the output over the whole K on its own: its rows' quantised bytes,
// its columns' sign bits and scales come from global memory straight into a ring of
// DEPTH groups of registers; the bits become +1/-1 operands through the byte table
// (LDS, written once before the loop); no barrier or LDS exchange sits in the loop, so
// the waves of a CU run their chains independently and the latency of one group's
// loads is covered by the DEPTH-1 groups ahead of it.  The K order inside a group is
// that of k_gemm_ks (lane chunk c: weights 32c .. 32c+31, MFMA half h the 16 from
// 32c + 16h), so a lane's operands are 32 contiguous row bytes and 4 contiguous bytes
// of bits.  Group g's MFMAs write one of two D sets while group g-1's epilogue reads
// the other; each output element's products are added in group order by one thread.
// The group count is padded to a multiple of DEPTH with groups of scale 0 (the
// clamped last group's operands), whose products are +0 and leave the sums unchanged.
template <int MS, int NS>
struct WvOps {
    v4i a[MS][2];
    uint32_t bits[NS];
    uint32_t s[NS];
};

template <int MS, int NS, int WM, int WN, int DEPTH>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_wv(GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band,
                                                         uint64_t seq, const uint64_t* __restrict__ flag) {
    constexpr uint32_t TM = 16u * MS * WM, TN = 16u * NS * WN, NT = 64u * WM * WN;
    static_assert(DEPTH >= 2 && DEPTH % 2 == 0, "two D sets alternate with the ring slots");
    static_assert(16 * NS <= 64 && 64 % (16 * NS) == 0, "a wave's columns lie in one 64-feature tile");
    __shared__ uint2 lut[256];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t m0 = tile.mt * TM + 16u * MS * wm, n0 = tile.nt * TN + 16u * NS * wn;
    const uint32_t groups = j.groups;
    for (uint32_t i = tid; i < 256u; i += NT)
        lut[i] = make_uint2(pm1_nibble(i & 15u), pm1_nibble(i >> 4));

    // rows past the end are clamped (never stored); so is the matrix tile of columns
    // past the last tile
    const uint32_t chunk = lane >> 4;
    const uint8_t* a_ptr[MS];
    const uint8_t* b_ptr[NS];
    const uint16_t* s_ptr[NS];
#pragma unroll
    for (int mi = 0; mi < MS; ++mi) {
        const uint32_t m = min(m0 + 16u * mi + (lane & 15u), j.rows - 1u);
        a_ptr[mi] = reinterpret_cast<const uint8_t*>(j.q) + (size_t)m * j.k + 32u * chunk;
    }
#pragma unroll
    for (int ni = 0; ni < NS; ++ni) {
        const uint32_t n = n0 + 16u * ni + (lane & 15u), st = min(n >> 6, j.tiles - 1u);
        b_ptr[ni] = reinterpret_cast<const uint8_t*>(j.wbits) + ((size_t)st * groups * kTile + (n & 63u)) * 16u +
                    4u * chunk;
        s_ptr[ni] = j.wscale + (size_t)st * groups * kTile + (n & 63u);
    }
    // every load is unconditional (group clamped into range): the same loads are in
    // flight on every path
    auto load = [&](WvOps<MS, NS>& o, uint32_t g) {
        const uint32_t gc = min(g, groups - 1u);
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                o.a[mi][h] = gload_v4i(a_ptr[mi] + (size_t)gc * kGroup + 16u * h);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            o.bits[ni] = *reinterpret_cast<const uint32_t*>(b_ptr[ni] + (size_t)gc * kTile * 16u);
            o.s[ni] = s_ptr[ni][(size_t)gc * kTile];
        }
    };

    float acc[MS][NS][4];
    v4i dd[2][MS][NS];
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
    float sc_prev[NS];
#pragma unroll
    for (int ni = 0; ni < NS; ++ni)
        sc_prev[ni] = 0.0f;  // the epilogue before group 0 adds +0
#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            dd[1][mi][ni] = c_init;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
        }
    auto epilogue = [&](const v4i (&d)[MS][NS]) {
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            const float sc = sc_prev[ni];
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (int mi = 0; mi < MS; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc, __int_as_float(d[mi][ni][r]), cneg);
        }
    };

    WvOps<MS, NS> o[DEPTH];
#pragma unroll
    for (int d = 0; d + 1 < DEPTH; ++d)
        load(o[d], d);
    barrier();  // the table is in LDS

    // group g = g0 + d from ring slot d: refill the slot emptied one group ago, expand
    // the bits, group g's MFMAs into D set d % 2, group g-1's epilogue from the other
    auto step = [&](int d, uint32_t g) {
        load(o[(d + DEPTH - 1) % DEPTH], g + DEPTH - 1u);
        const WvOps<MS, NS>& cur = o[d];
        v4i b[NS][2];
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint2 lo = lut[(cur.bits[ni] >> (16u * h)) & 0xffu];
                const uint2 hi = lut[(cur.bits[ni] >> (16u * h + 8u)) & 0xffu];
                b[ni][h] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
        v4i (&dn)[MS][NS] = dd[d & 1];
#pragma unroll
        for (int mi = 0; mi < MS; ++mi)
#pragma unroll
            for (int ni = 0; ni < NS; ++ni) {
                v4i x = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][0], b[ni][0], c_init, 0, 0, 0);
                dn[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.a[mi][1], b[ni][1], x, 0, 0, 0);
            }
        epilogue(dd[(d & 1) ^ 1]);
#pragma unroll
        for (int ni = 0; ni < NS; ++ni)
            sc_prev[ni] = g < groups ? __half2float(__ushort_as_half((uint16_t)cur.s[ni])) : 0.0f;
    };
    for (uint32_t g0 = 0; g0 < groups; g0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            step(d, g0 + d);
    }
    epilogue(dd[(DEPTH - 1) & 1]);  // the last step's group

#pragma unroll
    for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NS; ++ni) {
            const uint32_t n = n0 + 16u * ni + (lane & 15u);
            if (n >= j.n)
                continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = m0 + 16u * mi + 4u * (lane >> 4) + r;
                if (m >= j.rows)
                    continue;
                float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
                __builtin_nontemporal_store(j.mode == MODE_SUM_SCALED ? acc[mi][ni][r] * j.rscale[m] : acc[mi][ni][r],
                                            orow + n);
            }
        }
}

// k_gemm_kr<TMS, TNS, W, R>: F32-accumulating jobs with few rows, whose tiles are too
// few to hide a chain of per-group steps.  Workgroup tile (16 TMS) x (16 TNS); the W
// waves split K (round r of wave w: group W r + w, at most R rounds), and each wave
// requests everything its own groups need -- the tile rows' quantised bytes, the
// columns' sign bits and scales -- into its own part of LDS by DMA before it computes
// anything: no registers are held while the loads are in flight, and no wave reads
// another wave's part, so a round waits for the wave's own loads (vmcnt) and for no
// barrier.  A round expands the bits through the byte table, runs the MFMAs and keeps
// the exact products RN(scale * D) in registers.  After the last round: one barrier,
// every wave's products into LDS by group, a second barrier, and each output's products
// added in group order by one thread -- the reference's order; only the integer work
// ran in parallel.  The K order inside a group is that of k_gemm_ks (lane chunk c:
// weights 32c .. 32c+31, MFMA half h the 16 from 32c + 16h).
template <int TMS, int TNS, int W, int R>
struct KrLayout {
    static constexpr uint32_t TM = 16u * TMS, TN = 16u * TNS, SUBS = TMS * TNS, NT = 64u * W;
    // a round's part: rows [TM][128] (chunks swizzled as swz128), the columns' 16-byte
    // sign-bit chunks [TN][16], their fp16 scales [TN]
    static constexpr uint32_t A_BYTES = TM * 128u, A_INS = A_BYTES / 1024u;
    static constexpr uint32_t BITS_BYTES = TN * 16u, SC_BYTES = TN * 2u, SC_LANES = SC_BYTES / 16u;
    static constexpr uint32_t ROUND_BYTES = A_BYTES + BITS_BYTES + SC_BYTES;
    static constexpr uint32_t DMA_PER_ROUND = A_INS + 2u;
    static constexpr uint32_t OPS_BYTES = W * R * ROUND_BYTES;
    static constexpr uint32_t PROD_BYTES = W * R * SUBS * 1024u;  // float4 [group][subtile][lane]
    // the byte table after the operands (copies of it, one per lane group, measured no
    // faster: the larger LDS footprint costs more than the bank conflicts); the products
    // reuse both once every wave is done with them
    static constexpr uint32_t OFF_LUT = OPS_BYTES;
    static constexpr uint32_t SMEM = OPS_BYTES + 2048u > PROD_BYTES ? OPS_BYTES + 2048u : PROD_BYTES;
    static_assert(A_BYTES % 1024u == 0, "whole 1 KiB row DMAs");
    static_assert(TN <= 64u && 64u % TN == 0, "a tile's columns lie in one 64-feature tile of the matrix layout");
    static_assert(SC_BYTES % 16u == 0, "whole 16-byte scale DMAs");
    static_assert(R * DMA_PER_ROUND < 64u, "vmcnt range");
    static_assert(SMEM <= 160u * 1024u, "LDS");
};

// One round's operands of a lane, read from LDS
template <int TMS, int TNS>
struct KrOps {
    v4i a[TMS][2];
    uint32_t bits[TNS];
    uint32_t s[TNS];
};

// f(std::integral_constant<uint32_t, i>) for i = 0 .. N-1, each i a constant expression
template <class F, uint32_t... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<uint32_t, I...>) {
    (f(std::integral_constant<uint32_t, I>{}), ...);
}
template <uint32_t N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<uint32_t, N>{});
}

// s_waitcnt vmcnt(N) alone (lgkmcnt and expcnt not waited for); the gfx9 encoding
// splits vmcnt into bits 3:0 and 15:14
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64u, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((int)((N & 15u) | 0x0F70u | ((N >> 4) << 14)));
}

// dma16_s for the lanes of a constant mask only (exec set inside the assembly)
template <uint64_t LANES>
__device__ __forceinline__ void dma16_s_lanes(uint32_t voff, const void* sbase, uint32_t lds_addr) {
    if constexpr (LANES == ~0ull) {
        dma16_s(voff, sbase, lds_addr);
    } else {
        uint64_t saved;
        asm volatile(
            "s_mov_b64 %0, exec\n\ts_mov_b64 exec, %4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
            "s_mov_b64 exec, %0"
            : "=&s"(saved)
            : "v"(voff), "s"(sbase), "{m0}"(lds_addr), "s"(LANES)
            : "memory");
    }
}

template <int TMS, int TNS, int W, int R>
__global__ __launch_bounds__(64 * W) void k_gemm_kr(GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band,
                                                   uint64_t seq, const uint64_t* __restrict__ flag) {
    typedef KrLayout<TMS, TNS, W, R> T;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    // the job's error flag is read now and checked before anything is stored: the DMAs
    // below read only memory of the job, so they need not wait for it
    const uint64_t failed_seq = *flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t m0 = tile.mt * T::TM, n0 = tile.nt * T::TN;
    const uint32_t groups = j.groups;
    // the row scales of this thread's outputs (F32 jobs; the prep launch wrote them),
    // requested now: read at the store they had added a memory round trip after the sums
    constexpr uint32_t ELEMS = T::SUBS * 256u, ITEMS = (ELEMS + T::NT - 1u) / T::NT;
    float rs[ITEMS];
#pragma unroll
    for (uint32_t it = 0; it < ITEMS; ++it) {
        const uint32_t idx = T::NT * it + tid;
        const uint32_t blk = idx >> 2, e = idx & 3u, mi = (blk >> 6) / TNS;
        const uint32_t m = m0 + 16u * mi + 4u * ((blk & 63u) >> 4) + e;
        rs[it] = j.mode == MODE_SUM_SCALED && idx < ELEMS && m < j.rows ? row_scale(j, m) : 1.0f;
    }

    // 1. every round's DMAs.  Rows: position p = 64 i + lane of the 1 KiB DMA i holds
    // chunk (p & 7) ^ ((row >> 1) & 7) of row p >> 3, so that chunk c of row r sits at
    // swz128(r, c); rows past the end are clamped (never stored).  Columns: the tile's
    // TN 16-byte sign-bit chunks and TN scales are contiguous per group in the matrix
    // layout (one 64-feature tile; the tile past the last one is clamped).  Groups past
    // the last are clamped too, so that every path issues the same DMAs for the waits.
    const uint32_t part = lds_offset(smem) + wave * (R * T::ROUND_BYTES);
    uint32_t a_src[T::A_INS];
#pragma unroll
    for (uint32_t i = 0; i < T::A_INS; ++i) {
        const uint32_t p = 64u * i + lane, r = p >> 3;
        a_src[i] = min(m0 + r, j.rows - 1u) * j.k + 16u * ((p & 7u) ^ ((r >> 1) & 7u));
    }
    const uint32_t col0 = min(n0 >> 6, j.tiles - 1u) * groups * kTile + (n0 & 63u);
    const uint32_t bits_off = (col0 + min(lane, T::TN - 1u)) * 16u;
    const uint32_t sc_off = col0 * 2u + 16u * min(lane, T::SC_LANES - 1u);
    const uint32_t chunk = lane >> 4, lrow = lane & 15u;
#pragma unroll
    for (uint32_t r = 0; r < (uint32_t)R; ++r) {
        const uint32_t g = min(W * r + wave, groups - 1u);
        const uint32_t slot = part + r * T::ROUND_BYTES;
        const int8_t* qg = j.q + (size_t)g * kGroup;
#pragma unroll
        for (uint32_t i = 0; i < T::A_INS; ++i)
            dma16_s(a_src[i], qg, slot + 1024u * i);
        dma16_s_lanes<lane_mask<T::TN>()>(bits_off + g * (kTile * 16u), j.wbits, slot + T::A_BYTES);
        dma16_s_lanes<lane_mask<T::SC_LANES>()>(sc_off + g * (kTile * 2u), j.wscale,
                                                slot + T::A_BYTES + T::BITS_BYTES);
    }
    uint2* const lut = reinterpret_cast<uint2*>(smem + T::OFF_LUT);
    for (uint32_t i = tid; i < 256u; i += T::NT)
        lut[i] = make_uint2(pm1_nibble(i & 15u), pm1_nibble(i >> 4));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's table entries are written
    barrier();                           // ... and every wave's

    // 2. the rounds, software-pipelined: iteration i reads round i's operands from LDS
    // (after waiting for this wave's DMAs of round i: at most (R - 1 - i) rounds of them
    // still in flight), expands round i-1's sign bits through the byte table, and runs
    // round i-2's MFMAs with the exact products RN(scale * D) kept in registers
    const unsigned char* const mine = smem + wave * (R * T::ROUND_BYTES);
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
    v4f p[R][TMS][TNS];
    KrOps<TMS, TNS> raw[3];
    v4i b[2][TNS][2];
    const auto read = [&](auto rc) {
        constexpr uint32_t r = decltype(rc)::value;
        KrOps<TMS, TNS>& o = raw[r % 3u];
        const unsigned char* const slot = mine + r * T::ROUND_BYTES;
        wait_vm<((uint32_t)R - 1u - r) * T::DMA_PER_ROUND>();
#pragma unroll
        for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h)
                o.a[mi][h] = *reinterpret_cast<const v4i*>(slot + swz128(16u * mi + lrow, 2u * chunk + h));
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNS; ++ni) {
            const uint32_t f = 16u * ni + lrow;
            o.bits[ni] = *reinterpret_cast<const uint32_t*>(slot + T::A_BYTES + 16u * f + 4u * chunk);
            o.s[ni] = *reinterpret_cast<const uint16_t*>(slot + T::A_BYTES + T::BITS_BYTES + 2u * f);
        }
    };
    const auto expand = [&](auto rc) {
        constexpr uint32_t r = decltype(rc)::value;
        const KrOps<TMS, TNS>& o = raw[r % 3u];
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNS; ++ni)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) {
                const uint2 lo = lut[(o.bits[ni] >> (16u * h)) & 0xffu];
                const uint2 hi = lut[(o.bits[ni] >> (16u * h + 8u)) & 0xffu];
                b[r % 2u][ni][h] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
    };
    const auto mma = [&](auto rc) {
        constexpr uint32_t r = decltype(rc)::value;
        const KrOps<TMS, TNS>& o = raw[r % 3u];
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNS; ++ni) {
            const float sc = __half2float(__ushort_as_half((uint16_t)o.s[ni]));
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi) {
                v4i dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mi][0], b[r % 2u][ni][0], c_init, 0, 0, 0);
                dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mi][1], b[r % 2u][ni][1], dd, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    p[r][mi][ni][e] = __builtin_fmaf(sc, __int_as_float(dd[e]), cneg);
            }
        }
    };
    static_for<(uint32_t)R + 2u>([&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        if constexpr (i < (uint32_t)R)
            read(std::integral_constant<uint32_t, i>{});
        if constexpr (i >= 1u && i - 1u < (uint32_t)R)
            expand(std::integral_constant<uint32_t, i - 1u>{});
        if constexpr (i >= 2u)
            mma(std::integral_constant<uint32_t, i - 2u>{});
    });

    if (failed_seq == seq)
        return;  // an illegal input row in this job: write nothing (the whole workgroup)

    // 3. the products by group into LDS (over the operands: every wave has read its own
    // by the barrier), then the in-order sums
    __syncthreads();
    v4f* const prod = reinterpret_cast<v4f*>(smem);
#pragma unroll
    for (uint32_t r = 0; r < (uint32_t)R; ++r) {
        const uint32_t g = W * r + wave;
        if (g < groups) {
#pragma unroll
            for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
                for (uint32_t ni = 0; ni < (uint32_t)TNS; ++ni)
                    prod[(g * T::SUBS + mi * TNS + ni) * 64u + lane] = p[r][mi][ni];
        }
    }
    __syncthreads();
    // output elements tid, tid + NT, ... (element e of block (subtile, lane l) is
    // 4 (64 subtile + l) + e), their sums interleaved
    const bool scaled = j.mode == MODE_SUM_SCALED;
    const float* const prodf = reinterpret_cast<const float*>(smem) + tid;
    float acc[ITEMS];
#pragma unroll
    for (uint32_t it = 0; it < ITEMS; ++it)
        acc[it] = 0.0f;
    const auto add_group = [&](uint32_t g) {
        float v[ITEMS];
#pragma unroll
        for (uint32_t it = 0; it < ITEMS; ++it)
            v[it] = ELEMS % T::NT == 0 || T::NT * it + tid < ELEMS ? prodf[g * ELEMS + T::NT * it] : 0.0f;
#pragma unroll
        for (uint32_t it = 0; it < ITEMS; ++it)
            acc[it] = acc[it] + v[it];
    };
    uint32_t g = 0;
    for (; g + 4u <= groups; g += 4u) {
        add_group(g);
        add_group(g + 1u);
        add_group(g + 2u);
        add_group(g + 3u);
    }
    for (; g < groups; ++g)
        add_group(g);
#pragma unroll
    for (uint32_t it = 0; it < ITEMS; ++it) {
        const uint32_t idx = T::NT * it + tid;
        const uint32_t blk = idx >> 2, e = idx & 3u, sub = blk >> 6, l = blk & 63u;
        const uint32_t mi = sub / TNS, ni = sub % TNS;
        const uint32_t n = n0 + 16u * ni + (l & 15u), m = m0 + 16u * mi + 4u * (l >> 4) + e;
        if (idx >= ELEMS || n >= j.n || m >= j.rows)
            continue;
        float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
        __builtin_nontemporal_store(scaled ? acc[it] * rs[it] : acc[it], orow + n);
    }
}

// k_gemm_kc<TMS, TNW, WN, KS, G>: F32-accumulating jobs with few rows and at most G
// groups, as k_gemm_kr but with contiguous K slices handing on an accumulator instead
// of exchanging every product.  Workgroup tile (16 TMS) x (16 TNW WN); wave w = s WN + nn
// computes the 16 TMS x 16 TNW block nn of the tile over K slice s (groups s G/KS ..
// (s+1) G/KS - 1).  All waves first bring every group's rows, sign bits and scales into
// LDS by DMA (wave w the groups w, w + W, ...), one barrier; then each wave computes its
// products RN(scale * D) in registers; slice 0 adds its products in group order from +0,
// and each later slice, after a barrier, takes the running sums through LDS and adds its
// own in group order -- the reference's order with only KS - 1 exchanges of one value
// per output.  The K order inside a group is that of k_gemm_ks.
template <int TMS, int TNW, int WN, int KS, int G>
struct KcLayout {
    static constexpr uint32_t W = WN * KS, NT = 64u * W, GS = G / KS;
    static constexpr uint32_t TM = 16u * TMS, TN = 16u * TNW * WN;
    static constexpr uint32_t A_BYTES = TM * 128u, A_INS = A_BYTES / 1024u;
    static constexpr uint32_t BITS_BYTES = TN * 16u, SC_BYTES = TN * 2u, SC_LANES = SC_BYTES / 16u;
    static constexpr uint32_t ROUND_BYTES = A_BYTES + BITS_BYTES + SC_BYTES;
    static constexpr uint32_t RD = (G + W - 1u) / W;  // DMA rounds per wave
    static constexpr uint32_t OPS_BYTES = G * ROUND_BYTES;
    static constexpr uint32_t OFF_LUT = OPS_BYTES, OFF_X = OFF_LUT + 2048u;
    static constexpr uint32_t SMEM = OFF_X + WN * TMS * TNW * 1024u;
    static_assert(G % KS == 0, "whole K slices");
    static_assert(A_BYTES % 1024u == 0, "whole 1 KiB row DMAs");
    static_assert(TN <= 64u && 64u % TN == 0, "a tile's columns lie in one 64-feature tile of the matrix layout");
    static_assert(SC_BYTES % 16u == 0, "whole 16-byte scale DMAs");
    static_assert(RD * (A_INS + 2u) < 64u, "vmcnt range");
    static_assert(SMEM <= 160u * 1024u, "LDS");
};

template <int TMS, int TNW, int WN, int KS, int G>
__global__ __launch_bounds__(64 * WN * KS) void k_gemm_kc(GemmJob j, uint32_t mtiles, uint32_t ntiles, uint32_t band,
                                                         uint64_t seq, const uint64_t* __restrict__ flag) {
    typedef KcLayout<TMS, TNW, WN, KS, G> T;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    // the job's error flag, checked before anything is stored (the DMAs read only the job's
    // own memory, so they need not wait for it)
    const uint64_t failed_seq = *flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t m0 = tile.mt * T::TM, n0 = tile.nt * T::TN;
    // the row scales of this thread's outputs (F32 jobs), requested now (see k_gemm_kr)
    float rs[TMS][4];
#pragma unroll
    for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t m = m0 + 16u * mi + 4u * (lane >> 4) + e;
            rs[mi][e] = j.mode == MODE_SUM_SCALED && m < j.rows ? row_scale(j, m) : 1.0f;
        }
    const uint32_t groups = j.groups;

    // 1. the DMAs (the layout of a group as in k_gemm_kr; group g at g * ROUND_BYTES).
    // Groups past the last are clamped: the copies write the same bytes.
    uint32_t a_src[T::A_INS];
#pragma unroll
    for (uint32_t i = 0; i < T::A_INS; ++i) {
        const uint32_t p = 64u * i + lane, r = p >> 3;
        a_src[i] = min(m0 + r, j.rows - 1u) * j.k + 16u * ((p & 7u) ^ ((r >> 1) & 7u));
    }
    const uint32_t col0 = min(n0 >> 6, j.tiles - 1u) * groups * kTile + (n0 & 63u);
    const uint32_t bits_off = (col0 + min(lane, T::TN - 1u)) * 16u;
    const uint32_t sc_off = col0 * 2u + 16u * min(lane, T::SC_LANES - 1u);
    const uint32_t base = lds_offset(smem);
#pragma unroll
    for (uint32_t r = 0; r < T::RD; ++r) {
        const uint32_t g = min(T::W * r + wave, groups - 1u);
        const uint32_t slot = base + g * T::ROUND_BYTES;
        const int8_t* qg = j.q + (size_t)g * kGroup;
#pragma unroll
        for (uint32_t i = 0; i < T::A_INS; ++i)
            dma16_s(a_src[i], qg, slot + 1024u * i);
        dma16_s_lanes<lane_mask<T::TN>()>(bits_off + g * (kTile * 16u), j.wbits, slot + T::A_BYTES);
        dma16_s_lanes<lane_mask<T::SC_LANES>()>(sc_off + g * (kTile * 2u), j.wscale,
                                                slot + T::A_BYTES + T::BITS_BYTES);
    }
    uint2* const lut = reinterpret_cast<uint2*>(smem + T::OFF_LUT);
    for (uint32_t i = tid; i < 256u; i += T::NT)
        lut[i] = make_uint2(pm1_nibble(i & 15u), pm1_nibble(i >> 4));
    wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's DMAs and table entries are done
    barrier();                           // ... and every wave's

    // 2. this wave's products over its K slice, software-pipelined as in k_gemm_kr
    const uint32_t nn = wave % WN, s = wave / WN, g0 = s * T::GS;
    const uint32_t chunk = lane >> 4, lrow = lane & 15u;
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
    v4f p[T::GS][TMS][TNW];
    KrOps<TMS, TNW> raw[3];
    v4i b[2][TNW][2];
    const auto read = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        KrOps<TMS, TNW>& o = raw[i % 3u];
        const unsigned char* const slot = smem + min(g0 + i, groups - 1u) * T::ROUND_BYTES;
#pragma unroll
        for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h)
                o.a[mi][h] = *reinterpret_cast<const v4i*>(slot + swz128(16u * mi + lrow, 2u * chunk + h));
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni) {
            const uint32_t f = 16u * (nn * TNW + ni) + lrow;
            o.bits[ni] = *reinterpret_cast<const uint32_t*>(slot + T::A_BYTES + 16u * f + 4u * chunk);
            o.s[ni] = *reinterpret_cast<const uint16_t*>(slot + T::A_BYTES + T::BITS_BYTES + 2u * f);
        }
    };
    const auto expand = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        const KrOps<TMS, TNW>& o = raw[i % 3u];
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) {
                const uint2 lo = lut[(o.bits[ni] >> (16u * h)) & 0xffu];
                const uint2 hi = lut[(o.bits[ni] >> (16u * h + 8u)) & 0xffu];
                b[i % 2u][ni][h] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
    };
    const auto mma = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        const KrOps<TMS, TNW>& o = raw[i % 3u];
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni) {
            const float sc = __half2float(__ushort_as_half((uint16_t)o.s[ni]));
            const float cneg = sc * -kMagicValue;  // exact
#pragma unroll
            for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi) {
                v4i dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mi][0], b[i % 2u][ni][0], c_init, 0, 0, 0);
                dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[mi][1], b[i % 2u][ni][1], dd, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    p[i][mi][ni][e] = __builtin_fmaf(sc, __int_as_float(dd[e]), cneg);
            }
        }
    };
    static_for<T::GS + 2u>([&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        if constexpr (i < T::GS)
            read(std::integral_constant<uint32_t, i>{});
        if constexpr (i >= 1u && i - 1u < T::GS)
            expand(std::integral_constant<uint32_t, i - 1u>{});
        if constexpr (i >= 2u)
            mma(std::integral_constant<uint32_t, i - 2u>{});
    });
    if (failed_seq == seq)
        return;  // an illegal input row in this job: write nothing (the whole workgroup)

    // 3. the running sums along the slices: slice 0 from +0, slice t after barrier t
    v4f acc[TMS][TNW];
    v4f* const xchg = reinterpret_cast<v4f*>(smem + T::OFF_X) + nn * (TMS * TNW * 64u) + lane;
    const auto add_slice = [&]() {
#pragma unroll
        for (uint32_t i = 0; i < T::GS; ++i) {
            if (g0 + i < groups) {
#pragma unroll
                for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
                    for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[mi][ni][e] = acc[mi][ni][e] + p[i][mi][ni][e];
            }
        }
    };
#pragma unroll
    for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni)
            acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (s == 0u)
        add_slice();
#pragma unroll
    for (uint32_t t = 1; t < (uint32_t)KS; ++t) {
        if (s == t - 1u) {
#pragma unroll
            for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
                for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni)
                    xchg[(mi * TNW + ni) * 64u] = acc[mi][ni];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        barrier();
        if (s == t) {
#pragma unroll
            for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
                for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni)
                    acc[mi][ni] = xchg[(mi * TNW + ni) * 64u];
            add_slice();
        }
    }
    if (s != (uint32_t)KS - 1u)
        return;
    const bool scaled = j.mode == MODE_SUM_SCALED;
#pragma unroll
    for (uint32_t mi = 0; mi < (uint32_t)TMS; ++mi)
#pragma unroll
        for (uint32_t ni = 0; ni < (uint32_t)TNW; ++ni) {
            const uint32_t n = n0 + 16u * (nn * TNW + ni) + lrow;
            if (n >= j.n)
                continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + 16u * mi + 4u * chunk + e;
                if (m >= j.rows)
                    continue;
                float* orow = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride);
                __builtin_nontemporal_store(scaled ? acc[mi][ni][e] * rs[mi][e] : acc[mi][ni][e], orow + n);
            }
        }
}

// k_gemm_mx<TM, TN, WGM, WGN>: GEMM / GEMM_F32 with a chip's worth of TM x TN tiles,
// one workgroup of WGM x WGN waves per CU (two waves per SIMD for 8 waves).  Per
// 128-weight group g:
//   * the TM rows' quantised bytes and the TN columns' sign bits and scales reach LDS by
//     DMA, DEPTH groups ahead, in a ring of DEPTH + 1 slots: A_INS + 1 DMA instructions
//     per wave and group (one barrier per group: every wave has read slot g-1 before the
//     DMAs of group g+DEPTH reuse it);
//   * every wave expands its own columns' sign bits (4 bytes per lane) straight into
//     +1/-1 MFMA operands through the byte table -- no +1/-1 tile in LDS;
//   * group g-1's exact epilogue on each 16 x 16 subtile (the other D set) comes before
//     group g's first-half MFMA on it; the second halves follow, each accumulating onto
//     a first half issued MS * NS MFMAs earlier.
// The K order inside a group is that of k_gemm_ks / k_gemm_wv (lane chunk c: weights
// 32c .. 32c+31, MFMA half h the 16 from 32c + 16h).  The tile leaves through LDS as
// 16-byte row-contiguous stores where the output view allows (stored straight from the
// registers, 64 bytes per row and instruction, it ran as fast but wrote 1.3-1.45x the
// output's bytes).
template <int TM, int TN, int WGM, int WGN>
struct MxTiling {
    static constexpr uint32_t WAVES = WGM * WGN, THREADS = 64u * WAVES;
    static constexpr uint32_t WTM = TM / WGM, WTN = TN / WGN, MS = WTM / 16u, NS = WTN / 16u;
    static constexpr uint32_t DEPTH = 3, SLOTS = DEPTH + 1;
    static constexpr uint32_t A_INS = TM * 8u / THREADS;  // 16-byte row chunks per thread and group
    // a slot: rows [TM][128] (chunks swizzled), then the columns' 16-byte sign-bit chunks
    // [TN][16], then their fp16 scales [TN]; the column part as TN + TN / 8 chunks of 16
    // bytes, CPW per wave
    static constexpr uint32_t A_BYTES = TM * 128u, COL_CHUNKS = TN + TN / 8u, CPW = COL_CHUNKS / WAVES;
    static constexpr uint32_t SLOT_BYTES = A_BYTES + 16u * COL_CHUNKS;
    // vector-memory operations a wave issues per group (row DMAs, one column DMA)
    static constexpr uint32_t VM_PER_GROUP = A_INS + 1u;
    // the byte table in 32 copies, entry e of copy c at (32 e + c) * 8 bytes: lane l reads
    // copy l % 32, i.e. only its own pair of the 64 banks, so that the lanes' lookups of
    // arbitrary entries never conflict
    static constexpr uint32_t LUT_COPIES = 32;
    static constexpr uint32_t OFF_LUT = SLOTS * SLOT_BYTES, LOOP_BYTES = OFF_LUT + 256u * LUT_COPIES * 8u;
    static constexpr uint32_t OUT_STRIDE = TN + 4u;  // floats per staged output row
    static constexpr uint32_t OUT_BYTES = TM * OUT_STRIDE * 4u;
    static constexpr uint32_t SMEM = LOOP_BYTES > OUT_BYTES ? LOOP_BYTES : OUT_BYTES;
    static_assert(TM % (16 * WGM) == 0 && TN % (16 * WGN) == 0, "wave tiles of 16 x 16 subtiles");
    static_assert(TN % 64 == 0, "whole 64-feature tiles of the matrix layout");
    static_assert(TM * 8u % THREADS == 0 && A_INS >= 1u, "whole row DMAs per thread");
    static_assert(COL_CHUNKS % WAVES == 0 && CPW <= 64u, "column DMA chunks per wave");
    static_assert(SLOT_BYTES % 16u == 0 && OFF_LUT % 16u == 0, "16-byte DMA destinations");
    static_assert((DEPTH - 1u) * VM_PER_GROUP < 64u, "vmcnt range");
    static_assert(SMEM <= 160u * 1024u, "LDS");
    static_assert(TM * TN / 4u % THREADS == 0, "output chunks per thread");
};

// s_waitcnt vmcnt(N) lgkmcnt(0) for N < 64 (the gfx9 encoding splits vmcnt into bits
// 3:0 and 15:14)
template <uint32_t N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N < 64u, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((int)((N & 15u) | 0x0070u | ((N >> 4) << 14)));
}

template <int TM, int TN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_mx(GemmJob j, uint32_t mtiles, uint32_t ntiles,
                                                            uint32_t band, uint64_t seq,
                                                            const uint64_t* __restrict__ flag) {
    using T = MxTiling<TM, TN, WGM, WGN>;
    constexpr uint32_t MS = T::MS, NS = T::NS, THREADS = T::THREADS, DEPTH = T::DEPTH;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    if (*flag == seq)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, chunk = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    const TileRC tile = gemm_tile_of_block(blockIdx.x, gridDim.x, mtiles, ntiles, band);
    const uint32_t m0 = tile.mt * TM, n0 = tile.nt * TN;
    const uint32_t groups = j.groups;
    uint2* const lut_all = reinterpret_cast<uint2*>(smem + T::OFF_LUT);
    for (uint32_t i = tid; i < 256u * T::LUT_COPIES; i += THREADS) {
        const uint32_t e = i / T::LUT_COPIES;
        lut_all[i] = make_uint2(pm1_nibble(e & 15u), pm1_nibble(e >> 4));
    }
    const uint2* const lut = lut_all + (lane % T::LUT_COPIES);  // entry e at lut[32 e]

    // the rows' DMA: instruction i of wave w fills LDS chunks p = 64 (A_INS w + i) + lane
    // of a slot's rows, as a wave-uniform base plus a 32-bit per-lane offset (the rows of
    // one launch chunk are far below 4 GiB); rows past the end are clamped (never stored)
    uint32_t a_src[T::A_INS];
#pragma unroll
    for (uint32_t i = 0; i < T::A_INS; ++i) {
        const uint32_t p = 64u * (T::A_INS * wave + i) + lane, r = p >> 3;
        const uint32_t c = (p & 7u) ^ ((r >> 1) & 7u);
        a_src[i] = min(m0 + r, j.rows - 1u) * j.k + 16u * c;
    }
    // the columns' DMA: chunk k = CPW w + lane of wave w (lanes past CPW inactive): chunk
    // k < TN is the 16 bytes of sign bits of column n0 + k, chunk TN + c the scales of
    // columns n0 + 8c .. +7; per group the bits advance 1 KiB (one 64-feature tile) and
    // the scales 128 bytes.  The matrix tile of columns past the last one is clamped
    // (never stored).
    const unsigned char* col_src;
    uint32_t col_step;
    {
        const uint32_t k = T::CPW * wave + min(lane, T::CPW - 1u);
        const uint32_t col = k < (uint32_t)TN ? k : 8u * (k - TN);
        const size_t t = min((n0 + col) >> 6, j.tiles - 1u);
        if (k < (uint32_t)TN) {
            col_src = reinterpret_cast<const unsigned char*>(j.wbits) + (t * groups * kTile + (col & 63u)) * 16u;
            col_step = kTile * 16u;
        } else {
            col_src = reinterpret_cast<const unsigned char*>(j.wscale) + (t * groups * kTile + (col & 63u)) * 2u;
            col_step = kTile * 2u;
        }
    }
    const uint32_t la0 = lds_offset(smem);
    auto issue_group = [&](uint32_t g) {
        const uint32_t gg = min(g, groups - 1u);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(j.q) + (size_t)gg * kGroup;
        const uint32_t slot = la0 + (g % T::SLOTS) * T::SLOT_BYTES;
#pragma unroll
        for (uint32_t i = 0; i < T::A_INS; ++i)
            dma16_s(a_src[i], base, slot + 1024u * (T::A_INS * wave + i));
        dma16_lanes<lane_mask<T::CPW>()>(col_src + (size_t)gg * col_step, slot + T::A_BYTES + 16u * T::CPW * wave);
    };
    // A operand rows of this wave in a slot: row r = wm * WTM + 16 mi + (lane & 15)
    uint32_t a_off[MS][2];
#pragma unroll
    for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h)
            a_off[mi][h] = swz128(wm * T::WTM + 16u * mi + (lane & 15u), 2u * chunk + h);
    // this lane's columns in a slot: 4 bytes of sign bits (chunk c of the 16) and the scale
    const uint32_t col0 = wn * T::WTN + (lane & 15u);

    v4i dd[2][MS][NS];
    float acc[MS][NS][4];
#pragma unroll
    for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = 0.0f;
    float sc_prev[NS], cneg_prev[NS];
    const v4i c_init = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};

    // group g (D set e = g % 2): its MFMAs into dd[e]; with `epi`, group g-1's epilogue
    // from dd[e ^ 1] (scales sc_prev)
    auto step = [&](uint32_t g, uint32_t e, bool epi) {
        // this wave's DMAs of group g have landed (those of groups g+1 .. g+DEPTH-1 are
        // newer); then every wave's have, and every wave has read the slot that group
        // g+DEPTH takes
        wait_vm_lgkm0<(DEPTH - 1u) * T::VM_PER_GROUP>();
        barrier();
        const unsigned char* slot = smem + (g % T::SLOTS) * T::SLOT_BYTES;
        uint32_t bits[NS];
        uint16_t sraw[NS];
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni) {
            bits[ni] = *reinterpret_cast<const uint32_t*>(slot + T::A_BYTES + (col0 + 16u * ni) * 16u + 4u * chunk);
            sraw[ni] = *reinterpret_cast<const uint16_t*>(slot + T::A_BYTES + 16u * TN + (col0 + 16u * ni) * 2u);
        }
        v4i a[MS][2], b[NS][2];
#pragma unroll
        for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h)
                a[mi][h] = *reinterpret_cast<const v4i*>(slot + a_off[mi][h]);
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni)
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint2 lo = lut[T::LUT_COPIES * ((bits[ni] >> (16u * h)) & 0xffu)];
                const uint2 hi = lut[T::LUT_COPIES * ((bits[ni] >> (16u * h + 8u)) & 0xffu)];
                b[ni][h] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
        float sc[NS], cneg[NS];
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni) {
            sc[ni] = __half2float(__ushort_as_half(sraw[ni]));
            // the converted scale as a register operand of the epilogue's FMAs (folded into
            // them, the conversion would make each a mixed-precision FMA)
            asm volatile("" : "+v"(sc[ni]));
            cneg[ni] = sc[ni] * -kMagicValue;  // exact
        }
        issue_group(g + DEPTH);
        // the first halves of all subtiles (independent MFMAs, each after group g-1's
        // epilogue on that subtile), then the second halves, each accumulating onto a first
        // half issued MS * NS MFMAs earlier (a dependent MFMA right behind its source waits
        // for that one's result)
#pragma unroll
        for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
            for (uint32_t ni = 0; ni < NS; ++ni) {
                if (epi) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc_prev[ni],
                                                                         __int_as_float(dd[e ^ 1u][mi][ni][r]),
                                                                         cneg_prev[ni]);
                }
                dd[e][mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi][0], b[ni][0], c_init, 0, 0, 0);
            }
#pragma unroll
        for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
            for (uint32_t ni = 0; ni < NS; ++ni)
                dd[e][mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi][1], b[ni][1], dd[e][mi][ni], 0, 0, 0);
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni) {
            sc_prev[ni] = sc[ni];
            cneg_prev[ni] = cneg[ni];
        }
    };

    // prologue: groups 0 .. DEPTH-1 (the order the waits of step() count on)
#pragma unroll
    for (uint32_t g = 0; g < DEPTH; ++g)
        issue_group(g);
    step(0, 0, false);
    uint32_t g = 1;
    for (; g + 1u < groups; g += 2u) {
        step(g, 1, true);
        step(g + 1u, 0, true);
    }
    const bool last_in_d1 = g < groups;
    if (last_in_d1)
        step(g, 1, true);
    // epilogue of the last group
#pragma unroll
    for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mi][ni][r] = acc[mi][ni][r] + __builtin_fmaf(sc_prev[ni],
                                                                 __int_as_float(last_in_d1 ? dd[1][mi][ni][r]
                                                                                           : dd[0][mi][ni][r]),
                                                                 cneg_prev[ni]);
    // no DMA may still be writing LDS when it is reused for the staged tile
    wait_dma<0>();
    barrier();
    float* const so = reinterpret_cast<float*>(smem);
#pragma unroll
    for (uint32_t mi = 0; mi < MS; ++mi)
#pragma unroll
        for (uint32_t ni = 0; ni < NS; ++ni)
#pragma unroll
            for (uint32_t r = 0; r < 4; ++r)
                so[(wm * T::WTM + 16u * mi + 4u * chunk + r) * T::OUT_STRIDE + wn * T::WTN + 16u * ni + (lane & 15u)] =
                    acc[mi][ni][r];
    barrier();
    const bool vec = ((j.out_stride | (uint64_t)(uintptr_t)j.out) & 15u) == 0;
    const bool scaled = j.mode == MODE_SUM_SCALED;
#pragma unroll
    for (uint32_t c0 = 0; c0 < TM * TN / 4u; c0 += THREADS) {
        const uint32_t c = c0 + tid, row = c / (TN / 4u), col = 4u * (c % (TN / 4u));
        const uint32_t m = m0 + row, n = n0 + col;
        if (m >= j.rows || n >= j.n)
            continue;
        float4 v = *reinterpret_cast<const float4*>(so + row * T::OUT_STRIDE + col);
        if (scaled) {
            const float s = row_scale(j, m);
            v.x = v.x * s;
            v.y = v.y * s;
            v.z = v.z * s;
            v.w = v.w * s;
        }
        float* dst = reinterpret_cast<float*>(j.out + (size_t)m * j.out_stride) + n;
        if (vec && n + 4u <= j.n) {
            const v4f w = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(w, reinterpret_cast<v4f*>(dst));
        } else {
            dst[0] = v.x;
            if (n + 1u < j.n)
                dst[1] = v.y;
            if (n + 2u < j.n)
                dst[2] = v.z;
            if (n + 3u < j.n)
                dst[3] = v.w;
        }
    }
}

// The band width (in M tiles) of gemm_tile_of_block: an XCD covering band M tiles of
// mtiles and (tiles / 8 / band) N tiles makes the rows (rows * k bytes) be fetched
// into about 8 * band / mtiles L2s and the weights (1.125 bits each) into
// mtiles / band of them; the band minimising the sum.
uint32_t gemm_band(const GemmJob& job, uint32_t mtiles) {
    const double a = (double)job.rows * job.k, b = (double)job.n * job.k * 0.140625;
    uint32_t best = 1;
    double best_cost = 0.0;
    for (uint32_t band = 1; band <= mtiles; ++band) {
        const double xcds_per_mtile = std::min(8.0, 8.0 * band / mtiles);
        const double cost = a * std::max(1.0, xcds_per_mtile) + b * ((mtiles + band - 1u) / band);
        if (band == 1 || cost < best_cost)
            best = band, best_cost = cost;
    }
    return best;
}

template <int TMS, int TNS, int W, int DEPTH>
hipError_t launch_ks(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + 16u * TMS - 1u) / (16u * TMS);
    const uint32_t ntiles = (job.n + 16u * TNS - 1u) / (16u * TNS);
    launch_kernel((k_gemm_ks<TMS, TNS, W, DEPTH>), dim3(mtiles * ntiles), dim3(64 * W), 0, stream, job, mtiles, ntiles,
                  gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

template <int TMS, int TNS, int W, int R>
hipError_t launch_kr(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    if (job.groups > (uint32_t)(W * R) || job.mode == MODE_DOT_I16)
        return hipErrorInvalidValue;  // the selection below never asks for this
    const uint32_t mtiles = (job.rows + 16u * TMS - 1u) / (16u * TMS);
    const uint32_t ntiles = (job.n + 16u * TNS - 1u) / (16u * TNS);
    launch_kernel((k_gemm_kr<TMS, TNS, W, R>), dim3(mtiles * ntiles), dim3(64 * W), 0, stream, job, mtiles, ntiles,
                  gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

template <int TMS, int TNW, int WN, int KS, int G>
hipError_t launch_kc(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    if (job.groups > (uint32_t)G || job.mode == MODE_DOT_I16)
        return hipErrorInvalidValue;  // the selection below never asks for this
    const uint32_t mtiles = (job.rows + 16u * TMS - 1u) / (16u * TMS);
    const uint32_t ntiles = (job.n + 16u * TNW * WN - 1u) / (16u * TNW * WN);
    launch_kernel((k_gemm_kc<TMS, TNW, WN, KS, G>), dim3(mtiles * ntiles), dim3(64 * WN * KS), 0, stream, job, mtiles,
                  ntiles, gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

template <int TM, int TN, int WGM, int WGN>
hipError_t launch_mx(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + TM - 1u) / TM, ntiles = (job.n + TN - 1u) / TN;
    launch_kernel((k_gemm_mx<TM, TN, WGM, WGN>), dim3(mtiles * ntiles), dim3(64 * WGM * WGN), 0, stream, job,
                  mtiles, ntiles, gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

template <int MS, int NS, int WM, int WN, int DEPTH>
hipError_t launch_wv(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    constexpr uint32_t TM = 16u * MS * WM, TN = 16u * NS * WN;
    const uint32_t mtiles = (job.rows + TM - 1u) / TM, ntiles = (job.n + TN - 1u) / TN;
    launch_kernel((k_gemm_wv<MS, NS, WM, WN, DEPTH>), dim3(mtiles * ntiles), dim3(64 * WM * WN), 0, stream, job,
                  mtiles, ntiles, gemm_band(job, mtiles), seq, flag);
    return hipGetLastError();
}

template <int TM, int TN, int WGM, int WGN>
hipError_t launch_bits(hipStream_t stream, const GemmJob& job, uint64_t seq, const uint64_t* flag) {
    const uint32_t mtiles = (job.rows + TM - 1u) / TM, ntiles = (job.n + TN - 1u) / TN;
    const dim3 grid(mtiles * ntiles), block(64 * WGM * WGN);
    const uint32_t band = gemm_band(job, mtiles);
    if (job.mode == MODE_DOT_I16)
        launch_kernel((k_gemm_bits<TM, TN, WGM, WGN, true>), grid, block, 0, stream, job, mtiles, ntiles, band, seq,
                      flag);
    else
        launch_kernel((k_gemm_bits<TM, TN, WGM, WGN, false>), grid, block, 0, stream, job, mtiles, ntiles, band, seq,
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
#ifndef BNN_GEMM_CO
#define BNN_GEMM_CO 1  // F32-accumulating jobs with a 128 x 128 tile per CU: two workgroups per CU (k_gemm_co)
#endif
    // Few rows: K split over the waves of a workgroup, every wave's operands brought into
    // LDS by DMA before anything is computed (k_gemm_kr, k_gemm_kc).  The rules follow a
    // forced-choice sweep over K = 1024..8192, N = 1024..8192 and 8..256 rows (all outputs
    // bit-identical); against the kernels below, e.g. 2048->6144 x 64 rows 9.6 -> 5.8 us,
    // 6144->2048 x 64 rows 9.6 -> 6.4 us, 2048->2048 x 128 rows 7.7 -> 4.6 us, 4096->2048 x
    // 256 rows 14.5 -> 12.2 us, 6144->2048 x 128 rows 13.3 -> 9.6 us, 8192->2048 x 32 rows
    // 9.2 -> 7.0 us.  Up to 16 groups: 32 x 32 tiles while they fit one round of two per CU,
    // then 32 x 64 tiles while those fit one round (16 waves of one group each above 8 groups),
    // then 32 x 32 tiles up to 4.5 rounds
    // (not for 8 groups, where the tiled kernels win past one round); 17..32 groups: 16 x 32
    // tiles in one round, then 32 x 32 up to three rounds; 33..48 groups: 16 x 32 tiles, then
    // 16 x 64 tiles with the slices' running sums handed on (k_gemm_kc), each in one round;
    // 49..64 groups: 16 x 16 tiles in one round.
    if (job.mode != MODE_DOT_I16) {
        const uint32_t g = job.groups;
        if (g <= 16u) {
            if (job.rows <= 16u && blocks(16, 32) <= cus)
                return launch_kr<1, 2, 4, 4>(stream, job, seq, flag);
            if (blocks(32, 32) <= cus)
                return launch_kr<2, 2, 8, 2>(stream, job, seq, flag);
            if (blocks(32, 64) <= cus && g > 8u)
                return launch_kr<2, 4, 16, 1>(stream, job, seq, flag);  // 2048->6144 x 64 rows 6.2 -> 5.7 us
            if (blocks(32, 64) <= cus)
                return launch_kr<2, 4, 8, 2>(stream, job, seq, flag);
            if (g > 8u && blocks(32, 32) <= 9u * cus / 2u)
                return launch_kr<2, 2, 8, 2>(stream, job, seq, flag);
        } else if (g <= 32u) {
            if (blocks(16, 32) <= cus)
                return launch_kr<1, 2, 8, 4>(stream, job, seq, flag);
            if (blocks(32, 32) <= 3u * cus)
                return launch_kr<2, 2, 8, 4>(stream, job, seq, flag);
        } else if (g <= 48u) {
            if (blocks(16, 32) <= cus)
                return launch_kr<1, 2, 8, 6>(stream, job, seq, flag);
            if (blocks(16, 64) <= cus)
                return launch_kc<1, 1, 4, 2, 48>(stream, job, seq, flag);
        } else if (g <= 64u) {
            if (blocks(16, 16) <= cus)
                return launch_kc<1, 1, 1, 8, 64>(stream, job, seq, flag);
        }
    }
    // few rows past the rules above (more than 48 groups and more than a round of 16 x 16
    // tiles): one wave per 16 x 16 output block with its operands straight in registers,
    // while that makes at most three waves per CU (the blocks of 16 columns each load their
    // rows, and more of them outrun the loads a CU keeps in flight)
    if (job.mode != MODE_DOT_I16 && job.rows <= 64u && (job.rows <= 32u || job.groups <= 16u) &&
        blocks(16, 16) <= 3u * cus)
        return launch_wv<1, 1, 1, 1, 8>(stream, job, seq, flag);
    // K >= 6144 with between half a round and one round of 32 x 64 tiles: eight waves
    // splitting K per tile (6144->2048 x 256 rows 17.1 us against 19.1 us for a wave per
    // 32 x 32 block, 8192->2048 x 256 21.6 against 23.3, 8192->1024 x 320-512 21.7-22.2
    // against 24.2-28.4; forced-choice sweep, bit-identical outputs; it loses at K = 4096,
    // below half a round and from a second round on)
    if (job.mode != MODE_DOT_I16 && job.groups >= 48u && blocks(32, 64) > cus / 2u && blocks(32, 64) <= cus)
        return launch_ks<2, 4, 8, 3>(stream, job, seq, flag);
    // K split over four waves per 32 x 64 tile: 17..47 groups with between half a round and
    // one round of tiles (4096->2048 x 192 rows 14.0 us against 15.9 for 32 x 64
    // workgroup tiles, 4096->6144 x 48-64 rows 13.9-14.2 against 15.7-15.9,
    // 3072->8100 x 40-64 rows 12.0-12.2 against 13.3), and >= 48 groups with one to two
    // rounds (6144->2048 x 384-512 rows 24.7-25.4 against 26.3-26.8, 6144->6144 x
    // 96-128 rows 23.8-24.4 against 26.1-26.5; forced-choice sweeps, bit-identical
    // outputs; at 16 groups and from a third round on the tiled kernels win)
    if (job.mode != MODE_DOT_I16 && job.groups > 16u && job.groups < 48u && blocks(32, 64) > cus / 2u &&
        blocks(32, 64) <= cus)
        return launch_ks<2, 4, 4, 3>(stream, job, seq, flag);
    if (job.mode != MODE_DOT_I16 && job.groups >= 48u && blocks(32, 64) > cus && blocks(32, 64) <= 2u * cus)
        return launch_ks<2, 4, 4, 3>(stream, job, seq, flag);
    // a long K (>= 32 groups) with two to three 32 x 32 blocks per CU: a wave per block
    // beats the tiled kernels, whose per-group steps serialise over the long K
    if (job.mode != MODE_DOT_I16 && job.groups >= 32u && blocks(32, 32) >= 2u * cus && blocks(32, 32) <= 3u * cus)
        return launch_wv<2, 2, 1, 1, 4>(stream, job, seq, flag);
    if (job.mode != MODE_DOT_I16 && blocks(128, 192) >= cus)
        return launch_mx<128, 192, 2, 4>(stream, job, seq, flag);
    if (job.mode != MODE_DOT_I16 && blocks(64, 128) >= cus && job.groups >= 32u)
        return launch_mx<64, 128, 2, 4>(stream, job, seq, flag);
    if (BNN_GEMM_CO && job.mode != MODE_DOT_I16 && blocks(128, 128) >= cus)
        return launch_co<128, 128, 2, 2>(stream, job, seq, flag);
    // 128 x 128 tiles also where 64 x 128 ones would need a second round of workgroups
    // (one 8-wave 64 x 128 workgroup per CU fits the registers): 1.26-1.43x measured at
    // 144-192 tiles of 128 x 128
    if (blocks(128, 128) >= cus || blocks(64, 128) > cus)
        return launch_bits<128, 128, 2, 4>(stream, job, seq, flag);
    if (blocks(64, 128) >= cus)
        return launch_bits<64, 128, 2, 4>(stream, job, seq, flag);
    if (blocks(64, 64) >= cus)
        return launch_bits<64, 64, 2, 2>(stream, job, seq, flag);
    const uint64_t enough = cus * 3u / 4u;
    if (job.mode != MODE_DOT_I16 && blocks(32, 64) < enough && blocks(32, 32) <= cus) {
        // too few tiles for the CUs (jobs of more than 48 groups get here): K split across
        // eight waves of a workgroup with 32 x 32 tiles while those fit one round, else four
        // waves with 32 x 16 tiles
        if (blocks(32, 32) >= enough)
            return launch_ks<2, 2, 8, 3>(stream, job, seq, flag);
        return launch_ks<2, 1, 4, 3>(stream, job, seq, flag);
    }
    // three quarters of a round of 64 x 64 tiles: those beat a round and more of 32 x 64
    // ones (2048->2048 x 384 rows 11.7 us against 12.6, 2048->6144 x 96-128 rows 11.6-11.7
    // against 12.0-12.4)
    if (blocks(64, 64) >= enough)
        return launch_bits<64, 64, 2, 2>(stream, job, seq, flag);
    return launch_bits<32, 64, 2, 2>(stream, job, seq, flag);
}

}  // namespace bnnhip
