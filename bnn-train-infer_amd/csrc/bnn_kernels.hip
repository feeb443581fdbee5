// gfx950 kernels of the HIP backend for the BNN accelerator API v2.
//
// Numeric contract (reference bnn-accelerator/bnn-accelerator.h:133-149, 191-199;
// reference algorithm bnn-accelerator/soft-bnn-accelerator.c:175-276):
//   D[m][n][g] = sum over the 128 k of group g of Q[m][k] * (+1 | -1)   exact integer
//   Z[m][n]    = ((0 + F32(scale[n][0])*D[..][0]) + F32(scale[n][1])*D[..][1]) + ...
//                each product and each sum rounded to binary32, no FMA
//   F32 ops    : Q from full-row absmax quantisation, Y = F32(Z * s)
// Every FP32 operation below is a separately rounded IEEE operation: contraction
// is disabled for the whole file and the build passes -ffp-contract=off,
// -fhip-fp32-correctly-rounded-divide-sqrt and -fno-gpu-flush-denormals-to-zero.
// The products F32(scale)*F32(D) do not depend on order, so they are formed in
// parallel by the waves that computed D; only the additions run in group order.
//
// Group dot by bit planes.  With the activation byte Q as two's complement bits
// q_0..q_7 and the weight bits b_k (1 = +1):
//   pos = sum_{b_k = 1} Q_k = sum_{j<7} 2^j popc(B & P_j) - 2^7 popc(B & P_7)
//   D   = 2*pos - sum_k Q_k
// where P_j is the 128-bit mask of bit j over the group: 8 x 4 (AND + BCNT) per
// 128 weights, about 0.56 VALU op per weight, with the sign bits streamed
// straight from HBM at 1.125 bit per weight (bits + fp16 scales).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "bnn_bitplane.h"
#include "bnn_internal.h"

#pragma clang fp contract(off)

extern "C" __device__ int __ockl_wfred_add_i32(int);

namespace bnnhip {
namespace {

constexpr int kLdsPitch = 65;                     // words per group row of the D/term exchange


// Nontemporal (streaming) stores for results written once per launch: they are not
// kept dirty in the L2s, which the end-of-kernel release would otherwise write back
// (GEMV_F32 2048->6144 x 608: 182 -> 177 us per dot launch).
template <class T>
__device__ __forceinline__ void gstore_stream(T* p, T v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) T*)p);
}
// 16 bytes at a 16-byte aligned address
__device__ __forceinline__ void gstore16(int16_t* p, u32x4 v) { *(__attribute__((address_space(1))) u32x4*)p = v; }
// eight D values (|D| <= 16256) as int16 pairs, element 2i in the low half of word i
__device__ __forceinline__ u32x4 pack8(const int* d) {
    u32x4 v;
    v.x = ((uint32_t)d[0] & 0xffffu) | ((uint32_t)d[1] << 16);
    v.y = ((uint32_t)d[2] & 0xffffu) | ((uint32_t)d[3] << 16);
    v.z = ((uint32_t)d[4] & 0xffffu) | ((uint32_t)d[5] << 16);
    v.w = ((uint32_t)d[6] & 0xffffu) | ((uint32_t)d[7] << 16);
    return v;
}

__device__ __forceinline__ float load_f32(const unsigned char* row, uint32_t k, bool aligned) {
    if (aligned)
        return reinterpret_cast<const float*>(row)[k];
    float v;
    __builtin_memcpy(&v, row + (size_t)k * 4u, 4);  // byte loads for unaligned views
    return v;
}


// ---------------------------------------------------------------------------
// prep: one workgroup (256 threads) per activation row.  Checks the logical row
// (-128 for I8, NaN/Inf for F32: soft-bnn-accelerator.c:278-308), derives the
// row scale, quantises, and writes bit planes, group sums and (optionally) Q.
// Thread t owns elements k = t + 256 i; all its loads are issued before any use.
// ---------------------------------------------------------------------------
// Threads per row: a launch with few rows is latency-bound and gives each row 1024
// threads (short serial chains per wave); a launch with many rows gives each row
// 512 (measured best for a full chip of rows).
constexpr int kPrepThreadsFew = 1024, kPrepThreadsMany = 512;
constexpr uint32_t kPrepManyRows = 256;

// PER bounds the values per thread (K <= NT * PER): the kernel is instantiated per
// bound so that a row runs code only as long as its K needs -- a launch of a few
// microseconds is otherwise dominated by fetching the instructions of the longest
// (K = 8192) unrolled form into cold instruction caches.
template <int NT, int PER, bool F32, bool ALIGNED>
__device__ void prep_row_t(const PrepJob& j, uint32_t m, bool validate_only, uint64_t seq, uint64_t* flag,
                           uint64_t* host_status) {
    constexpr int kPrepThreads = NT, kPrepWaves = NT / 64, kPrepPerThread = PER;
    constexpr int kPrepGroupsPerIter = NT / kGroup;
    static_assert(NT % 128 == 0 && NT * PER <= (int)kMaxFeatures, "whole groups per iteration");
    static_assert(kMaxFeatures / kGroup <= NT, "one thread per group for the group sums");
    __shared__ float red_max[kPrepWaves];
    __shared__ int red_sum[kPrepPerThread][kPrepWaves];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t k_total = j.k, groups = k_total / kGroup;
    const uint32_t iters = (k_total + kPrepThreads - 1u) / kPrepThreads;
    constexpr bool f32 = F32, aligned = ALIGNED;
    const unsigned char* row = j.in + (size_t)m * j.in_stride;

    // pass 1: load the whole logical row (registers), legality and absmax
    int raw[kPrepPerThread];  // float bits (F32) or the sign-extended byte (I8)
#pragma unroll
    for (int i = 0; i < kPrepPerThread; ++i) {
        const uint32_t k = tid + (uint32_t)kPrepThreads * i;
        raw[i] = 0;
        if ((uint32_t)i < iters && k < k_total)
            raw[i] = f32 ? __float_as_int(load_f32(row, k, aligned)) : (int)(int8_t)row[k];
    }
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < kPrepPerThread; ++i) {
        if (f32) {
            const float v = __int_as_float(raw[i]);
            bad |= !__builtin_isfinite(v);
            amax = fmaxf(amax, fabsf(v));
        } else {
            bad |= (raw[i] == -128);
        }
    }
    if (__syncthreads_or(bad)) {
        if (tid == 0)
            raise_flag(seq, flag, host_status);
        return;
    }
    if (validate_only)
        return;

    float s = 1.0f;
    if (f32) {
        amax = wave_max_nonneg(amax);
        if (lane == 0)
            red_max[wave] = amax;
        __syncthreads();
        amax = red_max[0];
#pragma unroll
        for (int w = 1; w < kPrepWaves; ++w)
            amax = fmaxf(amax, red_max[w]);
        s = quant_row_scale(amax);
    }

    const float rcp = quant_rcp(s);
    const bool exact = quant_exact(s);  // 1 / s may overflow
    // pass 2: quantise; in iteration i wave w owns the 64 consecutive k of half (w & 1)
    // of group kPrepGroupsPerIter*i + (w >> 1)
    uint32_t* planes = j.planes ? j.planes + (size_t)m * groups * kPlaneWords : nullptr;
#pragma unroll
    for (int i = 0; i < kPrepPerThread; ++i) {
        const uint32_t base = (uint32_t)kPrepThreads * i;
        if ((uint32_t)i < iters && base + wave * 64u < k_total) {  // K % 128 == 0: whole waves
            const int q = f32 ? quantize_rcp(__int_as_float(raw[i]), s, rcp, exact) : raw[i];
            if (j.q)
                gstore_stream(j.q + (size_t)m * k_total + base + tid, (int8_t)q);
            if (!planes)  // matrix-core rows: Q only
                continue;
            // bit planes of these 64 values, and their sum as a wave reduction (vector
            // ops: popcounts of the masks would queue the CU's waves on its one scalar unit)
            uint32_t word = 0;
            plane_mask_words(q, word);  // lane 2b / 2b + 1: low / high half of plane b's mask
            const int part = __ockl_wfred_add_i32(q);
            const uint32_t g = (uint32_t)kPrepGroupsPerIter * i + (wave >> 1), half = wave & 1u;
            if (lane < 16u)
                gstore_stream(planes + g * kPlaneWords + (lane >> 1) * 4u + half * 2u + (lane & 1u), word);
            if (lane == 0)
                red_sum[i][wave] = part;
        }
    }
    __syncthreads();
    if (planes && tid < groups)
        gstore_stream(j.sums + (size_t)m * groups + tid,
                      red_sum[tid / kPrepGroupsPerIter][(tid % kPrepGroupsPerIter) * 2u] +
                          red_sum[tid / kPrepGroupsPerIter][(tid % kPrepGroupsPerIter) * 2u + 1u]);
    if (tid == 0)
        gstore_stream(j.rscale + m, s);
}

template <int NT, int PER>
__device__ __forceinline__ void prep_row(const PrepJob& j, uint32_t m, bool validate_only, uint64_t seq,
                                         uint64_t* flag, uint64_t* host_status) {
    if (j.f32 && j.aligned)
        prep_row_t<NT, PER, true, true>(j, m, validate_only, seq, flag, host_status);
    else if (j.f32)
        prep_row_t<NT, PER, true, false>(j, m, validate_only, seq, flag, host_status);
    else
        prep_row_t<NT, PER, false, true>(j, m, validate_only, seq, flag, host_status);
}

template <bool BATCH, int NT, int PER>
__global__ __launch_bounds__(NT) void k_prep(PrepJob single, const PrepJob* __restrict__ jobs,
                                              const uint32_t* __restrict__ block_job, int validate_only,
                                              uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    if (BATCH) {
        // block_job is null when every job of the batch has one row (block b = job b):
        // one dependent load less before the row's loads can issue
        const PrepJob j = jobs[block_job ? block_job[blockIdx.x] : blockIdx.x];
        prep_row<NT, PER>(j, blockIdx.x - j.first_block, false, seq, flag, host_status);
    } else {
        prep_row<NT, PER>(single, blockIdx.x, validate_only != 0, seq, flag, host_status);
    }
}

// ---------------------------------------------------------------------------
// dot: persistent workgroups of 4 waves; one work item = (job, row, TPI tiles of
// 64 features), items assigned round-robin (all workgroups stream through a
// common window of memory, which suits HBM better than one stream per workgroup).
// Wave w owns a contiguous run of the groups; lane = feature (one per tile of the
// item, sharing each group's activation planes).  With PREFETCH,
// the loads of item i + gridDim.x (job descriptor, weights, scales, the row's bit
// planes and group sums) are in flight in a second register set while item i is
// computed.  D and the rounded products go through double-buffered LDS so that
// one wave per tile adds the products in group order (F32 modes), or the
// workgroup stores D as int16 (DOT_GROUPS).
// MAXG bounds the groups per matrix (16 for K <= 2048, else 64).
// ---------------------------------------------------------------------------
enum ItemMap : int { MAP_SINGLE = 0, MAP_UNIFORM = 1, MAP_TABLE = 2 };

#ifndef BNN_DOT_TPI_SMALL
#define BNN_DOT_TPI_SMALL 1
#endif
#ifndef BNN_DOT_PREFETCH
#define BNN_DOT_PREFETCH 1
#endif
#ifndef BNN_DOT_WAVE_ITEMS
#define BNN_DOT_WAVE_ITEMS 1  // batches with K <= 2048 use one wave per item
#endif
#ifndef BNN_DOT_WAVE_WG_WAVES
#define BNN_DOT_WAVE_WG_WAVES 4  // items (waves) per workgroup; one item per wave, no persistent loop
#endif
#ifndef BNN_DOT_WAVE_MIN_ITEMS_PER_CU
// below this many items per CU the group-split kernel finishes sooner: the lm_head as 19
// chunks (2370 items, ~9 per CU) 12.0 us against 13.6 us with one wave per item; 32 no better
#define BNN_DOT_WAVE_MIN_ITEMS_PER_CU 16
#endif
#ifndef BNN_DOT_WAVE_XCDS
#define BNN_DOT_WAVE_XCDS 0  // > 1: keep consecutive workgroups on one XCD
#endif
#ifndef BNN_DOT_WAVE_LONG
#define BNN_DOT_WAVE_LONG 1  // batches with 16 < K/128 <= 64: one wave per item, groups in blocks
#endif
#ifndef BNN_DOT_WAVE_OCC
#define BNN_DOT_WAVE_OCC 4  // waves per SIMD the register budget is fitted to
#endif

template <int MAXG, int TPI>
struct DotRegs {
    static constexpr int kGpw = MAXG / (int)kDotWaves;
    static constexpr int kPlaneChunks = (MAXG * 8 + 255) / 256;  // uint4 of planes per thread
    uint4 w[TPI][kGpw];
    uint32_t sc[TPI][kGpw];
    uint4 pl[kPlaneChunks];
    int sum;
};

struct DotItem {
    DotJob j;
    uint32_t row, t0;  // first tile of the item
};

template <int MAP, int TPI>
__device__ __forceinline__ void locate(uint32_t item, const DotJob& single, const DotJob* __restrict__ jobs,
                                       const uint32_t* __restrict__ item_job, uint32_t uniform_items, DotItem& it,
                                       uint32_t& job_index) {
    uint32_t local;
    if (MAP == MAP_SINGLE) {
        it.j = single;
        local = item;
    } else if (MAP == MAP_UNIFORM) {
        const uint32_t ji = item / uniform_items;
        if (ji != job_index) {  // consecutive items mostly share the job: keep its descriptor
            it.j = jobs[ji];
            job_index = ji;
        }
        local = item - ji * uniform_items;
    } else {
        const uint32_t ji = item_job[item];
        if (ji != job_index) {
            it.j = jobs[ji];
            job_index = ji;
        }
        local = item - it.j.first_block;
    }
    const uint32_t per_row = (it.j.tiles + TPI - 1u) / TPI;
    it.row = local / per_row;
    it.t0 = (local - it.row * per_row) * TPI;
}

template <int MAXG, int TPI>
__device__ __forceinline__ void issue(const DotItem& it, uint32_t wave, uint32_t lane, uint32_t tid,
                                      DotRegs<MAXG, TPI>& r) {
    const uint32_t groups = it.j.groups;
    const uint32_t gpw = (groups + kDotWaves - 1u) / kDotWaves;
    const uint32_t g0 = wave * gpw;
    const uint32_t gcount = g0 < groups ? min(groups - g0, gpw) : 0u;
    const bool sum_mode = it.j.mode != MODE_DOT_I16;
#pragma unroll
    for (int tt = 0; tt < TPI; ++tt) {
        const uint32_t t = it.t0 + tt;
        const size_t first = ((size_t)t * groups + g0) * kTile + lane;
        const uint4* wb = it.j.wbits + first;
        const uint16_t* ws = it.j.wscale + first;
#pragma unroll
        for (int i = 0; i < DotRegs<MAXG, TPI>::kGpw; ++i) {
            if ((uint32_t)i < gcount && t < it.j.tiles) {
                r.w[tt][i] = gload(wb + i * kTile);
                r.sc[tt][i] = sum_mode ? gload(ws + i * kTile) : 0u;
            }
        }
    }
    const uint4* pl = reinterpret_cast<const uint4*>(it.j.planes + (size_t)it.row * groups * kPlaneWords);
#pragma unroll
    for (int c = 0; c < DotRegs<MAXG, TPI>::kPlaneChunks; ++c) {
        const uint32_t idx = tid + 256u * c;
        if (idx < groups * (kPlaneWords / 4u))
            r.pl[c] = gload(pl + idx);
    }
    if (tid < groups)
        r.sum = gload(it.j.sums + (size_t)it.row * groups + tid);
}

template <int MAXG, int MAP, int TPI, bool PREFETCH>
__global__ __launch_bounds__(64 * kDotWaves) void k_dot(DotJob single, const DotJob* __restrict__ jobs,
                                                        const uint32_t* __restrict__ item_job, uint32_t items,
                                                        uint32_t uniform_items, uint64_t seq,
                                                        const uint64_t* __restrict__ flag) {
    __shared__ uint4 lds_planes[2][MAXG * kPlaneWords / 4];
    __shared__ int lds_negsum[2][MAXG];
    __shared__ int lds_x[2][TPI * MAXG * kLdsPitch];  // D (int) or rounded product (float bits)
    if (*flag == seq)
        return;  // an illegal input row in this job (batch): write nothing

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t item = blockIdx.x;
    if (item >= items)
        return;
    DotItem cur, nxt;
    DotRegs<MAXG, TPI> rc, rn;
    uint32_t cur_job = 0xffffffffu, nxt_job = 0xffffffffu;
    locate<MAP, TPI>(item, single, jobs, item_job, uniform_items, cur, cur_job);
    issue<MAXG, TPI>(cur, wave, lane, tid, rc);
    nxt = cur;
    nxt_job = cur_job;
    int buf = 0;
    for (;;) {
        const uint32_t groups = cur.j.groups;
        // stage this item's planes and group sums
#pragma unroll
        for (int c = 0; c < DotRegs<MAXG, TPI>::kPlaneChunks; ++c) {
            const uint32_t idx = tid + 256u * c;
            if (idx < groups * (kPlaneWords / 4u))
                lds_planes[buf][idx] = rc.pl[c];
        }
        if (tid < groups)
            lds_negsum[buf][tid] = -rc.sum;
        const uint32_t next = item + gridDim.x;
        const bool more = next < items;
        if (PREFETCH && more) {
            locate<MAP, TPI>(next, single, jobs, item_job, uniform_items, nxt, nxt_job);
            issue<MAXG, TPI>(nxt, wave, lane, tid, rn);
        }
        __syncthreads();

        // group dots and rounded products; the planes of a group serve all TPI tiles
        const uint32_t gpw = (groups + kDotWaves - 1u) / kDotWaves;
        const uint32_t g0 = wave * gpw;
        const uint32_t gcount = g0 < groups ? min(groups - g0, gpw) : 0u;
        const bool sum_mode = cur.j.mode != MODE_DOT_I16;
        const uint32_t* lp = reinterpret_cast<const uint32_t*>(lds_planes[buf]);
#pragma unroll
        for (int i = 0; i < DotRegs<MAXG, TPI>::kGpw; ++i) {
            if ((uint32_t)i < gcount) {
                const uint32_t g = g0 + i;
                const int neg = lds_negsum[buf][g];
#pragma unroll
                for (int tt = 0; tt < TPI; ++tt) {
                    if (cur.t0 + tt < cur.j.tiles) {
                        const int d = group_dot(rc.w[tt][i], lp + g * kPlaneWords, neg);
                        int* x = &lds_x[buf][(tt * MAXG + g) * kLdsPitch + lane];
                        if (sum_mode)
                            *x = __float_as_int(__half2float(__ushort_as_half((uint16_t)rc.sc[tt][i])) * (float)d);
                        else
                            *x = d;
                    }
                }
            }
        }
        __syncthreads();

        // in-order sums (one wave per tile) or int16 stores
        unsigned char* orow = cur.j.out + (size_t)cur.row * cur.j.out_stride;
        if (!sum_mode) {
#pragma unroll
            for (int tt = 0; tt < TPI; ++tt) {
                const uint32_t t = cur.t0 + tt;
                if (t >= cur.j.tiles)
                    break;
                const uint32_t n0 = t * kTile;
                const uint32_t live = min(cur.j.n - n0, kTile);
                int16_t* o = reinterpret_cast<int16_t*>(orow) + (size_t)n0 * groups;
                for (uint32_t idx = tid; idx < live * groups; idx += 64u * kDotWaves) {
                    const uint32_t nl = idx / groups, g = idx - nl * groups;
                    o[idx] = (int16_t)lds_x[buf][(tt * MAXG + g) * kLdsPitch + nl];
                }
            }
        } else if (wave < (uint32_t)TPI && cur.t0 + wave < cur.j.tiles) {
            const uint32_t n0 = (cur.t0 + wave) * kTile;
            if (lane < min(cur.j.n - n0, kTile)) {
                const int* x = &lds_x[buf][wave * MAXG * kLdsPitch + lane];
                float acc = 0.0f;
                for (uint32_t g = 0; g < groups; ++g)
                    acc = acc + __int_as_float(x[g * kLdsPitch]);
                if (cur.j.mode == MODE_SUM_SCALED)
                    acc = acc * cur.j.rscale[cur.row];
                reinterpret_cast<float*>(orow)[n0 + lane] = acc;
            }
        }
        if (!more)
            break;
        item = next;
        if (PREFETCH) {
            cur = nxt;
            rc = rn;
        } else {
            locate<MAP, TPI>(item, single, jobs, item_job, uniform_items, cur, cur_job);
            issue<MAXG, TPI>(cur, wave, lane, tid, rc);
        }
        buf ^= 1;
    }
}

// ---------------------------------------------------------------------------
// dot, one wave per item (batches with K <= 2048): the wave loads all groups of its
// 64-feature tile (16 KB of sign bits + 2 KB of scales in flight per wave), stages
// the row's planes in its own LDS slice, and every lane adds its products in group
// order in a register -- no workgroup barriers, no product exchange.  There is no
// persistent loop: one wave per item and the hardware dispatcher balancing short
// workgroups measured faster than any fixed item-to-wave assignment.
// ---------------------------------------------------------------------------
constexpr int kWaveMaxGroups = 16;
static_assert(!BNN_DOT_WAVE_ITEMS || BNN_DOT_TPI_SMALL == 1, "wave items count one tile per item");

// Workgroups are handed out round-robin over the XCDs; with kWaveXcds > 0 the
// logical workgroup index is remapped so that consecutive items (the tiles of one
// job, which share the row's planes) run on the same XCD and its L2.
__device__ __forceinline__ uint32_t xcd_local_block(uint32_t b, uint32_t grid) {
    if (BNN_DOT_WAVE_XCDS <= 1)
        return b;
    const uint32_t x = b % BNN_DOT_WAVE_XCDS, i = b / BNN_DOT_WAVE_XCDS;
    const uint32_t q = grid / BNN_DOT_WAVE_XCDS, r = grid % BNN_DOT_WAVE_XCDS;
    return (x < r ? x * (q + 1u) : r * (q + 1u) + (x - r) * q) + i;
}

// SCALES: some job of the batch sums scaled products (GEMV, GEMV_F32, GEMM*).  A batch of
// DOT_GROUPS jobs only (SCALES = false) issues no scale loads: DOT stores D alone
// (soft-bnn-accelerator.c:260-262), so its bytes per job are bits + row + D.
template <int MAP, bool SCALES>
__global__ __launch_bounds__(64 * BNN_DOT_WAVE_WG_WAVES) __attribute__((amdgpu_waves_per_eu(BNN_DOT_WAVE_OCC)))
void k_dot_wave(const DotJob* __restrict__ jobs, const uint32_t* __restrict__ item_job, uint32_t items,
                uint32_t uniform_items, uint64_t seq, const uint64_t* __restrict__ flag) {
    __shared__ uint4 lds_planes[BNN_DOT_WAVE_WG_WAVES][kWaveMaxGroups * kPlaneWords / 4];
    // the job's error flag is only needed before the stores: its load overlaps the
    // job descriptor's instead of preceding it
    const bool failed = *flag == seq;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t item = xcd_local_block(blockIdx.x, gridDim.x) * BNN_DOT_WAVE_WG_WAVES + wave;
    if (item >= items)
        return;
    uint32_t job_index = 0xffffffffu;
    DotItem it;
    locate<MAP, 1>(item, DotJob{}, jobs, item_job, uniform_items, it, job_index);
    const uint32_t groups = it.j.groups;
    // Loads are unconditional (indexes clamped into the job's arrays) and issued
    // in the order they are consumed: the in-order load counter then lets group g
    // start as soon as its own weights have arrived.
    const uint32_t plane_chunks = groups * (kPlaneWords / 4u);
    const uint4* pl = reinterpret_cast<const uint4*>(it.j.planes + (size_t)it.row * groups * kPlaneWords);
    const uint4 p0 = gload(pl + min(lane, plane_chunks - 1u));
    const uint4 p1 = gload(pl + min(lane + 64u, plane_chunks - 1u));
    const int sum = gload(it.j.sums + (size_t)it.row * groups + min(lane, groups - 1u));
    // the row scale is loaded with the row's planes (every job's rscale is valid; the
    // prep writes 1 for integer rows), not after the dots
    const float rs = gload(it.j.rscale + it.row);
    const size_t first = (size_t)it.t0 * groups * kTile + lane;
    uint4 w[kWaveMaxGroups];
    uint32_t sc[kWaveMaxGroups];
#pragma unroll
    for (int g = 0; g < kWaveMaxGroups; ++g) {
        const size_t at = first + (size_t)min((uint32_t)g, groups - 1u) * kTile;
        w[g] = gload_stream(it.j.wbits + at);
        sc[g] = SCALES ? gload_stream(it.j.wscale + at) : 0u;
    }
    lds_planes[wave][lane] = p0;
    lds_planes[wave][lane + 64u] = p1;
    __builtin_amdgcn_wave_barrier();
    const uint4* lp = lds_planes[wave];
    const uint32_t n0 = it.t0 * kTile;
    const bool live = n0 + lane < it.j.n;
    unsigned char* orow = it.j.out + (size_t)it.row * it.j.out_stride;
    if (SCALES && it.j.mode != MODE_DOT_I16) {
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < kWaveMaxGroups; ++g) {
            if ((uint32_t)g < groups) {
                const int d = group_dot_v(w[g], lp + g * (kPlaneWords / 4), -__shfl(sum, g));
                acc = acc + __half2float(__ushort_as_half((uint16_t)sc[g])) * (float)d;
            }
        }
        if (it.j.mode == MODE_SUM_SCALED)
            acc = acc * rs;
        if (live && !failed)
            gstore_stream(reinterpret_cast<float*>(orow) + n0 + lane, acc);
    } else {
        int dv[kWaveMaxGroups];
#pragma unroll
        for (int g = 0; g < kWaveMaxGroups; ++g) {
            if ((uint32_t)g < groups)
                dv[g] = group_dot_v(w[g], lp + g * (kPlaneWords / 4), -__shfl(sum, g));
        }
        int16_t* o = reinterpret_cast<int16_t*>(orow) + (size_t)(n0 + lane) * groups;
        if (live && !failed) {
            if (groups % 8u == 0 && ((uintptr_t)o & 15u) == 0) {
                // the lane's groups are contiguous: 16-byte stores of 8 D values each
#pragma unroll
                for (int c = 0; c < kWaveMaxGroups / 8; ++c)
                    if ((uint32_t)(8 * c) < groups)
                        gstore16(o + 8 * c, pack8(dv + 8 * c));
            } else {
#pragma unroll
                for (int g = 0; g < kWaveMaxGroups; ++g)
                    if ((uint32_t)g < groups)
                        gstore(o + g, (int16_t)dv[g]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dot, one wave per item for 16 < K/128 <= 64: as k_dot_wave, with the groups in
// NB blocks of 8 and two register sets -- block b+1's weights and scales load while
// block b computes.  The block loop is unrolled (NB from the batch's largest group
// count) and every load is unconditional (group index clamped), so each wait leaves
// exactly the next block in flight.  Products are added in group order in one
// register per lane; DOT_GROUPS stores each group's D.
// ---------------------------------------------------------------------------
constexpr int kLongBlock = 8;
constexpr int kLongMaxGroups = 64;
constexpr int kLongWaves = 4;

template <int MAP, int NB, bool SCALES>
__global__ __launch_bounds__(64 * kLongWaves) __attribute__((amdgpu_waves_per_eu(4)))
void k_dot_wave_long(const DotJob* __restrict__ jobs, const uint32_t* __restrict__ item_job, uint32_t items,
                     uint32_t uniform_items, uint64_t seq, const uint64_t* __restrict__ flag) {
    constexpr int kChunks = NB * kLongBlock * (int)kPlaneWords / 4 / 64;  // uint4 of planes per lane
    __shared__ uint4 lds_planes[kLongWaves][NB * kLongBlock * kPlaneWords / 4];
    const bool failed = *flag == seq;  // checked before the stores (see k_dot_wave)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t item = xcd_local_block(blockIdx.x, gridDim.x) * kLongWaves + wave;
    if (item >= items)
        return;
    uint32_t job_index = 0xffffffffu;
    DotItem it;
    locate<MAP, 1>(item, DotJob{}, jobs, item_job, uniform_items, it, job_index);
    const uint32_t groups = it.j.groups;
    const uint32_t plane_chunks = groups * (kPlaneWords / 4u);
    const uint4* pl = reinterpret_cast<const uint4*>(it.j.planes + (size_t)it.row * groups * kPlaneWords);
    uint4 p[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
        p[c] = gload(pl + min(lane + 64u * c, plane_chunks - 1u));
    const int sum = gload(it.j.sums + (size_t)it.row * groups + min(lane, groups - 1u));
    const float rs = gload(it.j.rscale + it.row);  // with the row's planes (see k_dot_wave)
    const size_t first = (size_t)it.t0 * groups * kTile + lane;
    uint4 w[2][kLongBlock];
    uint32_t sc[2][kLongBlock];
    auto load_block = [&](int buf, int blk) {
#pragma unroll
        for (int i = 0; i < kLongBlock; ++i) {
            const size_t at = first + (size_t)min((uint32_t)(blk * kLongBlock + i), groups - 1u) * kTile;
            w[buf][i] = gload_stream(it.j.wbits + at);
            sc[buf][i] = SCALES ? gload_stream(it.j.wscale + at) : 0u;  // see k_dot_wave
        }
    };
    load_block(0, 0);
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
        lds_planes[wave][lane + 64u * c] = p[c];
    __builtin_amdgcn_wave_barrier();
    const uint4* lp = lds_planes[wave];
    const uint32_t n0 = it.t0 * kTile;
    const bool live = n0 + lane < it.j.n;
    unsigned char* orow = it.j.out + (size_t)it.row * it.j.out_stride;
    const bool sum_mode = SCALES && it.j.mode != MODE_DOT_I16;
    const bool store = live && !failed;
    int16_t* od = reinterpret_cast<int16_t*>(orow) + (size_t)(n0 + lane) * groups;
    float acc = 0.0f;
    // DOT_GROUPS: a block's 8 D values are one 16-byte store when the lane's row is aligned
    const bool packed = groups % 8u == 0 && ((uintptr_t)od & 15u) == 0;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
        if (blk + 1 < NB)
            load_block((blk + 1) & 1, blk + 1);
        int dv[kLongBlock];
#pragma unroll
        for (int i = 0; i < kLongBlock; ++i) {
            const uint32_t g = blk * kLongBlock + i;
            dv[i] = 0;
            if (g < groups) {
                const int d = group_dot_v(w[blk & 1][i], lp + g * (kPlaneWords / 4), -__shfl(sum, g));
                dv[i] = d;
                if (sum_mode)
                    acc = acc + __half2float(__ushort_as_half((uint16_t)sc[blk & 1][i])) * (float)d;
                else if (store && !packed)
                    gstore(od + g, (int16_t)d);
            }
        }
        if (!sum_mode && store && packed && (uint32_t)(blk * kLongBlock) < groups)
            gstore16(od + blk * kLongBlock, pack8(dv));
    }
    if (sum_mode) {
        if (it.j.mode == MODE_SUM_SCALED)
            acc = acc * rs;
        if (store)
            gstore_stream(reinterpret_cast<float*>(orow) + n0 + lane, acc);
    }
}

template <int MAP, bool SCALES>
hipError_t launch_dot_long(hipStream_t stream, const DotJob* jobs, const uint32_t* item_job, uint32_t items,
                           uint32_t uniform_items, uint32_t max_groups, uint64_t seq, const uint64_t* flag) {
    const uint32_t grid = (items + kLongWaves - 1u) / kLongWaves;
    const dim3 block(64 * kLongWaves);
    switch ((max_groups + kLongBlock - 1u) / kLongBlock) {
    case 3: launch_kernel((k_dot_wave_long<MAP, 3, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    case 4: launch_kernel((k_dot_wave_long<MAP, 4, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    case 5: launch_kernel((k_dot_wave_long<MAP, 5, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    case 6: launch_kernel((k_dot_wave_long<MAP, 6, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    case 7: launch_kernel((k_dot_wave_long<MAP, 7, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    default: launch_kernel((k_dot_wave_long<MAP, 8, SCALES>), dim3(grid), block, 0, stream, jobs, item_job, items, uniform_items, seq, flag); break;
    }
    return hipGetLastError();
}

template <int MAP, bool SCALES>
void launch_dot_wave(hipStream_t stream, const DotJob* jobs, const uint32_t* item_job, uint32_t items,
                     uint32_t uniform_items, uint64_t seq, const uint64_t* flag) {
    const uint32_t grid = (items + BNN_DOT_WAVE_WG_WAVES - 1u) / BNN_DOT_WAVE_WG_WAVES;
    launch_kernel((k_dot_wave<MAP, SCALES>), dim3(grid), dim3(64 * BNN_DOT_WAVE_WG_WAVES), 0, stream, jobs,
                  item_job, items, uniform_items, seq, flag);
}

template <int MAXG, int MAP, int TPI>
hipError_t launch_dot_t(hipStream_t stream, const DotJob& single, const DotJob* jobs, const uint32_t* item_job,
                        uint32_t items, uint32_t uniform_items, uint32_t grid, uint64_t seq, const uint64_t* flag) {
    launch_kernel((k_dot<MAXG, MAP, TPI, BNN_DOT_PREFETCH != 0>), dim3(grid), dim3(64 * kDotWaves), 0, stream,
                       single, jobs, item_job, items, uniform_items, seq, flag);
    return hipGetLastError();
}

// Copies tight staged rows into an arbitrarily aligned / strided view,
// touching only the logical bytes of each row.
__global__ __launch_bounds__(256) void k_scatter(const unsigned char* __restrict__ src, size_t src_stride,
                                                 unsigned char* __restrict__ dst, size_t dst_stride,
                                                 size_t row_bytes, uint64_t seq, const uint64_t* __restrict__ flag) {
    if (*flag == seq)
        return;
    const uint32_t m = blockIdx.y;
    const unsigned char* s = src + (size_t)m * src_stride;
    unsigned char* d = dst + (size_t)m * dst_stride;
    for (size_t i = (size_t)blockIdx.x * 256u + threadIdx.x; i < row_bytes; i += (size_t)gridDim.x * 256u)
        d[i] = s[i];
}

// Instantiations by (threads per row, values per thread): K <= NT * PER.
template <bool BATCH, int NT>
hipError_t launch_prep_nt(hipStream_t stream, uint32_t blocks, uint32_t max_k, const PrepJob& single,
                          const PrepJob* jobs, const uint32_t* block_job, int validate_only, uint64_t seq,
                          uint64_t* flag, uint64_t* host_status) {
    constexpr int kMaxPer = (int)kMaxFeatures / NT;
    const uint32_t per = (max_k + NT - 1u) / NT;
    if (per <= (uint32_t)kMaxPer / 4u)
        launch_kernel((k_prep<BATCH, NT, kMaxPer / 4>), dim3(blocks), dim3(NT), 0, stream, single, jobs,
                           block_job, validate_only, seq, flag, host_status);
    else if (per <= (uint32_t)kMaxPer / 2u)
        launch_kernel((k_prep<BATCH, NT, kMaxPer / 2>), dim3(blocks), dim3(NT), 0, stream, single, jobs,
                           block_job, validate_only, seq, flag, host_status);
    else
        launch_kernel((k_prep<BATCH, NT, kMaxPer>), dim3(blocks), dim3(NT), 0, stream, single, jobs,
                           block_job, validate_only, seq, flag, host_status);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_prep(hipStream_t stream, const PrepJob& job, bool validate_only, uint64_t seq, uint64_t* flag,
                       uint64_t* host_status) {
    if (job.rows >= kPrepManyRows)
        return launch_prep_nt<false, kPrepThreadsMany>(stream, job.rows, job.k, job, nullptr, nullptr,
                                                       (int)validate_only, seq, flag, host_status);
    return launch_prep_nt<false, kPrepThreadsFew>(stream, job.rows, job.k, job, nullptr, nullptr,
                                                  (int)validate_only, seq, flag, host_status);
}

hipError_t launch_prep_batch(hipStream_t stream, const PrepJob* jobs, const uint32_t* block_job, uint32_t blocks,
                             uint32_t max_groups, uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    const PrepJob none = {};
    const uint32_t max_k = max_groups * kGroup;
    if (blocks >= kPrepManyRows)
        return launch_prep_nt<true, kPrepThreadsMany>(stream, blocks, max_k, none, jobs, block_job, 0, seq, flag,
                                                      host_status);
    return launch_prep_nt<true, kPrepThreadsFew>(stream, blocks, max_k, none, jobs, block_job, 0, seq, flag,
                                                 host_status);
}

uint32_t dot_tiles_per_item(uint32_t max_groups) { return max_groups <= 16u ? BNN_DOT_TPI_SMALL : 1u; }

uint32_t dot_items(uint32_t tiles, uint32_t rows, uint32_t max_groups) {
    const uint32_t tpi = dot_tiles_per_item(max_groups);
    return rows * ((tiles + tpi - 1u) / tpi);
}

static uint32_t dot_grid(uint32_t items, uint32_t max_groups, uint32_t cu_count) {
    const uint32_t per_cu = max_groups <= 16u ? kDotWgsPerCuSmall : kDotWgsPerCuLarge;
    const uint32_t cap = (cu_count ? cu_count : 256u) * per_cu;
    return items < cap ? items : cap;
}

hipError_t launch_dot(hipStream_t stream, const DotJob& job, uint32_t cu_count, uint64_t seq,
                      const uint64_t* flag) {
    const uint32_t items = dot_items(job.tiles, job.rows, job.groups);
    const uint32_t grid = dot_grid(items, job.groups, cu_count);
    if (job.groups <= 16u)
        return launch_dot_t<16, MAP_SINGLE, BNN_DOT_TPI_SMALL>(stream, job, nullptr, nullptr, items, 0, grid, seq,
                                                               flag);
    return launch_dot_t<64, MAP_SINGLE, 1>(stream, job, nullptr, nullptr, items, 0, grid, seq, flag);
}

hipError_t launch_dot_batch(hipStream_t stream, const DotJob* jobs, const uint32_t* item_job, uint32_t items,
                            uint32_t uniform_items, uint32_t max_groups, bool scales, uint32_t cu_count, uint64_t seq,
                            const uint64_t* flag) {
    DotJob none = {};
    // One wave per item streams best when the items fill the chip several times;
    // a small batch is latency-bound, and the group-split kernel (4 waves per item)
    // finishes each item sooner.
    const bool many = (uint64_t)items >= (uint64_t)(cu_count ? cu_count : 256u) * BNN_DOT_WAVE_MIN_ITEMS_PER_CU;
    if (BNN_DOT_WAVE_ITEMS && max_groups <= (uint32_t)kWaveMaxGroups && many) {
        if (uniform_items && scales)
            launch_dot_wave<MAP_UNIFORM, true>(stream, jobs, item_job, items, uniform_items, seq, flag);
        else if (uniform_items)
            launch_dot_wave<MAP_UNIFORM, false>(stream, jobs, item_job, items, uniform_items, seq, flag);
        else if (scales)
            launch_dot_wave<MAP_TABLE, true>(stream, jobs, item_job, items, 0u, seq, flag);
        else
            launch_dot_wave<MAP_TABLE, false>(stream, jobs, item_job, items, 0u, seq, flag);
        return hipGetLastError();
    }
#if BNN_DOT_WAVE_LONG
    if (BNN_DOT_WAVE_ITEMS && max_groups <= (uint32_t)kLongMaxGroups && many) {
        if (uniform_items)
            return scales ? launch_dot_long<MAP_UNIFORM, true>(stream, jobs, item_job, items, uniform_items,
                                                               max_groups, seq, flag)
                          : launch_dot_long<MAP_UNIFORM, false>(stream, jobs, item_job, items, uniform_items,
                                                                max_groups, seq, flag);
        return scales ? launch_dot_long<MAP_TABLE, true>(stream, jobs, item_job, items, 0u, max_groups, seq, flag)
                      : launch_dot_long<MAP_TABLE, false>(stream, jobs, item_job, items, 0u, max_groups, seq, flag);
    }
#endif
    const uint32_t grid = dot_grid(items, max_groups, cu_count);
    if (max_groups <= 16u)
        return uniform_items ? launch_dot_t<16, MAP_UNIFORM, BNN_DOT_TPI_SMALL>(stream, none, jobs, item_job, items,
                                                                               uniform_items, grid, seq, flag)
                             : launch_dot_t<16, MAP_TABLE, BNN_DOT_TPI_SMALL>(stream, none, jobs, item_job, items, 0,
                                                                             grid, seq, flag);
    return uniform_items
               ? launch_dot_t<64, MAP_UNIFORM, 1>(stream, none, jobs, item_job, items, uniform_items, grid, seq, flag)
               : launch_dot_t<64, MAP_TABLE, 1>(stream, none, jobs, item_job, items, 0, grid, seq, flag);
}

hipError_t launch_scatter(hipStream_t stream, const unsigned char* src, size_t src_stride, unsigned char* dst,
                          size_t dst_stride, size_t row_bytes, uint32_t rows, uint64_t seq, const uint64_t* flag) {
    size_t blocks = (row_bytes + 255u) / 256u;
    if (blocks > 1024u)
        blocks = 1024u;
    launch_kernel(k_scatter, dim3((uint32_t)blocks, rows), dim3(256), 0, stream, src, src_stride, dst,
                       dst_stride, row_bytes, seq, flag);
    return hipGetLastError();
}

}  // namespace bnnhip
