// Fused batches (BNNX_BatchCreateFused): GEMV_F32 jobs that share one input row,
// with the row produced on the device by a pre-operation and quantised inside the
// one kernel launch that also computes the dots.
//
// Workgroups of 16 waves; each produces the row once and then takes every
// grid-th 64-feature tile of the batch's jobs.  Each workgroup
//   1. issues the loads of its first tile's sign bits and scales (wave w: groups
//      w, w+16, ...), which arrive while it
//   2. produces the whole input row (in registers) -- the pre-operation in the reference
//      engine's operation order (bnn-sw-v2/qwen3/qwen3.c:342-353 for RMSNorm with the
//      residual add of :497-498/:510-511 folded in, :491-495 for SiLU(gate)*up) --
//      and checks it like the GEMV_F32 input check (soft-bnn-accelerator.c:278-308);
//   3. quantises it exactly as the prep kernel does (absmax scale, round half away,
//      bit planes and group sums), each wave the groups of its own dots;
//   4. per tile computes D per group (bit-plane dots), the rounded products
//      F32(scale)*D, and adds them in group order (one lane per feature), times
//      the row scale, with the next tiles' weights already loading (a register ring
//      of three tiles for K <= 2048, two above).
// Every workgroup produces the same row from the same inputs, so all of them take
// the same decisions; workgroup 0 alone stores the pre-operation's residual sum.
// With the post-operation SILU_MUL the tiles are half-tiles of job pairs (32 features
// of each job of the pair, the same indices), and each also stores SiLU(y_a) * y_b.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "bnn_bitplane.h"
#include "bnn_internal.h"

#define BNNE_EXPF_QUALIFIER static __device__ __forceinline__
#include "libc_expf.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

__constant__ uint64_t kFusedExp2Table[32] = BNNE_EXP2_TABLE;

// The expf table into LDS for per-lane lookups (called by one whole wave): scalar loads,
// whose wait (lgkmcnt) leaves the wave's vector loads in flight -- a vector load of the
// table would complete in order behind the row operands and the weights already requested
template <int I>
__device__ __forceinline__ void fused_exp_table_fill_lanes(uint32_t& lo, uint32_t& hi) {
    const uint64_t e = kFusedExp2Table[I];  // uniform address: a scalar load
    asm("v_writelane_b32 %0, %1, %2" : "+v"(lo) : "s"((uint32_t)e), "n"(I));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(hi) : "s"((uint32_t)(e >> 32)), "n"(I));
    if constexpr (I < 31)
        fused_exp_table_fill_lanes<I + 1>(lo, hi);
}
__device__ __forceinline__ void fused_exp_table_fill(uint64_t* tab, uint32_t lane) {
    uint32_t lo = 0, hi = 0;
    fused_exp_table_fill_lanes<0>(lo, hi);
    if (lane < 32u)
        tab[lane] = (uint64_t)hi << 32 | lo;
}

extern "C" __device__ uint32_t __ockl_wfred_max_u32(uint32_t);
extern "C" __device__ double __ockl_wfred_add_f64(double);
extern "C" __device__ int __ockl_wfred_add_i32(int);

// Bit planes B..7 of the wave's 64 quantised values q: lane 2b of `word` receives
// the low and lane 2b + 1 the high half of plane b's mask (put_plane_mask), and `sum`
// accumulates sum(q) from the same masks.
template <int B>
__device__ __forceinline__ void plane_words(int q, uint32_t& word, int& sum) {
    const unsigned long long mask = __ballot(plane_bit(q, B));
    const int cnt = __popcll(mask);
    sum += B == 7 ? -(cnt << 7) : (cnt << B);
    put_plane_mask<B>(mask, word);
    if constexpr (B < 7)
        plane_words<B + 1>(q, word, sum);
}


// The sum of the squares in index order, s_{i+1} = F32(s_i + t_i) from s_0 = +0,
// evaluated in segments of kSegment terms.  Segment j is run from kWindow candidate
// starts at once (one lane each): the binary32 values whose bit patterns lie around
// that of F32(E_j), E_j the sum of the earlier terms in binary64.  Afterwards one
// wave walks the segments in order: when the running sum is one of segment j's
// candidates, the lane that started from exactly that value has performed the same
// additions from the same value, and its end value is taken; otherwise the segment
// is added term by term.  Either way the result is bit-identical to the sequential
// loop; the walk costs one table lookup per segment in the usual case, where the
// accumulated rounding of the sequential sum stays within +-16 ulps of E_j.
constexpr uint32_t kSegment = 128;
constexpr uint32_t kWindow = 32;
constexpr uint32_t kChunk = 64;  // terms per binary64 partial sum (one wave's)

// s plus the n terms at p, one rounding per addition, in index order (n % 16 == 0)
__device__ __forceinline__ float add_in_order_lds(const float* p, uint32_t n, float s) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll 1
    for (uint32_t i = 0; i < n / 4u; i += 4u) {
        float4 v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
            v[c] = p4[i + c];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s = s + v[c].x;
            s = s + v[c].y;
            s = s + v[c].z;
            s = s + v[c].w;
        }
    }
    return s;
}

// NC interleaved candidate chains of one wave over kSegment terms each
template <int NC>
__device__ __forceinline__ void run_chains(float (&c)[NC], const float4* const (&src)[NC]) {
#pragma unroll 2
    for (uint32_t i = 0; i < kSegment / 4u; i += 8u) {
        float4 v[NC][8];
#pragma unroll
        for (int r = 0; r < NC; ++r)
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v[r][q] = src[r][i + q];
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int r = 0; r < NC; ++r) {
                c[r] = c[r] + v[r][q].x;
                c[r] = c[r] + v[r][q].y;
                c[r] = c[r] + v[r][q].z;
                c[r] = c[r] + v[r][q].w;
            }
    }
}


// System-coherent stores (write-through to memory: sc0 sc1) for the results of a single job,
// so that once they are complete (vmcnt) the host can read them without an L2 writeback
__device__ __forceinline__ void store_sys(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_sys(int16_t* p, uint32_t v) {
    asm volatile("global_store_short %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_sys(int16_t* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ void fused_raise(uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    __hip_atomic_store(flag, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(host_status, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr uint32_t kFusedThreads = 1024;
constexpr uint32_t kFusedWaves = kFusedThreads / 64;
constexpr uint32_t kFusedMaxGroups = kFusedMaxWidth / kGroup;
constexpr uint32_t kFusedPad = 32;  // spare floats after the row (16-byte aligned product buffers)

// The tile's weights for one lane: wave w holds groups w, w+16, ... (clamped).
template <int GPW>
struct TileRegs {
    uint4 w[GPW];
    uint32_t s[GPW];
};

// The job table, written by the host only: read through the constant address space
// (scalar loads through the scalar cache).  Up to kFusedInline jobs (a single job of
// BNN_Execute, SINGLE, or a decode step's small batches) also come in the kernel
// arguments, loaded with them at the start: the first tile's job is taken from there, so
// its weights are requested without first waiting for a table read (or the dependent
// reads of a walk); later tiles (prefetches) read the table.
// A kernel-argument value as an opaque scalar register: the compiler then keeps it as a
// value loaded with the other arguments at the start, and a uniform choice among such
// values stays a choice of values (left to itself it turns a choice among argument
// fields into a choice of address and loads the field afterwards, one dependent round
// of scalar loads per choice).
__device__ __forceinline__ uint32_t sreg(uint32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}
template <class T>
__device__ __forceinline__ T* sreg(T* p) {
    uint64_t x = (uint64_t)p;
    asm volatile("" : "+s"(x));
    return (T*)x;
}

// slot i of three, as a choice of values (uniform i)
template <class T>
__device__ __forceinline__ T pick3(uint32_t i, T a, T b, T c) {
    a = sreg(a);
    b = sreg(b);
    c = sreg(c);
    return i == 0u ? a : i == 1u ? b : c;
}

template <bool SINGLE>
struct JobTable {
    const FusedArgs& fa;
    typedef const __attribute__((address_space(4))) FusedJob* Ptr;
    static_assert(kFusedInline == 3, "the inline selections name three slots");
    // the inline slots, every field read at the start (SINGLE: the one job)
    FusedJob slot[kFusedInline];
    __device__ __forceinline__ static FusedJob held(const FusedJob& s) {
        FusedJob j;
        j.wbits = sreg(s.wbits);
        j.wscale = sreg(s.wscale);
        j.out = sreg(s.out);
        j.n = sreg(s.n);
        j.tiles = sreg(s.tiles);
        j.first_tile = sreg(s.first_tile);
        j.post_off = sreg(s.post_off);
        return j;
    }
    __device__ __forceinline__ explicit JobTable(const FusedArgs& f) : fa(f) {
        slot[0] = held(f.inl[0]);
        if constexpr (!SINGLE) {
            slot[1] = held(f.inl[1]);
            slot[2] = held(f.inl[2]);
        }
    }
    __device__ __forceinline__ uint32_t first_tile(uint32_t i) const {
        if constexpr (SINGLE)
            return slot[0].first_tile;
        else
            return ((Ptr)fa.jobs)[i].first_tile;
    }
    // the job (or pair) of a workgroup's first tile t, and that job
    __device__ __forceinline__ uint32_t first_job_of(uint32_t t, uint32_t nwalk) const {
        if (SINGLE || nwalk == 1u)
            return 0;
        if (fa.inline_jobs)
            return t >= slot[2].first_tile && nwalk > 2u ? 2u : t >= slot[1].first_tile ? 1u : 0u;
        if (fa.walk_shift < 32u)
            return min(t >> fa.walk_shift, nwalk - 1u);
        uint32_t from = 0;
        while (from + 1u < nwalk && first_tile(from + 1u) <= t)
            ++from;
        return from;
    }
    __device__ __forceinline__ FusedJob first(uint32_t i) const {
        if constexpr (SINGLE)
            return slot[0];
        if (fa.inline_jobs) {
            FusedJob j;
            j.wbits = pick3(i, slot[0].wbits, slot[1].wbits, slot[2].wbits);
            j.wscale = pick3(i, slot[0].wscale, slot[1].wscale, slot[2].wscale);
            j.out = pick3(i, slot[0].out, slot[1].out, slot[2].out);
            j.n = pick3(i, slot[0].n, slot[1].n, slot[2].n);
            j.tiles = pick3(i, slot[0].tiles, slot[1].tiles, slot[2].tiles);
            j.first_tile = pick3(i, slot[0].first_tile, slot[1].first_tile, slot[2].first_tile);
            j.post_off = pick3(i, slot[0].post_off, slot[1].post_off, slot[2].post_off);
            return j;
        }
        return (*this)[i];
    }
    __device__ __forceinline__ FusedJob operator[](uint32_t i) const {
        if constexpr (SINGLE)
            return slot[0];
        const Ptr c = (Ptr)fa.jobs;
        FusedJob j;
        j.wbits = c[i].wbits;
        j.wscale = c[i].wscale;
        j.out = c[i].out;
        j.n = c[i].n;
        j.tiles = c[i].tiles;
        j.first_tile = c[i].first_tile;
        j.post_off = c[i].post_off;
        return j;
    }
};

// The lane's row of a tile: feature `lane` of 64-feature tile `tile` of `job`, or for
// paired batches (POST_SILU_MUL) half-tile `tile` of the pair (ja, jb): feature
// 32 (tile % 2) + lane % 32 of 64-feature tile tile / 2, of ja in lanes 0..31 and of jb
// in lanes 32..63.
struct LaneRow {
    const uint4* wbits;
    const uint16_t* wscale;
    size_t base;   // the lane's offset in tile units of kTile (group 0)
    uint32_t row;  // feature index within the job
};
// a and b as opaque scalar-register values: a per-lane choice between fields of two
// descriptors would otherwise become a choice of descriptor address (on the stack)
template <class T>
__device__ __forceinline__ T lane_pick(bool second, T a, T b) {
    uint64_t x = (uint64_t)a, y = (uint64_t)b;
    asm volatile("" : "+s"(x), "+s"(y));
    return (T)(second ? y : x);
}

__device__ __forceinline__ LaneRow lane_row(const FusedJob& ja, const FusedJob& jb, bool paired, uint32_t tile,
                                            uint32_t G, uint32_t lane) {
    LaneRow lr;
    if (paired) {
        const bool second = lane >= 32u;
        lr.wbits = lane_pick(second, ja.wbits, jb.wbits);
        lr.wscale = lane_pick(second, ja.wscale, jb.wscale);
        lr.row = (tile >> 1) * kTile + 32u * (tile & 1u) + (lane & 31u);
        lr.base = (size_t)(tile >> 1) * G * kTile + 32u * (tile & 1u) + (lane & 31u);
    } else {
        lr.wbits = ja.wbits;
        lr.wscale = ja.wscale;
        lr.row = tile * kTile + lane;
        lr.base = (size_t)tile * G * kTile + lane;
    }
    return lr;
}

template <int GPW>
__device__ __forceinline__ void load_tile(const LaneRow& lr, uint32_t G, uint32_t wave, TileRegs<GPW>& r) {
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
        const uint32_t g = min(wave + kFusedWaves * i, G - 1u);
        r.w[i] = gload(lr.wbits + lr.base + (size_t)g * kTile);
        r.s[i] = gload(lr.wscale + lr.base + (size_t)g * kTile);
    }
}

// GPW: groups per wave of a tile's dots; EPT: row elements per thread.  Workgroup
// b produces the row once and then takes tiles b, b + grid, ... of the batch, the
// next tile's weights loading while the current one is computed.
// SINGLE: one job in the kernel arguments (BNN_Execute): its row may be int8, its output
// DOT_GROUPS' D or mirrored into host memory.  Batches compile without those branches.
// RING: tiles of weights in flight per workgroup -- 1 when every workgroup has one tile
// (no prefetch), 2 or 3 when workgroups walk several tiles.
template <int GPW, int EPT, bool PAIRED, bool SINGLE, int RING>
__device__ __forceinline__ void fused_body(const FusedArgs& fa, uint32_t tiles_total, uint64_t seq, uint64_t* flag,
                                           uint64_t* host_status) {
    static_assert(EPT == 2 * GPW, "a wave quantises exactly the groups of its dots");
    __shared__ float4 scratch4[(kFusedMaxWidth + kFusedPad) / 4];  // squares, then products [2][group][64]
    // bit planes of the groups (GPW > 1; one group per wave keeps them in scalar registers),
    // each written and read by the wave that owns the group
    __shared__ uint4 planes[GPW > 1 ? kFusedMaxGroups * kPlaneWords / 4 : 1];
    __shared__ uint32_t amax_w[kFusedWaves];
    __shared__ uint64_t exp_tab[32];
    __shared__ float rms_s;
    // the speculative sum of squares: binary64 sums of 64 terms, the candidates' end
    // values (segments 2p and 2p + 1 in the two halves of row p), the segments' first
    // candidate bit pattern
    constexpr uint32_t kRowMax = EPT * kFusedThreads;
    constexpr uint32_t kPairs = kRowMax / kSegment / 2u;
    __shared__ double chunk_sum[kRowMax / kChunk];
    __shared__ float seg_end[kPairs * 64u];
    __shared__ float seg_comp[kPairs * 32u];  // pair p's two segments composed, per candidate of segment 2p
    __shared__ int seg_base[kPairs * 2u];
    float* scratch = reinterpret_cast<float*>(scratch4);

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = fa.width, G = K / kGroup;
    // the row's operands, read with the job slots in the first round of argument loads
    const int32_t kind = (int32_t)sreg((uint32_t)fa.kind);
    const float* const row_a = sreg(fa.kind == PRE_ROW ? fa.row : fa.a);
    const float* const row_b = sreg(fa.b);
    const float* const row_gain = sreg(fa.gain);

    // row element i of a thread: half i % 2 of group w + 16 (i / 2), w its wave -- the
    // groups of the wave's dots (whole waves: K % 128 == 0)
    const auto elem = [&](int i) { return (wave + kFusedWaves * (uint32_t)(i >> 1)) * kGroup + 64u * (i & 1) + lane; };
    const auto live = [&](int i) { return wave + kFusedWaves * (uint32_t)(i >> 1) < G; };

    // 1. the row operands load first and the first tile's weights after them (the
    // load counter completes in order: the row is needed first), arriving while the
    // row is produced
    // tiles are walked over the jobs, or over the pairs (the first half of the table)
    const JobTable<SINGLE> jobs(fa);
    constexpr bool paired = PAIRED;  // fa.post == POST_SILU_MUL
    const uint32_t nwalk = paired ? fa.njobs / 2u : fa.njobs, pair_step = paired ? nwalk : 0u;
    // the job (or pair) of tile t: first tiles at multiples of 2^walk_shift give it in one
    // step, else a walk from a job at or before it
    const auto job_of = [&](uint32_t t, uint32_t from) -> uint32_t {
        if (fa.walk_shift < 32u)
            return min(t >> fa.walk_shift, nwalk - 1u);
        while (from + 1u < nwalk && jobs.first_tile(from + 1u) <= t)
            ++from;
        return from;
    };
    uint32_t tile = blockIdx.x, ji = jobs.first_job_of(tile, nwalk);
    FusedJob job = jobs.first(ji), job2 = jobs.first(ji + pair_step);
    const bool int_row = SINGLE && kind == PRE_ROW_I8;
    const bool dot_out = SINGLE && fa.dot_out;
    float* const mirror = SINGLE ? fa.mirror : nullptr;
    float xv[EPT], bv[EPT], gv[EPT];
    if (int_row) {  // int8 values, exact in binary32
        const int8_t* src8 = reinterpret_cast<const int8_t*>(fa.row);
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            xv[i] = (float)(int)*(const __attribute__((address_space(1))) int8_t*)(src8 + min(elem(i), K - 1u));
    } else {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            xv[i] = gload(row_a + min(elem(i), K - 1u));
    }
    if (row_b) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            bv[i] = gload(row_b + min(elem(i), K - 1u));
    }
    if (kind == PRE_RMSNORM) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            gv[i] = gload(row_gain + min(elem(i), K - 1u));
    }
    // a ring of RING tiles' weights in flight: a workgroup that walks several tiles (the
    // lm_head's 2370 over one workgroup per CU) would otherwise wait one memory latency per tile
    constexpr int kRing = RING;
    TileRegs<GPW> ring[kRing];
    LaneRow lr = lane_row(job, job2, paired, tile - job.first_tile, G, lane);
    load_tile<GPW>(lr, G, wave, ring[0]);
    // the prefetch cursor: the last tile whose weights were requested, and its job.  Past
    // the workgroup's last tile the cursor's tile is loaded again (an L2 hit, never used):
    // with the same number of loads on every path the compiler's wait for a slot leaves
    // the later slots' loads in flight (a skipped load would make it wait for all)
    uint32_t pf_tile = tile, pf_ji = ji;
    const auto prefetch = [&](TileRegs<GPW>& r) {
        const uint32_t t = pf_tile + gridDim.x;
        if (t < tiles_total) {
            pf_tile = t;
            pf_ji = job_of(t, pf_ji);
        }
        const FusedJob pj = jobs[pf_ji], pj2 = jobs[pf_ji + pair_step];
        load_tile<GPW>(lane_row(pj, pj2, paired, pf_tile - pj.first_tile, G, lane), G, wave, r);
    };
#pragma unroll
    for (int r = 1; r < kRing; ++r)
        prefetch(ring[r]);
    // the expf table of a SiLU (the post-operation's, read after the first product
    // barrier, or the pre-operation's, published by the barrier below), by the last wave
    if ((paired || fa.kind == PRE_SILU_MUL) && wave == kFusedWaves - 1u)
        fused_exp_table_fill(exp_tab, lane);

    // 2. the input row
    if (fa.kind == PRE_RMSNORM) {
        if (fa.b) {
#pragma unroll
            for (int i = 0; i < EPT; ++i)
                xv[i] = xv[i] + bv[i];
        }
        // the terms, and their binary64 sums per 64 (chunk k / 64)
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const uint32_t k = elem(i);
            const float sq = xv[i] * xv[i];
            if (live(i)) {
                scratch[k] = sq;
                if (fa.a_out && blockIdx.x == 0)
                    gstore(fa.a_out + k, xv[i]);
                const double h = __ockl_wfred_add_f64((double)sq);
                if (lane == 0)
                    chunk_sum[k / kChunk] = h;
            }
        }
        lds_barrier();
        // candidate chains: wave w runs pairs w, w + 16, ... (segments 2p, 2p + 1)
        const uint32_t nseg = K / kSegment, npairs = (nseg + 1u) / 2u;
        const uint32_t half = lane >> 5, cand = lane & (kWindow - 1u);
        constexpr int kPairsPerWave = (kPairs + kFusedWaves - 1) / kFusedWaves;
        float c[kPairsPerWave];
        int bs[kPairsPerWave];
        const float4* src[kPairsPerWave];
#pragma unroll
        for (int r = 0; r < kPairsPerWave; ++r) {
            const uint32_t p = min(wave + kFusedWaves * r, npairs - 1u);
            // E_{2p}: the chunks before segment 2p; E_{2p+1} adds segment 2p's two
            double e = 0.0;
#pragma unroll
            for (uint32_t cc = 0; cc < kRowMax / kChunk; cc += 64u)
                if (cc + lane < 4u * p)
                    e += chunk_sum[cc + lane];
            e = __ockl_wfred_add_f64(e);
            if (half)
                e = e + chunk_sum[4u * p] + chunk_sum[4u * p + 1u];
            const int base = __float_as_int((float)e) - (int)(kWindow / 2u);
            bs[r] = base;
            c[r] = __int_as_float(base + (int)cand);
            const uint32_t j = min(2u * p + half, nseg - 1u);
            src[r] = reinterpret_cast<const float4*>(scratch + kSegment * j);
            if (cand == 0 && wave + kFusedWaves * r < npairs && 2u * p + half < nseg)
                seg_base[2u * p + half] = base;
        }
        if (kPairsPerWave > 1 && wave + kFusedWaves < npairs) {
            run_chains<kPairsPerWave>(c, src);
        } else if (wave < npairs) {
            float c1[1] = {c[0]};
            const float4* const s1[1] = {src[0]};
            run_chains<1>(c1, s1);
            c[0] = c1[0];
        }
        // each pair's two segments composed in its own wave: candidate c of segment 2p ends at
        // a value whose offset in segment 2p + 1's window names the lane that continued from
        // it; an offset outside that window leaves the marker 0xffffffff (no candidate)
#pragma unroll
        for (int r = 0; r < kPairsPerWave; ++r) {
            const uint32_t pr = wave + kFusedWaves * r;
            const uint32_t idx = (uint32_t)__float_as_int(c[r]) - (uint32_t)__builtin_amdgcn_readlane(bs[r], 32);
            const float nxt = __shfl(c[r], (int)(32u + (idx & (kWindow - 1u))));
            const float comp = 2u * pr + 1u >= nseg ? c[r] : idx < kWindow ? nxt : __int_as_float(-1);
            if (pr < npairs) {
                seg_end[pr * 64u + lane] = c[r];
                if (lane < kWindow)
                    seg_comp[pr * kWindow + lane] = comp;
            }
        }
        lds_barrier();
        // the walk (wave 0) over the composed pairs: bits of the running sum, uniform across
        // the wave
        if (wave == 0) {
            float comps[kPairs];
#pragma unroll
            for (uint32_t m = 0; m < kPairs; ++m)
                comps[m] = seg_comp[min(m, npairs - 1u) * kWindow + (lane & (kWindow - 1u))];
            const int bases = seg_base[min(lane, nseg - 1u)];
            // branch-free lookups (a scalar branch per step costs more than the step); an
            // offset outside a window sets a bit above the window's in `any`, a composed miss
            // leaves the marker (caught by the next offset, or at the end), and either repeats
            // the walk below
            uint32_t v = 0, any = 0;
            if (npairs == kPairs) {
#pragma unroll
                for (uint32_t m = 0; m < kPairs; ++m) {
                    const uint32_t idx = v - (uint32_t)__builtin_amdgcn_readlane(bases, 2u * m);
                    any |= idx;
                    v = (uint32_t)__builtin_amdgcn_readlane(__float_as_int(comps[m]), (int)(idx & (kWindow - 1u)));
                }
            } else {
#pragma unroll
                for (uint32_t m = 0; m < kPairs; ++m) {
                    const uint32_t idx = v - (uint32_t)__builtin_amdgcn_readlane(bases, 2u * m);
                    const uint32_t nv =
                        (uint32_t)__builtin_amdgcn_readlane(__float_as_int(comps[m]), (int)(idx & (kWindow - 1u)));
                    const bool live = m < npairs;
                    any |= live ? idx : 0u;
                    v = live ? nv : v;
                }
            }
            const uint32_t miss = (any & ~(kWindow - 1u)) | (uint32_t)(v == 0xffffffffu);
            if (miss) {  // the walk with term-by-term additions where the running sum is no candidate
                v = 0;
                for (uint32_t j = 0; j < nseg; ++j) {
                    const uint32_t idx = v - (uint32_t)seg_base[j];
                    if (idx < kWindow)
                        v = __float_as_uint(seg_end[(j / 2u) * 64u + (j & 1u) * 32u + idx]);
                    else
                        v = __float_as_uint(add_in_order_lds(scratch + kSegment * j, kSegment, __uint_as_float(v)));
                }
            }
            if (lane == 0)
                rms_s = sqrtf(__uint_as_float(v) / (float)K + fa.eps);
        }
        lds_barrier();
        const float rms = rms_s;
        if (!__builtin_isfinite(rms) || rms == 0.0f) {
            if (tid == 0) {
                if (fa.err)
                    atomicCAS(fa.err, 0, fa.err_code);
                fused_raise(seq, flag, host_status);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            xv[i] = xv[i] / rms * gv[i];
    } else if (fa.kind == PRE_SILU_MUL) {
        lds_barrier();  // the expf table in LDS (its lookups are per-lane gathers)
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const float silu = xv[i] / (1.0f + bnne_expf_libc(-xv[i], exp_tab));
            xv[i] = silu * bv[i];
        }
    }

    // 3. the input check and the row scale, in one exchange: a wave with an illegal
    // value (non-finite; -128 in an int8 row: soft-bnn-accelerator.c:278-308) posts the
    // all-ones word (above every finite |x| bit pattern)
    uint32_t abits = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        if (live(i)) {
            const uint32_t a = __float_as_uint(xv[i]) & 0x7fffffffu;
            const bool bad = int_row ? xv[i] == -128.0f : a >= 0x7f800000u;
            abits = max(abits, bad ? 0xffffffffu : a);
        }
    }
    abits = __ockl_wfred_max_u32(abits);
    if (lane == 0)
        amax_w[wave] = abits;
    lds_barrier();
    abits = amax_w[0];
#pragma unroll
    for (uint32_t w = 1; w < kFusedWaves; ++w)
        abits = max(abits, amax_w[w]);
    if (abits == 0xffffffffu) {
        if (tid == 0)
            fused_raise(seq, flag, host_status);
        return;
    }
    float amax = __uint_as_float(abits);
    float s = 1.0f;
    if (!int_row)
        s = quant_row_scale(amax);

    // 4. quantise the wave's own groups; their bit planes are ballots (wave-uniform
    // masks: kept in scalar registers for one group per wave or, with one tile per
    // workgroup, formed group by group next to that group's dots; else in LDS), and
    // -sum(Q) per group; no exchange between waves
    const float rcp = quant_rcp(s);
    const bool exact = quant_exact(s);  // 1 / s may overflow
    int q[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i)
        q[i] = !live(i) ? 0 : int_row ? (int)xv[i] : quantize_rcp(xv[i], s, rcp, exact);
    uint64_t masks[2][8];  // GPW == 1: the planes of group `wave`
    int neg_sum[GPW];
    if constexpr (GPW == 1) {
        // -sum(Q) as a wave reduction (the 16 waves' scalar popcount chains would share one
        // scalar unit)
        neg_sum[0] = -__ockl_wfred_add_i32(q[0] + q[1]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < 8; ++b)
                masks[h][b] = __ballot(plane_bit(q[h], b));
    } else if constexpr (RING == 1) {
        // the tile's dots form each group's masks themselves (no planes in LDS: the 16 waves'
        // plane words would queue on the CU's one scalar unit); -sum(Q) of two groups per
        // wave reduction, packed: each lane's pair sum lies in [-254, 254], a group's in
        // [-16256, 16256], so S0 + 65536 S1 neither overflows nor mixes the halves
#pragma unroll
        for (int gi = 0; gi < GPW; gi += 2) {
            const int v0 = q[2 * gi] + q[2 * gi + 1];
            if (gi + 1 < GPW) {
                const int v1 = q[2 * gi + 2] + q[2 * gi + 3];
                const int total = __ockl_wfred_add_i32(v0 + v1 * 65536);
                const int s0 = (int)(int16_t)(uint16_t)((uint32_t)total & 0xffffu);
                neg_sum[gi] = -s0;
                neg_sum[gi + 1] = -((total - s0) / 65536);
            } else {
                neg_sum[gi] = -__ockl_wfred_add_i32(v0);
            }
        }
    } else {
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            neg_sum[gi] = 0;
            const uint32_t g = wave + kFusedWaves * gi;
            if (g < G) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint32_t word = 0;
                    int sum = 0;
                    plane_words<0>(q[2 * gi + h], word, sum);
                    neg_sum[gi] -= sum;
                    if (lane < 16u)
                        reinterpret_cast<uint32_t*>(planes)[g * kPlaneWords + (lane >> 1) * 4u + h * 2u + (lane & 1u)] =
                            word;
                }
            }
        }
    }

    // 5. per tile: group dots and the rounded products F32(scale) * D into one of two
    // product buffers, then wave 0 adds them in group order (one lane per feature)
    // and applies the row scale.  One barrier per tile: a buffer is rewritten only
    // two tiles later, after wave 0 has passed the barrier that follows its sums.
    uint32_t buf = 0;
    // one tile: its dots from ring slot `cur`, the slot refilled kRing tiles ahead (with a
    // ring), the in-order sums, then (`more`: another tile follows) the cursor on the next tile
    const auto step = [&](TileRegs<GPW>& cur, bool more) {
        float* prod = scratch + buf * (kFusedMaxGroups * 64u);
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const uint32_t g = wave + kFusedWaves * i;
            if (g < G) {
                int d;
                if constexpr (GPW == 1) {
                    d = group_dot_s(cur.w[i], masks, neg_sum[i]);
                } else if constexpr (RING == 1) {
                    uint64_t m[2][8];
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int b = 0; b < 8; ++b)
                            m[h][b] = __ballot(plane_bit(q[2 * i + h], b));
                    d = group_dot_s(cur.w[i], m, neg_sum[i]);
                    // one group's 32 mask registers at a time (scheduled together, the
                    // groups' masks would not fit the scalar register file)
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    d = group_dot_v(cur.w[i], planes + g * (kPlaneWords / 4u), neg_sum[i]);
                }
                // DOT_GROUPS: D itself goes through the exchange
                prod[g * 64u + lane] = dot_out ? __int_as_float(d)
                                                  : __half2float(__ushort_as_half((uint16_t)cur.s[i])) * (float)d;
            }
        }
        if constexpr (kRing > 1)
            prefetch(cur);
        lds_barrier();
        if (wave == 0 && dot_out) {
            // int16 D[n][g]: a lane's groups are contiguous, 16-byte stores of 8 when aligned
            const uint32_t n = lr.row;
            if (n < job.n) {
                int16_t* o = reinterpret_cast<int16_t*>(job.out) + (size_t)n * G;
                if (G % 8u == 0 && ((uintptr_t)o & 15u) == 0) {
                    for (uint32_t g = 0; g < G; g += 8u) {
                        uint32_t v[8];
#pragma unroll
                        for (int c = 0; c < 8; ++c)
                            v[c] = (uint32_t)__float_as_int(prod[(g + c) * 64u + lane]) & 0xffffu;
                        const u32x4 w = {v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                                         v[6] | (v[7] << 16)};
                        store_sys(o + g, w);
                    }
                } else {
                    for (uint32_t g = 0; g < G; ++g)
                        store_sys(o + g, (uint32_t)__float_as_int(prod[g * 64u + lane]));
                }
            }
        } else if (wave == 0) {
            const uint32_t n = lr.row;
            float acc = 0.0f;
            uint32_t g = 0;
            for (; g + 8u <= G; g += 8u) {
                float v[8];
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    v[c] = prod[(g + c) * 64u + lane];
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    acc = acc + v[c];
            }
            for (; g < G; ++g)
                acc = acc + prod[g * 64u + lane];
            acc = acc * s;
            if (n < job.n) {
                if constexpr (SINGLE) {
                    store_sys(job.out + n, acc);
                    if (mirror)
                        store_sys(mirror + n, acc);
                } else {
                    gstore(lane_pick(paired && lane >= 32u, job.out, job2.out) + n, acc);
                }
            }
            if (paired) {
                // y_p / (1 + expf(-y_p)) * y_(m+p) (qwen3.c:491-495), y_(m+p) from lane + 32
                const float second = __shfl(acc, (int)(lane | 32u));
                if (lane < 32u && n < job.n)
                    gstore(fa.post_out + job.post_off + n, acc / (1.0f + bnne_expf_libc(-acc, exp_tab)) * second);
            }
        }
        if (more) {
            tile += gridDim.x;
            ji = job_of(tile, ji);
            job = jobs[ji];
            job2 = jobs[ji + pair_step];
            lr = lane_row(job, job2, paired, tile - job.first_tile, G, lane);
            buf ^= 1u;
        }
    };
    static_assert(kRing >= 1 && kRing <= 3, "ring slots are named statically");
    if constexpr (kRing == 1) {
        // one tile per workgroup: the host launches this form only with a workgroup per tile
        step(ring[0], false);
    } else {
        // whole rounds of the ring, then the rest: the loop has one exit, so the compiler's
        // waits see the ring's loads in flight on every path into the loop
        const uint32_t mine = (tiles_total - blockIdx.x + gridDim.x - 1u) / gridDim.x;  // grid <= tiles
        uint32_t done = 0;
        for (; done + kRing <= mine; done += kRing) {
            step(ring[0], true);
            step(ring[1], kRing > 2 || done + 2u < mine);
            if constexpr (kRing == 3)
                step(ring[kRing - 1], done + 3u < mine);
        }
        if (done < mine)
            step(ring[0], done + 1u < mine);
        if (done + 1u < mine)
            step(ring[1], false);
    }
}

template <int GPW, int EPT, bool PAIRED, bool SINGLE, int RING>
__global__ __launch_bounds__(kFusedThreads) void k_fused(FusedArgs fa, uint32_t tiles_total, uint64_t seq,
                                                         uint64_t* flag, uint64_t* host_status) {
    fused_body<GPW, EPT, PAIRED, SINGLE, RING>(fa, tiles_total, seq, flag, host_status);
    // Completion signal of a single job, so that the host need not wait for the end of the
    // kernel: in this form every global store (outputs, host mirror, error words) comes from
    // wave 0 and is system-coherent (written through to memory), so once wave 0's stores are
    // complete (vmcnt(0)) its workgroup's results are visible to the host, and it stores seq
    // into its workgroup's own pinned host word (the host waits for all of them).  A
    // system-scope fence per workgroup instead (a writeback of its XCD's whole L2, 96 at
    // once) had cost ~3 us per call, and one device-scope counter shared by the workgroups
    // nothing measurable on top.
    if (SINGLE && fa.done_flags != nullptr && threadIdx.x < 64u) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
        if (threadIdx.x == 0)
            __hip_atomic_store(fa.done_flags + blockIdx.x, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace

namespace {
// one tile per workgroup: no weight ring; several: a ring of three tiles (two for K > 2048)
template <int GPW, int EPT, bool PAIRED, bool SINGLE>
void launch_fused_ring(hipStream_t stream, const FusedArgs& args, uint32_t tiles, uint32_t grid, uint64_t seq,
                       uint64_t* flag, uint64_t* host_status) {
    const dim3 g(grid), b(kFusedThreads);
    if (tiles <= grid)
        launch_kernel((k_fused<GPW, EPT, PAIRED, SINGLE, 1>), g, b, 0, stream, args, tiles, seq, flag, host_status);
    else
        launch_kernel((k_fused<GPW, EPT, PAIRED, SINGLE, GPW == 1 ? 3 : 2>), g, b, 0, stream, args, tiles, seq, flag,
                      host_status);
}
}  // namespace

hipError_t launch_fused(hipStream_t stream, const FusedArgs& args, uint32_t tiles, uint32_t grid, uint64_t seq,
                        uint64_t* flag, uint64_t* host_status) {
    static_assert(kFusedMaxGroups * 64u * 2u <= kFusedMaxWidth, "two product buffers fit the scratch");
    constexpr int kWideGpw = kFusedMaxGroups / kFusedWaves, kWideEpt = kFusedMaxWidth / kFusedThreads;
    const bool paired = args.post == POST_SILU_MUL;
    if (args.jobs == nullptr) {  // a single job in the kernel arguments
        if (args.width <= 2048u)
            launch_fused_ring<1, 2, false, true>(stream, args, tiles, grid, seq, flag, host_status);
        else
            launch_fused_ring<kWideGpw, kWideEpt, false, true>(stream, args, tiles, grid, seq, flag, host_status);
    } else if (args.width <= 2048u && !paired) {
        launch_fused_ring<1, 2, false, false>(stream, args, tiles, grid, seq, flag, host_status);
    } else if (args.width <= 2048u) {
        launch_fused_ring<1, 2, true, false>(stream, args, tiles, grid, seq, flag, host_status);
    } else if (!paired) {
        launch_fused_ring<kWideGpw, kWideEpt, false, false>(stream, args, tiles, grid, seq, flag, host_status);
    } else {
        launch_fused_ring<kWideGpw, kWideEpt, true, false>(stream, args, tiles, grid, seq, flag, host_status);
    }
    return hipGetLastError();
}

}  // namespace bnnhip
