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
//      bit planes and group sums);
//   4. per tile computes D per group (bit-plane dots), the rounded products
//      F32(scale)*D, and adds them in group order (one lane per feature), times
//      the row scale, with the next tile's weights already loading.
// Every workgroup produces the same row from the same inputs, so all of them take
// the same decisions; workgroup 0 alone stores the pre-operation's residual sum.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "bnn_internal.h"

#define BNNE_EXPF_QUALIFIER static __device__ __forceinline__
#include "libc_expf.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

__constant__ uint64_t kFusedExp2Table[32] = BNNE_EXP2_TABLE;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 fload(const uint4* p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t fload(const uint16_t* p) {
    return *(const __attribute__((address_space(1))) uint16_t*)p;
}
__device__ __forceinline__ float fload(const float* p) { return *(const __attribute__((address_space(1))) float*)p; }
__device__ __forceinline__ void fstore(float* p, float v) { *(__attribute__((address_space(1))) float*)p = v; }

extern "C" __device__ uint32_t __ockl_wfred_max_u32(uint32_t);

// popc(x) + acc and (c << SHIFT) + acc as single instructions (the compiler would
// otherwise re-associate the chains)
__device__ __forceinline__ uint32_t f_bcnt_acc(uint32_t x, uint32_t acc) {
    uint32_t r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
    return r;
}
template <int SHIFT>
__device__ __forceinline__ uint32_t f_lshl_add(uint32_t c, uint32_t acc) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, %2, %3" : "=v"(r) : "v"(c), "i"(SHIFT), "v"(acc));
    return r;
}
template <int B>
__device__ __forceinline__ uint32_t f_plane_count(uint4 w, const uint4* p) {
    const uint4 pb = p[B];
    uint32_t c = (uint32_t)__builtin_popcount(w.x & pb.x);
    c = f_bcnt_acc(w.y & pb.y, c);
    c = f_bcnt_acc(w.z & pb.z, c);
    return f_bcnt_acc(w.w & pb.w, c);
}
// D = sum_{b<7} 2^(b+1) popc(w & P_b) - 2^8 popc(w & P_7) - sum(Q)  (exact)
__device__ __forceinline__ int f_group_dot(uint4 w, const uint4* p, int neg_sum) {
    uint32_t d = (uint32_t)neg_sum;
    d = f_lshl_add<1>(f_plane_count<0>(w, p), d);
    d = f_lshl_add<2>(f_plane_count<1>(w, p), d);
    d = f_lshl_add<3>(f_plane_count<2>(w, p), d);
    d = f_lshl_add<4>(f_plane_count<3>(w, p), d);
    d = f_lshl_add<5>(f_plane_count<4>(w, p), d);
    d = f_lshl_add<6>(f_plane_count<5>(w, p), d);
    d = f_lshl_add<7>(f_plane_count<6>(w, p), d);
    d -= f_plane_count<7>(w, p) << 8;
    return (int)d;
}

// Bit planes B..7 of the wave's 64 quantised values q: lane 2b of `word` receives
// the low and lane 2b + 1 the high half of plane b's mask (v_writelane_b32 with the
// lane as an inline constant), and `sum` accumulates sum(q) from the same masks.
template <int B>
__device__ __forceinline__ void plane_words(int q, uint32_t& word, int& sum) {
    const unsigned long long mask = __ballot((q >> B) & 1);
    const int cnt = __popcll(mask);
    sum += B == 7 ? -(cnt << 7) : (cnt << B);
    // s_nop 1: the two wait states between a VALU write of an SGPR (the ballot) and a
    // VALU read of it, which the compiler cannot insert for inline assembly
    asm("s_nop 1\n\tv_writelane_b32 %0, %1, %2" : "+v"(word) : "s"((uint32_t)mask), "n"(2 * B));
    asm("s_nop 1\n\tv_writelane_b32 %0, %1, %2" : "+v"(word) : "s"((uint32_t)(mask >> 32)), "n"(2 * B + 1));
    if constexpr (B < 7)
        plane_words<B + 1>(q, word, sum);
}

// Q = clamp(round-half-away(F32(x / s)), -127, 127)  (soft-bnn-accelerator.c:197-208)
__device__ __forceinline__ int f_quantize(float x, float s) {
    float r = roundf(x / s);
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    return (int)r;
}

// sum of p[0..n) in index order (n a multiple of 64): steps of 64 values read with
// 16-byte loads at constant offsets, two steps per iteration so that the second
// step's reads are in flight while the first step is added.
__device__ __forceinline__ float sum_in_order_lds(const float* p, uint32_t n) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float sum = 0.0f;
#pragma unroll 2
    for (uint32_t i = 0; i < n / 4u; i += 16u) {
        float4 v[16];
#pragma unroll
        for (int c = 0; c < 16; ++c)
            v[c] = p4[i + c];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            sum = sum + v[c].x;
            sum = sum + v[c].y;
            sum = sum + v[c].z;
            sum = sum + v[c].w;
        }
    }
    return sum;
}

// Workgroup barrier for data exchanged through LDS: waits for this wave's LDS
// accesses only.  __syncthreads would also wait for every outstanding global load
// and store of the wave (its release fence), i.e. for the weight prefetch and for
// the acknowledgement of earlier output stores, none of which the other waves read.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
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

template <int GPW>
__device__ __forceinline__ void load_tile(const FusedJob& job, uint32_t tile, uint32_t G, uint32_t wave,
                                          uint32_t lane, TileRegs<GPW>& r) {
    const size_t base = (size_t)tile * G * kTile + lane;
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
        const uint32_t g = min(wave + kFusedWaves * i, G - 1u);
        r.w[i] = fload(job.wbits + base + (size_t)g * kTile);
        r.s[i] = fload(job.wscale + base + (size_t)g * kTile);
    }
}

// GPW: groups per wave of a tile's dots; EPT: row elements per thread.  Workgroup
// b produces the row once and then takes tiles b, b + grid, ... of the batch, the
// next tile's weights loading while the current one is computed.
template <int GPW, int EPT>
__global__ __launch_bounds__(kFusedThreads) void k_fused(FusedArgs fa, uint32_t tiles_total, uint64_t seq,
                                                         uint64_t* flag, uint64_t* host_status) {
    __shared__ float4 scratch4[(kFusedMaxWidth + kFusedPad) / 4];  // squares, then products [2][group][64]
    __shared__ uint4 planes[kFusedMaxGroups * kPlaneWords / 4];
    __shared__ int part[kFusedMaxGroups][2];
    __shared__ uint32_t amax_w[kFusedWaves];
    __shared__ uint64_t exp_tab[32];
    __shared__ float rms_s;
    float* scratch = reinterpret_cast<float*>(scratch4);

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = fa.width, G = K / kGroup;

    // 1. the row operands load first and the first tile's weights after them (the
    // load counter completes in order: the row is needed first), arriving while the
    // row is produced; thread t owns k = t + 1024 i
    uint32_t tile = blockIdx.x, ji = 0;
    while (ji + 1u < fa.njobs && fa.jobs[ji + 1u].first_tile <= tile)
        ++ji;
    FusedJob job = fa.jobs[ji];
    const float* src_a = fa.kind == PRE_ROW ? fa.row : fa.a;
    float xv[EPT], bv[EPT], gv[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i)
        xv[i] = fload(src_a + min(tid + kFusedThreads * i, K - 1u));
    if (fa.b) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            bv[i] = fload(fa.b + min(tid + kFusedThreads * i, K - 1u));
    }
    if (fa.kind == PRE_RMSNORM) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            gv[i] = fload(fa.gain + min(tid + kFusedThreads * i, K - 1u));
    }
    TileRegs<GPW> cur, nxt;
    load_tile<GPW>(job, tile - job.first_tile, G, wave, lane, cur);

    // 2. the input row
    if (fa.kind == PRE_RMSNORM) {
        if (fa.b) {
#pragma unroll
            for (int i = 0; i < EPT; ++i)
                xv[i] = xv[i] + bv[i];
        }
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const uint32_t k = tid + kFusedThreads * i;
            if (k < K) {
                scratch[k] = xv[i] * xv[i];
                if (fa.a_out && blockIdx.x == 0)
                    fstore(fa.a_out + k, xv[i]);
            }
        }
        lds_barrier();
        if (tid == 0)
            rms_s = sqrtf(sum_in_order_lds(scratch, K) / (float)K + fa.eps);
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
        // the expf table in LDS: its lookups are per-lane gathers
        if (tid < 32u)
            exp_tab[tid] = kFusedExp2Table[tid];
        lds_barrier();
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const float silu = xv[i] / (1.0f + bnne_expf_libc(-xv[i], exp_tab));
            xv[i] = silu * bv[i];
        }
    }

    // 3. the GEMV_F32 input check and the row scale, in one exchange: a wave with a
    // non-finite value posts the all-ones word (above every finite |x| bit pattern)
    uint32_t abits = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        if (tid + kFusedThreads * i < K) {
            const uint32_t a = __float_as_uint(xv[i]) & 0x7fffffffu;
            abits = max(abits, a < 0x7f800000u ? a : 0xffffffffu);
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
    if (amax != 0.0f) {
        s = amax / 127.0f;
        if (s == 0.0f)
            s = __int_as_float(1);  // smallest subnormal
    }

    // 4. quantise: in step i wave w holds the 64 consecutive k of half (w & 1) of
    // group 8i + (w >> 1); bit planes by ballot, the group sums from the same masks
    uint32_t* pw = reinterpret_cast<uint32_t*>(planes);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t chunk = kFusedThreads * i + 64u * wave;
        if (chunk < K) {  // K % 128 == 0: whole waves
            const int q = f_quantize(xv[i], s);
            uint32_t word = 0;
            int sum = 0;
            plane_words<0>(q, word, sum);
            const uint32_t g = (kFusedThreads / kGroup) * i + (wave >> 1), half = wave & 1u;
            if (lane < 16u)
                pw[g * kPlaneWords + (lane >> 1) * 4u + half * 2u + (lane & 1u)] = word;
            if (lane == 0)
                part[g][half] = sum;
        }
    }
    lds_barrier();

    // 5. per tile: group dots and the rounded products F32(scale) * D into one of two
    // product buffers, then wave 0 adds them in group order (one lane per feature)
    // and applies the row scale.  One barrier per tile: a buffer is rewritten only
    // two tiles later, after wave 0 has passed the barrier that follows its sums.
    uint32_t buf = 0;
    for (;;) {
        const uint32_t next = tile + gridDim.x;
        uint32_t nji = ji;
        if (next < tiles_total) {
            while (nji + 1u < fa.njobs && fa.jobs[nji + 1u].first_tile <= next)
                ++nji;
            const FusedJob nj = fa.jobs[nji];
            load_tile<GPW>(nj, next - nj.first_tile, G, wave, lane, nxt);
        }
        float* prod = scratch + buf * (kFusedMaxGroups * 64u);
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const uint32_t g = wave + kFusedWaves * i;
            if (g < G) {
                const int d = f_group_dot(cur.w[i], planes + g * (kPlaneWords / 4u), -(part[g][0] + part[g][1]));
                prod[g * 64u + lane] = __half2float(__ushort_as_half((uint16_t)cur.s[i])) * (float)d;
            }
        }
        lds_barrier();
        if (wave == 0) {
            const uint32_t n = (tile - job.first_tile) * kTile + lane;
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
            if (n < job.n)
                fstore(job.out + n, acc);
        }
        if (next >= tiles_total)
            break;
        tile = next;
        ji = nji;
        job = fa.jobs[ji];
        cur = nxt;
        buf ^= 1u;
    }
}

}  // namespace

hipError_t launch_fused(hipStream_t stream, const FusedArgs& args, uint32_t tiles, uint32_t grid, uint64_t seq,
                        uint64_t* flag, uint64_t* host_status) {
    static_assert(kFusedMaxGroups * 64u * 2u <= kFusedMaxWidth, "two product buffers fit the scratch");
    if (args.width <= 2048u)
        hipLaunchKernelGGL((k_fused<1, 2>), dim3(grid), dim3(kFusedThreads), 0, stream, args, tiles, seq, flag,
                           host_status);
    else
        hipLaunchKernelGGL((k_fused<kFusedMaxGroups / kFusedWaves, kFusedMaxWidth / kFusedThreads>), dim3(grid),
                           dim3(kFusedThreads), 0, stream, args, tiles, seq, flag, host_status);
    return hipGetLastError();
}

}  // namespace bnnhip
