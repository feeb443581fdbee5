// Device helpers shared by the group-dot kernels (bnn_kernels.hip) and the fused
// kernels (bnn_fused.hip): global-memory access through the global address space,
// and the exact group dot by bit planes.
//
// Group dot (reference soft-bnn-accelerator.c:226-258).  With the activation byte Q as
// two's complement bits q_0..q_7 and the 128 weight bits b_k of a group (1 = +1):
//   pos = sum_{b_k = 1} Q_k = sum_{j<7} 2^j popc(B & P_j) - 2^7 popc(B & P_7)
//   D   = 2*pos - sum_k Q_k   (exact, |D| <= 16256)
// where P_j is the 128-bit mask of bit j of Q over the group: 32 AND + 32 accumulating
// BCNT + 8 shift-adds per group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bnnhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Pointers taken from job descriptors are generic; loading through these
// global-address-space views makes the compiler emit global_load, not flat_load
// (a flat access also counts on the LDS counter, so later LDS waits would wait for it).
__device__ __forceinline__ uint4 gload(const uint4* p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gload(const uint16_t* p) {
    return *(const __attribute__((address_space(1))) uint16_t*)p;
}
__device__ __forceinline__ int gload(const int32_t* p) {
    return *(const __attribute__((address_space(1))) int32_t*)p;
}
__device__ __forceinline__ float gload(const float* p) {
    return *(const __attribute__((address_space(1))) float*)p;
}
// Nontemporal loads for weight streams read once per launch (not kept in the caches).
__device__ __forceinline__ uint4 gload_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gload_stream(const uint16_t* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) uint16_t*)p);
}
__device__ __forceinline__ void gstore(float* p, float v) { *(__attribute__((address_space(1))) float*)p = v; }
__device__ __forceinline__ void gstore(int16_t* p, int16_t v) {
    *(__attribute__((address_space(1))) int16_t*)p = v;
}

extern "C" __device__ uint32_t __ockl_wfred_max_u32(uint32_t);

// Max over the wave of non-negative finite floats: their bit patterns order
// like the values, so the DPP-based unsigned wave reduction applies.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    return __uint_as_float(__ockl_wfred_max_u32(__float_as_uint(v)));
}

// Workgroup barrier for data exchanged through LDS: waits for this wave's LDS
// accesses only.  __syncthreads would also wait for every outstanding global load
// and store of the wave (its release fence), i.e. for weight prefetches and for
// the acknowledgement of earlier output stores, none of which the other waves read.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// An illegal input of launch `seq`: the device flag (later kernels of the launch skip their
// stores) and the host-visible status word (BNNX_DeviceSynchronize reports BNN_ERANGE).
__device__ __forceinline__ void raise_flag(uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    __hip_atomic_store(flag, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(host_status, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// popc(x) + acc in one VALU op.  Written as asm because the compiler otherwise
// re-associates the chain into ADD3 trees (11 instead of 9 ops per plane).
// Bit b of the two's complement byte of a quantised value q in [-127, 127] (plane P_b):
// bit 7 is the sign, one signed compare where the other bits take an extract and a compare
__device__ __forceinline__ bool plane_bit(int q, int b) { return b == 7 ? q < 0 : ((q >> b) & 1) != 0; }

// Plane b's 64-bit wave mask into lanes 2b (low half) and 2b + 1 (high half) of `word`:
// two v_writelane_b32 with the lane as an inline constant, where a per-lane select of the
// sixteen halves costs ~47 VALU instructions.  s_nop 1: the two wait states between a VALU
// write of an SGPR (the ballot) and a VALU read of it, which the compiler cannot insert
// for inline assembly.
template <int B>
__device__ __forceinline__ void put_plane_mask(unsigned long long mask, uint32_t& word) {
    asm("s_nop 1\n\tv_writelane_b32 %0, %1, %2" : "+v"(word) : "s"((uint32_t)mask), "n"(2 * B));
    asm("s_nop 1\n\tv_writelane_b32 %0, %1, %2" : "+v"(word) : "s"((uint32_t)(mask >> 32)), "n"(2 * B + 1));
}

// All eight plane masks of the wave's 64 quantised values q, laid out as put_plane_mask does.
template <int B = 0>
__device__ __forceinline__ void plane_mask_words(int q, uint32_t& word) {
    put_plane_mask<B>(__ballot(plane_bit(q, B)), word);
    if constexpr (B < 7)
        plane_mask_words<B + 1>(q, word);
}

__device__ __forceinline__ uint32_t bcnt_acc(uint32_t x, uint32_t acc) {
    uint32_t r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
    return r;
}

// (c << SHIFT) + acc in one VALU op, kept fused for the same reason.
template <int SHIFT>
__device__ __forceinline__ uint32_t lshl_add(uint32_t c, uint32_t acc) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, %2, %3" : "=v"(r) : "v"(c), "i"(SHIFT), "v"(acc));
    return r;
}

// D of one group from the weights w (128 bits) and the eight planes, given through
// `plane_count<B>` (popc(w & P_B)); neg_sum = -sum(Q) of the group.
template <class Count>
__device__ __forceinline__ int group_dot_by(Count count, int neg_sum) {
    uint32_t d = (uint32_t)neg_sum;  // two's complement arithmetic, exact result in [-16256, 16256]
    d = lshl_add<1>(count.template at<0>(), d);
    d = lshl_add<2>(count.template at<1>(), d);
    d = lshl_add<3>(count.template at<2>(), d);
    d = lshl_add<4>(count.template at<3>(), d);
    d = lshl_add<5>(count.template at<4>(), d);
    d = lshl_add<6>(count.template at<5>(), d);
    d = lshl_add<7>(count.template at<6>(), d);
    d -= count.template at<7>() << 8;  // the sign plane weighs -2^7, doubled
    return (int)d;
}

// Planes as four 32-bit words each, P_B = p[4B .. 4B + 3] (in LDS or registers).
struct PlaneWords {
    uint4 w;
    const uint32_t* p;
    template <int B>
    __device__ __forceinline__ uint32_t at() const {
        uint32_t c = (uint32_t)__builtin_popcount(w.x & p[4 * B + 0]);
        c = bcnt_acc(w.y & p[4 * B + 1], c);
        c = bcnt_acc(w.z & p[4 * B + 2], c);
        return bcnt_acc(w.w & p[4 * B + 3], c);
    }
};
// Planes as one 16-byte word each, P_B = p[B].
struct PlaneVecs {
    uint4 w;
    const uint4* p;
    template <int B>
    __device__ __forceinline__ uint32_t at() const {
        const uint4 pb = p[B];
        uint32_t c = (uint32_t)__builtin_popcount(w.x & pb.x);
        c = bcnt_acc(w.y & pb.y, c);
        c = bcnt_acc(w.z & pb.z, c);
        return bcnt_acc(w.w & pb.w, c);
    }
};
// Planes as wave-uniform ballot masks: bit l of m[h][B] is bit B of element 64 h + l.
struct PlaneMasks {
    uint4 w;
    const uint64_t (&m)[2][8];
    template <int B>
    __device__ __forceinline__ uint32_t at() const {
        uint32_t c = (uint32_t)__builtin_popcount(w.x & (uint32_t)m[0][B]);
        c = bcnt_acc(w.y & (uint32_t)(m[0][B] >> 32), c);
        c = bcnt_acc(w.z & (uint32_t)m[1][B], c);
        return bcnt_acc(w.w & (uint32_t)(m[1][B] >> 32), c);
    }
};

__device__ __forceinline__ int group_dot(uint4 w, const uint32_t* p, int neg_sum) {
    return group_dot_by(PlaneWords{w, p}, neg_sum);
}
__device__ __forceinline__ int group_dot_v(uint4 w, const uint4* p, int neg_sum) {
    return group_dot_by(PlaneVecs{w, p}, neg_sum);
}
__device__ __forceinline__ int group_dot_s(uint4 w, const uint64_t (&m)[2][8], int neg_sum) {
    return group_dot_by(PlaneMasks{w, m}, neg_sum);
}

}  // namespace
}  // namespace bnnhip
