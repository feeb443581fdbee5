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

#include "bnn_internal.h"

#pragma clang fp contract(off)

namespace bnnhip {
namespace {

constexpr int kLdsPitch = 65;                     // words per group row of the D/term exchange
constexpr int kMaxGroupsPerWave = kMaxGroups / kDotWaves;

__device__ __forceinline__ float f32_min_subnormal() { return __int_as_float(1); }

__device__ __forceinline__ float load_f32(const unsigned char* row, uint32_t k, bool aligned) {
    if (aligned)
        return reinterpret_cast<const float*>(row)[k];
    float v;
    __builtin_memcpy(&v, row + (size_t)k * 4u, 4);  // byte loads for unaligned views
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v += __shfl_xor(v, off);
    return v;
}

// Q = clamp(round-half-away(F32(x / s)), -127, 127)  (soft-bnn-accelerator.c:197-208)
__device__ __forceinline__ int quantize(float x, float s) {
    float y = x / s;      // correctly rounded IEEE division
    float r = roundf(y);  // half away from zero
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    return (int)r;
}

__device__ __forceinline__ void raise_flag(uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    __hip_atomic_store(flag, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(host_status, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---------------------------------------------------------------------------
// prep: one workgroup (256 threads) per activation row.  Checks the logical row
// (-128 for I8, NaN/Inf for F32: soft-bnn-accelerator.c:278-308), derives the
// row scale, quantises, and writes bit planes, group sums and (optionally) Q.
// ---------------------------------------------------------------------------
__device__ void prep_row(const PrepJob& j, uint32_t m, bool validate_only, uint64_t seq, uint64_t* flag,
                         uint64_t* host_status) {
    __shared__ float red_max[4];
    __shared__ int red_sum[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t k_total = j.k, groups = k_total / kGroup;
    const bool f32 = j.f32 != 0, aligned = j.aligned != 0;
    const unsigned char* row = j.in + (size_t)m * j.in_stride;

    // pass 1: legality and absmax over the whole logical row
    float amax = 0.0f;
    int bad = 0;
    for (uint32_t k = tid; k < k_total; k += 256u) {
        if (f32) {
            float v = load_f32(row, k, aligned);
            bad |= !__builtin_isfinite(v);
            amax = fmaxf(amax, fabsf(v));
        } else {
            bad |= ((int8_t)row[k] == -128);
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
        amax = wave_max(amax);
        if (lane == 0)
            red_max[wave] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));
        if (amax != 0.0f) {
            s = amax / 127.0f;
            if (s == 0.0f)
                s = f32_min_subnormal();
        }
    }

    // pass 2: quantise; each wave owns 64 consecutive k = one half group
    uint32_t* planes = j.planes + (size_t)m * groups * kPlaneWords;
    for (uint32_t base = 0; base < k_total; base += 256u) {
        const uint32_t k = base + tid;
        const bool wave_live = base + wave * 64u < k_total;  // K % 128 == 0: whole waves
        if (wave_live) {
            const int q = f32 ? quantize(load_f32(row, k, aligned), s) : (int)(int8_t)row[k];
            if (j.q)
                j.q[(size_t)m * k_total + k] = (int8_t)q;
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const unsigned long long mask = __ballot((q >> b) & 1);
                if (lane == 2u * b)
                    word = (uint32_t)mask;
                if (lane == 2u * b + 1u)
                    word = (uint32_t)(mask >> 32);
            }
            const uint32_t g = (base >> 7) + (wave >> 1), half = wave & 1u;
            if (lane < 16u)
                planes[g * kPlaneWords + (lane >> 1) * 4u + half * 2u + (lane & 1u)] = word;
            const int part = wave_sum(q);
            if (lane == 0)
                red_sum[wave] = part;
        }
        __syncthreads();
        if (tid == 0)
            j.sums[(size_t)m * groups + (base >> 7)] = red_sum[0] + red_sum[1];
        if (tid == 128 && base + 128u < k_total)
            j.sums[(size_t)m * groups + (base >> 7) + 1u] = red_sum[2] + red_sum[3];
        __syncthreads();
    }
    if (tid == 0)
        j.rscale[m] = s;
}

template <bool BATCH>
__global__ __launch_bounds__(256) void k_prep(PrepJob single, const PrepJob* __restrict__ jobs,
                                              const uint32_t* __restrict__ block_job, int validate_only,
                                              uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    if (BATCH) {
        const PrepJob j = jobs[block_job[blockIdx.x]];
        prep_row(j, blockIdx.x - j.first_block, false, seq, flag, host_status);
    } else {
        prep_row(single, blockIdx.x, validate_only != 0, seq, flag, host_status);
    }
}

// Positive-bit sum of one group: weights w (128 bits), activation planes p[32].
__device__ __forceinline__ int group_pos(uint4 w, const uint32_t* p) {
    int pos = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const int c = __popc(w.x & p[4 * b + 0]) + __popc(w.y & p[4 * b + 1]) + __popc(w.z & p[4 * b + 2]) +
                      __popc(w.w & p[4 * b + 3]);
        pos += (b == 7) ? -(c << 7) : (c << b);
    }
    return pos;
}

// ---------------------------------------------------------------------------
// dot: one workgroup of 4 waves per (row, tile of 64 features).  Wave w owns a
// contiguous run of groups, issues all its weight and scale loads first, then
// computes D (and the rounded product) per group; lane = feature.  The row's
// bit planes are staged once in LDS.  Wave 0 then adds the products in group
// order (F32 modes) or the workgroup stores D as int16 (DOT_GROUPS).
// ---------------------------------------------------------------------------
__device__ void dot_tile(const DotJob& j, uint32_t local) {
    __shared__ uint4 lds_planes[kMaxGroups * kPlaneWords / 4];
    __shared__ int lds_sums[kMaxGroups];
    __shared__ int lds_x[kMaxGroups * kLdsPitch];  // D (int) or product (float bits)

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t groups = j.groups;
    const uint32_t row = local / j.tiles, t = local - row * j.tiles;
    const uint32_t gpw = (groups + kDotWaves - 1u) / kDotWaves;
    const uint32_t g0 = wave * gpw;
    const uint32_t gcount = g0 < groups ? (groups - g0 < gpw ? groups - g0 : gpw) : 0u;
    const bool sum_mode = j.mode != MODE_DOT_I16;

    // 1. issue this wave's weight and scale loads (up to 16 groups)
    uint4 w[kMaxGroupsPerWave];
    uint16_t sc[kMaxGroupsPerWave];
    const size_t tile_base = (size_t)t * groups;
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)kMaxGroupsPerWave; ++i) {
        if (i < gcount) {
            w[i] = j.wbits[(tile_base + g0 + i) * kTile + lane];
            sc[i] = sum_mode ? j.wscale[(tile_base + g0 + i) * kTile + lane] : (uint16_t)0;
        }
    }
    // 2. stage the row's planes and group sums in LDS (coalesced, shared by all waves)
    const uint4* src = reinterpret_cast<const uint4*>(j.planes + (size_t)row * groups * kPlaneWords);
    for (uint32_t i = tid; i < groups * (kPlaneWords / 4u); i += 64u * kDotWaves)
        lds_planes[i] = src[i];
    if (tid < groups)
        lds_sums[tid] = j.sums[(size_t)row * groups + tid];
    __syncthreads();

    // 3. group dots (+ rounded products)
    const uint32_t* lp = reinterpret_cast<const uint32_t*>(lds_planes);
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)kMaxGroupsPerWave; ++i) {
        if (i < gcount) {
            const uint32_t g = g0 + i;
            const int d = 2 * group_pos(w[i], lp + g * kPlaneWords) - lds_sums[g];
            if (sum_mode) {
                const float prod = __half2float(__ushort_as_half(sc[i])) * (float)d;
                lds_x[g * kLdsPitch + lane] = __float_as_int(prod);
            } else {
                lds_x[g * kLdsPitch + lane] = d;
            }
        }
    }
    __syncthreads();

    // 4. in-order sums or int16 stores
    const uint32_t n0 = t * kTile;
    const uint32_t live = j.n - n0 < kTile ? j.n - n0 : kTile;
    unsigned char* orow = j.out + (size_t)row * j.out_stride;
    if (!sum_mode) {
        int16_t* o = reinterpret_cast<int16_t*>(orow) + (size_t)n0 * groups;
        for (uint32_t idx = tid; idx < live * groups; idx += 64u * kDotWaves) {
            const uint32_t nl = idx / groups, g = idx - nl * groups;
            o[idx] = (int16_t)lds_x[g * kLdsPitch + nl];
        }
    } else if (wave == 0 && lane < live) {
        float acc = 0.0f;
        for (uint32_t g = 0; g < groups; ++g)
            acc = acc + __int_as_float(lds_x[g * kLdsPitch + lane]);
        if (j.mode == MODE_SUM_SCALED)
            acc = acc * j.rscale[row];
        reinterpret_cast<float*>(orow)[n0 + lane] = acc;
    }
}

template <bool BATCH>
__global__ __launch_bounds__(64 * kDotWaves) void k_dot(DotJob single, const DotJob* __restrict__ jobs,
                                                        const uint32_t* __restrict__ block_job, uint64_t seq,
                                                        const uint64_t* __restrict__ flag) {
    if (*flag == seq)
        return;  // some row of this job (batch) is illegal: write nothing
    if (BATCH) {
        const DotJob j = jobs[block_job[blockIdx.x]];
        dot_tile(j, blockIdx.x - j.first_block);
    } else {
        dot_tile(single, blockIdx.x);
    }
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

}  // namespace

hipError_t launch_prep(hipStream_t stream, const PrepJob& job, bool validate_only, uint64_t seq, uint64_t* flag,
                       uint64_t* host_status) {
    hipLaunchKernelGGL(k_prep<false>, dim3(job.rows), dim3(256), 0, stream, job, nullptr, nullptr,
                       (int)validate_only, seq, flag, host_status);
    return hipGetLastError();
}

hipError_t launch_dot(hipStream_t stream, const DotJob& job, uint64_t seq, const uint64_t* flag) {
    hipLaunchKernelGGL(k_dot<false>, dim3(job.tiles * job.rows), dim3(64 * kDotWaves), 0, stream, job, nullptr,
                       nullptr, seq, flag);
    return hipGetLastError();
}

hipError_t launch_prep_batch(hipStream_t stream, const PrepJob* jobs, const uint32_t* block_job, uint32_t blocks,
                             uint64_t seq, uint64_t* flag, uint64_t* host_status) {
    PrepJob none = {};
    hipLaunchKernelGGL(k_prep<true>, dim3(blocks), dim3(256), 0, stream, none, jobs, block_job, 0, seq, flag,
                       host_status);
    return hipGetLastError();
}

hipError_t launch_dot_batch(hipStream_t stream, const DotJob* jobs, const uint32_t* block_job, uint32_t blocks,
                            uint64_t seq, const uint64_t* flag) {
    DotJob none = {};
    hipLaunchKernelGGL(k_dot<true>, dim3(blocks), dim3(64 * kDotWaves), 0, stream, none, jobs, block_job, seq,
                       flag);
    return hipGetLastError();
}

hipError_t launch_scatter(hipStream_t stream, const unsigned char* src, size_t src_stride, unsigned char* dst,
                          size_t dst_stride, size_t row_bytes, uint32_t rows, uint64_t seq, const uint64_t* flag) {
    size_t blocks = (row_bytes + 255u) / 256u;
    if (blocks > 1024u)
        blocks = 1024u;
    hipLaunchKernelGGL(k_scatter, dim3((uint32_t)blocks, rows), dim3(256), 0, stream, src, src_stride, dst,
                       dst_stride, row_bytes, seq, flag);
    return hipGetLastError();
}

}  // namespace bnnhip
