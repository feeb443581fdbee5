// Chained batches (BNNX_BatchCreateChain): GEMM_F32 layers applied one after another to
// every row, each layer's outputs optionally mapped (post_scale * y, then + post_bias,
// then ReLU) and fed to the next layer, in one launch.  One 1024-thread workgroup carries
// one row through every layer; the row between layers stays in LDS.  Per layer the
// workgroup does what the prep and dot kernels do for a GEMM_F32 row (reference
// bnn-accelerator/soft-bnn-accelerator.c:175-276): the legality check and absmax, the row
// scale, the quantisation into bit planes and group sums, the group dots D, the products
// RN(scale * D) and their sum in group order from +0, times the row scale -- so the
// outputs equal separate GEMM_F32 jobs with the mapping done on the host, bit for bit.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "bnn_bitplane.h"
#include "bnn_internal.h"

namespace bnnhip {
namespace {

extern "C" __device__ int __ockl_wfred_add_i32(int);

constexpr uint32_t kChainWaves = 16;
constexpr uint32_t kChainGroups = kChainMaxWidth / kGroup;
// (tile, group) products per pass over a layer's tiles: 24 KiB of LDS; a wave takes
// every 16th pair and requests the weights of all of its pairs before the first dot
// (only of pairs that exist: a workgroup streams a whole layer's weights through its
// CU, and the issue of those loads bounds the layer as much as its dots do)
constexpr uint32_t kChainPairs = 96;
constexpr uint32_t kPairsPerWave = kChainPairs / kChainWaves;

// A layer descriptor read from LDS, with its fields made wave-uniform (scalar registers)
// so that the layer's loops and branches stay scalar.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const void*>((uint64_t)hi << 32 | lo);
}
__device__ __forceinline__ ChainLayer uniform(const ChainLayer& t) {
    ChainLayer u;
    u.wbits = static_cast<const uint4*>(uniform_ptr(t.wbits));
    u.wscale = static_cast<const uint16_t*>(uniform_ptr(t.wscale));
    u.post_scale = static_cast<const float*>(uniform_ptr(t.post_scale));
    u.post_bias = static_cast<const float*>(uniform_ptr(t.post_bias));
    u.k = __builtin_amdgcn_readfirstlane(t.k);
    u.n = __builtin_amdgcn_readfirstlane(t.n);
    u.groups = __builtin_amdgcn_readfirstlane(t.groups);
    u.tiles = __builtin_amdgcn_readfirstlane(t.tiles);
    u.relu = __builtin_amdgcn_readfirstlane(t.relu);
    u.pad_ = 0;
    return u;
}

__global__ __launch_bounds__(64 * kChainWaves) void k_chain(ChainArgs a, uint64_t seq, uint64_t* flag,
                                                            uint64_t* host_status) {
    __shared__ float rows[2][kChainMaxWidth];   // a layer's input row and output row
    __shared__ uint4 planes[kChainGroups * 8];  // plane B of group g at [8 g + B]
    __shared__ int half_sums[2 * kChainGroups]; // sum of Q over each 64-value half of a group
    __shared__ float prods[kChainPairs][kTile];
    __shared__ float red[kChainWaves];
    __shared__ int red_bad[kChainWaves];
    __shared__ ChainLayer table[kChainMaxLayers];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t row = blockIdx.x;

    // the layer table into LDS once (a scalar fetch of a layer's descriptor had cost ~1,600
    // cycles at the start of every layer), with the row
    constexpr uint32_t kLayerWords = sizeof(ChainLayer) / 4u;
    if (tid < a.count * kLayerWords)
        reinterpret_cast<int32_t*>(table)[tid] = gload(reinterpret_cast<const int32_t*>(a.layers) + tid);
    const float* in = reinterpret_cast<const float*>(a.in + (size_t)row * a.in_stride);
    for (uint32_t k = tid; k < a.k0; k += 64u * kChainWaves)
        rows[0][k] = gload(in + k);
    lds_barrier();
    float* x = rows[0];
    float* y = rows[1];
    for (uint32_t l = 0; l < a.count; ++l) {
        const ChainLayer L = uniform(table[l]);
        const bool last = l + 1u == a.count;
        const uint32_t G = L.groups;
        const uint32_t per_pass = kChainPairs / G > 0u ? kChainPairs / G : 1u;
        // pair p of a pass is (tile p / G, group p % G); for p < kChainPairs and G <= 32,
        // p / G = (p * ceil(2^16 / G)) >> 16 exactly (the rounding up adds less than
        // 96 / 2^16, the fraction of p / G is at most 31 / 32): one division per layer
        const uint32_t g_inv = (65535u + G) / G;
        auto tile_of = [&](uint32_t p) { return (p * g_inv) >> 16; };
        // this wave's weights of a pass (every 16th (tile, group) pair) and the mapping of
        // its first tile: the first pass's are requested here, before the row is quantised,
        // so that their latency passes under the check and the quantisation
        uint4 wbits[kPairsPerWave];
        uint32_t wscale[kPairsPerWave];
        float map_scale = 0.0f, map_bias = 0.0f;
        auto request = [&](uint32_t t0) {
            const uint32_t t1 = t0 + per_pass < L.tiles ? t0 + per_pass : L.tiles;
            const uint32_t pairs = (t1 - t0) * G;
#pragma unroll
            for (uint32_t i = 0; i < kPairsPerWave; ++i) {
                const uint32_t p = wave + kChainWaves * i;
                if (p < pairs) {  // wave-uniform
                    const uint32_t tr = tile_of(p), t = t0 + tr, g = p - tr * G;
                    const size_t at = ((size_t)t * G + g) * kTile + lane;
                    wbits[i] = gload(L.wbits + at);
                    wscale[i] = gload(L.wscale + at);
                }
            }
            const uint32_t o = (t0 + wave) * kTile + lane;
            if (L.post_scale && t0 + wave < t1 && o < L.n) {
                map_scale = gload(L.post_scale + o);
                map_bias = gload(L.post_bias + o);
            }
        };
        request(0);
        // legality and absmax of the layer's input row, exchanged in one barrier
        float amax = 0.0f;
        int bad = 0;
        for (uint32_t k = tid; k < L.k; k += 64u * kChainWaves) {
            const float v = x[k];
            bad |= !__builtin_isfinite(v);
            amax = fmaxf(amax, fabsf(v));
        }
        const bool wave_bad = __ballot(bad) != 0ull;
        amax = wave_max_nonneg(amax);  // bit-pattern maximum: meaningful only when no value is bad
        if (lane == 0) {
            red[wave] = amax;
            red_bad[wave] = wave_bad;
        }
        lds_barrier();
        int any_bad = red_bad[0];
        amax = red[0];
#pragma unroll
        for (uint32_t w = 1; w < kChainWaves; ++w) {
            any_bad |= red_bad[w];
            amax = fmaxf(amax, red[w]);
        }
        if (any_bad) {  // this row writes nothing more; the launch reports it
            if (tid == 0)
                raise_flag(seq, flag, host_status);
            return;
        }
        const float s = quant_row_scale(amax);
        const float rcp = quant_rcp(s);
        const bool exact = quant_exact(s);
        // quantise: wave w takes the 64-value halves w, w + 16, ... of the groups; the
        // planes in the prep kernel's layout (lane 2b / 2b + 1: low / high half of plane b)
        uint32_t* plane_words = reinterpret_cast<uint32_t*>(planes);
        for (uint32_t h = wave; h < 2u * G; h += kChainWaves) {
            const int q = quantize_rcp(x[64u * h + lane], s, rcp, exact);
            uint32_t word = 0;
            plane_mask_words(q, word);
            const int part = __ockl_wfred_add_i32(q);
            if (lane < 16u)
                plane_words[(h >> 1) * kPlaneWords + (lane >> 1) * 4u + (h & 1u) * 2u + (lane & 1u)] = word;
            if (lane == 0)
                half_sums[h] = part;
        }
        lds_barrier();
        // the tiles in passes of at most kChainPairs (tile, group) products
        for (uint32_t t0 = 0; t0 < L.tiles; t0 += per_pass) {
            const uint32_t t1 = t0 + per_pass < L.tiles ? t0 + per_pass : L.tiles;
            const uint32_t pairs = (t1 - t0) * G;
            if (t0 > 0)
                request(t0);
#pragma unroll
            for (uint32_t i = 0; i < kPairsPerWave; ++i) {
                const uint32_t p = wave + kChainWaves * i;
                if (p < pairs) {
                    const uint32_t g = p - tile_of(p) * G;
                    const int d = group_dot_v(wbits[i], planes + 8u * g, -(half_sums[2u * g] + half_sums[2u * g + 1u]));
                    prods[p][lane] = __half2float(__ushort_as_half((uint16_t)wscale[i])) * (float)d;
                }
            }
            lds_barrier();
            // wave w adds the products of tiles t0 + w, t0 + w + 16, ... in group order
            for (uint32_t t = t0 + wave; t < t1; t += kChainWaves) {
                const uint32_t o = t * kTile + lane;
                const float* pr = &prods[(t - t0) * G][lane];
                float acc = 0.0f;
                for (uint32_t g = 0; g < G; ++g)
                    acc = acc + pr[g * kTile];
                acc = acc * s;
                if (o < L.n) {
                    if (L.post_scale) {
                        const float sc = t == t0 + wave ? map_scale : gload(L.post_scale + o);
                        const float bi = t == t0 + wave ? map_bias : gload(L.post_bias + o);
                        const float scaled = sc * acc;
                        acc = scaled + bi;
                    }
                    if (L.relu && acc < 0.0f)
                        acc = 0.0f;
                    if (last)
                        gstore(reinterpret_cast<float*>(a.out + (size_t)row * a.out_stride) + o, acc);
                    else
                        y[o] = acc;
                }
            }
            lds_barrier();  // the products are rewritten by the next pass, the row read by the next layer
        }
        float* const t = x;
        x = y;
        y = t;
    }
}

}  // namespace

hipError_t launch_chain(hipStream_t stream, const ChainArgs& args, uint64_t seq, uint64_t* flag,
                        uint64_t* host_status) {
    launch_kernel(k_chain, dim3(args.rows), dim3(64 * kChainWaves), 0, stream, args, seq, flag, host_status);
    return hipGetLastError();
}

}  // namespace bnnhip
