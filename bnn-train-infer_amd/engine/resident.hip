// Device-resident Qwen3 decode step (see resident.h).
//
// Per token, on the accelerator device's stream:
//   embed -> for each layer: [x += o] RMSNorm -> q/k/v batch -> q/k head norms, RoPE,
//   KV-cache store -> attention -> o batch -> x += o, RMSNorm -> gate/up batch ->
//   SiLU(gate)*up -> down batch;  then x += o, final RMSNorm, lm_head batch.
// One host wait per Decode call.  Each kernel restates one piece of the host step
// (bnn-sw-v2/qwen3/qwen3.c:342-512) with its operation order: products and
// quotients are formed elementwise, every sum runs in index order in one lane.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <algorithm>

#include "bnn-accelerator-hip.h"
#include "resident.h"

#define BNNE_EXPF_QUALIFIER static __device__ __forceinline__
#include "../csrc/libc_expf.h"

#pragma clang fp contract(off)

namespace bnne {
namespace {

constexpr uint32_t kMaxHeadDim = 512;
constexpr uint32_t kMaxNormWidth = 16384;
enum : int { kErrNone = 0, kErrNorm = 1, kErrScore = 2, kErrSoftmax = 3 };

// expf of the host C library, bit for bit (see libc_expf.h)
__constant__ uint64_t kExp2Table[32] = BNNE_EXP2_TABLE;

__device__ __forceinline__ float expf_libc(float x) { return bnne_expf_libc(x, kExp2Table); }

// The table into LDS for per-lane lookups (called by one whole wave): scalar loads, whose
// wait (lgkmcnt) leaves the wave's vector loads in flight -- a vector load of the table
// would complete in order behind every key row and V row the wave has requested
template <int I>
__device__ __forceinline__ void exp_table_fill_lanes(uint32_t& lo, uint32_t& hi) {
    const uint64_t e = kExp2Table[I];  // uniform address: a scalar load
    asm("v_writelane_b32 %0, %1, %2" : "+v"(lo) : "s"((uint32_t)e), "n"(I));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(hi) : "s"((uint32_t)(e >> 32)), "n"(I));
    if constexpr (I < 31)
        exp_table_fill_lanes<I + 1>(lo, hi);
}
__device__ __forceinline__ void exp_table_fill(uint64_t* tab, uint32_t lane) {
    uint32_t lo = 0, hi = 0;
    exp_table_fill_lanes<0>(lo, hi);
    if (lane < 32u)
        tab[lane] = (uint64_t)hi << 32 | lo;
}

// Sequential sums with latency hiding: the values of a chunk are loaded into
// registers first (independent loads, issued back to back), then added one after
// another in index order -- the same roundings as a plain loop.
template <int CHUNK, class Load>
__device__ __forceinline__ float sum_in_order(uint32_t n, Load load) {
    float sum = 0.0f;
    uint32_t i = 0;
    for (; i + CHUNK <= n; i += CHUNK) {
        float v[CHUNK];
#pragma unroll
        for (int c = 0; c < CHUNK; ++c)
            v[c] = load(i + c);
#pragma unroll
        for (int c = 0; c < CHUNK; ++c)
            sum = sum + v[c];
    }
    for (; i < n; ++i)
        sum = sum + load(i);
    return sum;
}

// sum plus the n floats held in LDS (16-byte aligned), added in index order: 16-byte
// loads; the second half of each 64-value step is loading while the first is added.
__device__ __forceinline__ float sum_lds_in_order(const float* p, uint32_t n, float sum = 0.0f) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    const uint32_t n4 = n / 4u;
    uint32_t i = 0;
    for (; i + 16u <= n4; i += 16u) {
        float4 a[8], b[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            a[c] = p4[i + c];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            b[c] = p4[i + 8u + c];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            sum = sum + a[c].x;
            sum = sum + a[c].y;
            sum = sum + a[c].z;
            sum = sum + a[c].w;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            sum = sum + b[c].x;
            sum = sum + b[c].y;
            sum = sum + b[c].z;
            sum = sum + b[c].w;
        }
    }
    for (uint32_t k = i * 4u; k < n; ++k)
        sum = sum + p[k];
    return sum;
}

__device__ void set_error(int* err, int code) { atomicCAS(err, kErrNone, code); }

extern "C" __device__ float __ockl_wfred_max_f32(float);

// Greedy decoding on the device takes the caller's argmax (bnn-infer-v2.c:48-54: the
// first index of the largest logit) as the largest of 64-bit keys: the order-preserving
// image of the value's bits above the complement of the index, so that equal values
// order by the smaller index.  -0 is made +0 first (the reference compares values, and
// -0 == +0).  Every key is nonzero, and the index it carries is one of the logits'.
__device__ __forceinline__ unsigned long long logit_key(float v, uint32_t i) {
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (0xffffffffu - i);
}
__device__ __forceinline__ uint32_t key_token(unsigned long long key) { return 0xffffffffu - (uint32_t)key; }

// x[i] = +scale or -scale of the token's Q1_0 embedding row (qwen3.c:355-366).  In a
// greedy run the token is the one the previous step's argmax left in *key_in; the first
// workgroup records it in *tok_out and clears *key_reset for this step's argmax.  The
// first token of a call also clears the step error word and the logits flag (err_reset,
// bad_reset; null otherwise), so that nothing a failed earlier call left behind is
// reported by this one.
__global__ __launch_bounds__(256) void k_embed(uint32_t token, const unsigned long long* __restrict__ key_in,
                                               int32_t* __restrict__ tok_out, unsigned long long* __restrict__ key_reset,
                                               int* __restrict__ err_reset, int* __restrict__ bad_reset,
                                               const uint8_t* __restrict__ bits,
                                               const uint16_t* __restrict__ scales, uint32_t C,
                                               float* __restrict__ x) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (key_in)
        token = key_token(*key_in);
    if (i == 0) {
        if (tok_out)
            *tok_out = (int32_t)token;
        if (key_reset)
            *key_reset = 0;
        if (err_reset)
            *err_reset = kErrNone;
        if (bad_reset)
            *bad_reset = 0;
    }
    if (i >= C)
        return;
    const float s = __half2float(__ushort_as_half(scales[(size_t)token * (C / 128u) + i / 128u]));
    const bool bit = (bits[(size_t)token * (C / 8u) + i / 8u] >> (i & 7u)) & 1u;
    x[i] = bit ? s : -s;
}

// The argmax of the logits as the largest key (above), merged into *key, which the
// step's embedding launch cleared; a non-finite logit sets *bad (the engine's check of
// the logits).
constexpr uint32_t kArgmaxThreads = 256;
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax(const float* __restrict__ logits, uint32_t V,
                                                           unsigned long long* __restrict__ key, int* __restrict__ bad) {
    __shared__ unsigned long long wave_best[kArgmaxThreads / 64u];
    unsigned long long best = 0;
    bool nonfinite = false;
    for (uint32_t i = blockIdx.x * kArgmaxThreads + threadIdx.x; i < V; i += gridDim.x * kArgmaxThreads) {
        const float v = logits[i];
        nonfinite |= !__builtin_isfinite(v);
        best = max(best, logit_key(v, i));
    }
    if (nonfinite)
        *bad = 1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)best, off), hi = __shfl_xor((uint32_t)(best >> 32), off);
        best = max(best, ((unsigned long long)hi << 32) | lo);
    }
    if ((threadIdx.x & 63u) == 0)
        wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (uint32_t w = 1; w < kArgmaxThreads / 64u; ++w)
            best = max(best, wave_best[w]);
        atomicMax(key, best);
    }
}

// The last greedy step's token, which no later embedding launch records.
__global__ __launch_bounds__(64) void k_key_token(const unsigned long long* __restrict__ key, int32_t* __restrict__ out) {
    if (threadIdx.x == 0)
        *out = (int32_t)key_token(*key);
}

// [x += add] then out = x / rms * gain, rms = sqrt(sum x^2 / n + eps) with the sum
// in index order (qwen3.c:342-353).  One workgroup of kNormThreads; every thread
// loads its values (and gains) before anything else, so that the global-memory
// latency is paid once.
constexpr uint32_t kNormThreads = 1024;
constexpr uint32_t kNormPerThread = kMaxNormWidth / kNormThreads;

__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(float* __restrict__ x, const float* __restrict__ add,
                                                          uint32_t n, float eps, const float* __restrict__ gain,
                                                          float* __restrict__ out, int* err) {
    extern __shared__ float4 sq_lds[];
    float* sq = reinterpret_cast<float*>(sq_lds);
    __shared__ float rms_s;
    const uint32_t tid = threadIdx.x;
    // unconditional loads at clamped indexes: all of them in flight at once
    float xv[kNormPerThread], av[kNormPerThread], gv[kNormPerThread];
#pragma unroll
    for (uint32_t c = 0; c < kNormPerThread; ++c)
        xv[c] = x[min(tid + c * kNormThreads, n - 1u)];
    if (add) {
#pragma unroll
        for (uint32_t c = 0; c < kNormPerThread; ++c)
            av[c] = add[min(tid + c * kNormThreads, n - 1u)];
#pragma unroll
        for (uint32_t c = 0; c < kNormPerThread; ++c)
            xv[c] = xv[c] + av[c];
    }
#pragma unroll
    for (uint32_t c = 0; c < kNormPerThread; ++c)
        gv[c] = gain[min(tid + c * kNormThreads, n - 1u)];
#pragma unroll
    for (uint32_t c = 0; c < kNormPerThread; ++c) {
        const uint32_t i = tid + c * kNormThreads;
        if (i < n) {
            if (add)
                x[i] = xv[c];
            sq[i] = xv[c] * xv[c];
        }
    }
    __syncthreads();
    if (tid == 0) {
        const float sum = sum_lds_in_order(sq, n);
        const float rms = sqrtf(sum / (float)n + eps);
        if (!isfinite(rms) || rms == 0.0f)
            set_error(err, kErrNorm);
        rms_s = rms;
    }
    __syncthreads();
    const float rms = rms_s;
#pragma unroll
    for (uint32_t c = 0; c < kNormPerThread; ++c) {
        const uint32_t i = tid + c * kNormThreads;
        if (i < n)
            out[i] = xv[c] / rms * gv[c];
    }
}

// Per head (blocks 0..H-1: q heads, H..H+Hk-1: k heads): RMSNorm over head_dim,
// then the RoPE rotation of pairs (j, j + HD/2) (qwen3.c:419-438); k heads and the
// matching v values are stored into the layer's cache row at `pos`.
__global__ __launch_bounds__(64) void k_head_norm_rope(float* __restrict__ q, float* __restrict__ k,
                                                       const float* __restrict__ v, uint32_t H, uint32_t HD,
                                                       float eps, const float* __restrict__ q_gain,
                                                       const float* __restrict__ k_gain,
                                                       const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                       float* __restrict__ k_row, float* __restrict__ v_row,
                                                       int* err) {
    __shared__ float buf[kMaxHeadDim];
    __shared__ float rms_s;
    const uint32_t h = blockIdx.x, lane = threadIdx.x;
    const bool is_q = h < H;
    const uint32_t kh = h - H;
    float* vec = is_q ? q + (size_t)h * HD : k + (size_t)kh * HD;
    const float* gain = is_q ? q_gain : k_gain;
    __shared__ float4 sq4[kMaxHeadDim / 4];
    float* sq = reinterpret_cast<float*>(sq4);
    for (uint32_t i = lane; i < HD; i += 64u) {
        const float x = vec[i];
        buf[i] = x;
        sq[i] = x * x;
    }
    __syncthreads();
    if (lane == 0) {
        const float sum = sum_lds_in_order(sq, HD);
        const float rms = sqrtf(sum / (float)HD + eps);
        if (!isfinite(rms) || rms == 0.0f)
            set_error(err, kErrNorm);
        rms_s = rms;
    }
    __syncthreads();
    const float rms = rms_s;
    for (uint32_t i = lane; i < HD; i += 64u)
        buf[i] = buf[i] / rms * gain[i];
    __syncthreads();
    const uint32_t half = HD / 2u;
    for (uint32_t j = lane; j < half; j += 64u) {
        const float a = buf[j], b = buf[j + half];
        const float lo = a * cosv[j] - b * sinv[j];
        const float hi = a * sinv[j] + b * cosv[j];
        vec[j] = lo;
        vec[j + half] = hi;
        if (!is_q) {
            k_row[(size_t)kh * HD + j] = lo;
            k_row[(size_t)kh * HD + j + half] = hi;
        }
    }
    if (!is_q)
        for (uint32_t i = lane; i < HD; i += 64u)
            v_row[(size_t)kh * HD + i] = v[(size_t)kh * HD + i];
}

// value[i] = sum over t = 0..pos in order of p[t] * V[t][i] for the head's i (one
// per thread, HD <= 512 over two rounds).  V rows come through LDS in chunks of
// kVChunk rows, loaded with coalesced 16-byte reads by the whole workgroup; row pos
// is read from `v_last` when it is not null (the row not yet in the cache).
constexpr uint32_t kVChunkFloats = 4096;  // 16 KB of V rows per chunk

__device__ __forceinline__ void pv_accumulate(const float* __restrict__ sc, const float* __restrict__ vc,
                                              const float* __restrict__ v_last, size_t head_off, uint32_t pos,
                                              uint32_t kv_dim, uint32_t HD, float4* vs4, float* __restrict__ y) {
    const uint32_t tid = threadIdx.x;
    const float* vs = reinterpret_cast<const float*>(vs4);
    const uint32_t rows = kVChunkFloats / HD, hd4 = HD / 4u;
    float acc0 = 0.0f, acc1 = 0.0f;
    for (uint32_t t0 = 0; t0 <= pos; t0 += rows) {
        const uint32_t n = min(rows, pos + 1u - t0);
        for (uint32_t idx = tid; idx < n * hd4; idx += 256u) {
            const uint32_t r = idx / hd4, c = idx - r * hd4;
            const uint32_t t = t0 + r;
            const float* src = (t == pos && v_last) ? v_last + head_off : vc + (size_t)t * kv_dim + head_off;
            vs4[idx] = reinterpret_cast<const float4*>(src)[c];
        }
        __syncthreads();
        if (tid < HD) {
            uint32_t r = 0;
            for (; r + 8u <= n; r += 8u) {
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    acc0 = acc0 + sc[t0 + r + c] * vs[(r + c) * HD + tid];
            }
            for (; r < n; ++r)
                acc0 = acc0 + sc[t0 + r] * vs[r * HD + tid];
        }
        if (tid + 256u < HD) {
            for (uint32_t r = 0; r < n; ++r)
                acc1 = acc1 + sc[t0 + r] * vs[r * HD + tid + 256u];
        }
        __syncthreads();
    }
    if (tid < HD)
        y[tid] = acc0;
    if (tid + 256u < HD)
        y[tid + 256u] = acc1;
}

// Causal attention of one head against cache rows 0..pos (qwen3.c:441-478):
// scores (each dot sequential over head_dim), max, exp, the sum in position order,
// probabilities, and each output element's sum in position order.  Scores and
// probabilities live in LDS up to kLdsPositions positions, in `scores` beyond.
constexpr uint32_t kLdsPositions = 8192;  // 32 KB of scores; beyond, `scores` in global memory

__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q, const float* __restrict__ kc,
                                                   const float* __restrict__ vc, uint32_t pos, uint32_t kv_dim,
                                                   uint32_t HD, uint32_t kv_mul, float scale,
                                                   float* __restrict__ scores, uint32_t n_ctx,
                                                   float* __restrict__ y, int* err) {
    __shared__ float qs[kMaxHeadDim];
    __shared__ float red[256];
    __shared__ float sum_s;
    __shared__ float4 lds_sc4[kLdsPositions / 4];
    __shared__ float4 vs4[kVChunkFloats / 4];
    float* lds_sc = reinterpret_cast<float*>(lds_sc4);
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const size_t head_off = (size_t)(h / kv_mul) * HD;
    float* sc = pos < kLdsPositions ? lds_sc : scores + (size_t)h * n_ctx;
    for (uint32_t i = tid; i < HD; i += 256u)
        qs[i] = q[(size_t)h * HD + i];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t t = tid; t <= pos; t += 256u) {
        const float* key = kc + (size_t)t * kv_dim + head_off;
        float dot = 0.0f;
        uint32_t i = 0;
        for (; i + 16u <= HD; i += 16u) {
            float4 kv[4];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                kv[c] = *reinterpret_cast<const float4*>(key + i + 4u * c);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dot = dot + qs[i + 4u * c] * kv[c].x;
                dot = dot + qs[i + 4u * c + 1u] * kv[c].y;
                dot = dot + qs[i + 4u * c + 2u] * kv[c].z;
                dot = dot + qs[i + 4u * c + 3u] * kv[c].w;
            }
        }
        for (; i < HD; ++i)
            dot = dot + qs[i] * key[i];
        const float score = dot * scale;
        if (!isfinite(score))
            set_error(err, kErrScore);
        sc[t] = score;
        mx = score > mx ? score : mx;
    }
    red[tid] = mx;
    __syncthreads();
    for (uint32_t s = 128u; s > 0; s >>= 1) {
        if (tid < s)
            red[tid] = red[tid + s] > red[tid] ? red[tid + s] : red[tid];
        __syncthreads();
    }
    const float maximum = red[0];
    for (uint32_t t = tid; t <= pos; t += 256u)
        sc[t] = expf_libc(sc[t] - maximum);
    __threadfence_block();
    __syncthreads();
    if (tid == 0) {
        const float sum = pos < kLdsPositions ? sum_lds_in_order(sc, pos + 1u)
                                              : sum_in_order<32>(pos + 1u, [&](uint32_t t) { return sc[t]; });
        if (!(sum > 0.0f) || !isfinite(sum))
            set_error(err, kErrSoftmax);
        sum_s = sum;
    }
    __syncthreads();
    const float sum = sum_s;
    for (uint32_t t = tid; t <= pos; t += 256u)
        sc[t] = sc[t] / sum;
    __threadfence_block();
    __syncthreads();
    pv_accumulate(sc, vc, nullptr, head_off, pos, kv_dim, HD, vs4, y + (size_t)h * HD);
}

// Error words of the fused step: the code of the earliest failure in the host
// step's order wins.  Per layer l the codes are l * span + p, with p = 1 for the
// attention RMSNorm, 2 for the q/k head norms, 3 + 2h / 4 + 2h for the score /
// softmax checks of head h and 3 + 2H for the FFN RMSNorm (span = 4 + 2H); the
// final RMSNorm is L * span + 1.  Codes only grow along the step, so "smallest
// code" is "first failure"; the backend's fused batches store theirs only into a
// clear word, which they can only meet after every earlier code of the step.
__device__ void set_error_first(int* err, int code) {
    int old = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (old == kErrNone || old > code) {
        const int prev = atomicCAS(err, old, code);
        if (prev == old)
            break;
        old = prev;
    }
}

// Attention of the fused step (qwen3.c:417-478) in two launches that spread the
// layer's K and V rows over many workgroups:
//   k_attn_scores, workgroup (query head h, block of 64 positions), one wave: the
//   RMSNorm of the head and of its kv head's new key over head_dim (the two in-order
//   sums interleaved, in every lane), RoPE of both, the cache row at pos (stored by
//   the kv head's first query head, in the block that holds pos), then one score per
//   lane, each an in-order dot over head_dim -- position pos from the wave's own new
//   key, so no workgroup reads a row another is writing;
//   k_attn_pv, workgroup (query head h, slice of 32 head dims), two waves: the maximum,
//   expf, the in-order sum and the probabilities over positions 0..pos, then
//   value[i] = sum over t in order of p[t] * V[t][i] for the slice's i, the V rows
//   moved into LDS by DMA by a second wave meanwhile.
// Every sum runs in index / position order, as in the host step.
constexpr uint32_t kAttnHD = 128;             // head_dim of the fused step
constexpr uint32_t kScoreBlock = 64;          // positions per k_attn_scores workgroup
constexpr uint32_t kPvSlice = 32;             // head dims per k_attn_pv workgroup
constexpr uint32_t kPvLdsPositions = 4096;    // probabilities in LDS (16 KB); beyond, recomputed

// Orders one wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(64) void k_attn_scores(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, uint32_t kv_mul, float eps,
    const float* __restrict__ q_gain, const float* __restrict__ k_gain, const float* __restrict__ cosv,
    const float* __restrict__ sinv, float* __restrict__ kc, float* __restrict__ vc, uint32_t pos, uint32_t kv_dim,
    float scale, float* __restrict__ scores, uint32_t n_ctx, int* err, int code_base) {
    constexpr uint32_t HD = kAttnHD, hd4 = HD / 4, half = HD / 2;
    __shared__ float4 sq4[2][hd4];  // the squares of q and k
    __shared__ float4 qk4[2][hd4];  // q and k normalised and rotated
    const uint32_t lane = threadIdx.x, h = blockIdx.x, t = blockIdx.y * kScoreBlock + lane;
    const size_t head_off = (size_t)(h / kv_mul) * HD;
    const bool row_owner = h % kv_mul == 0 && blockIdx.y == pos / kScoreBlock;

    // reads, in the order they are needed: elements lane and lane + 64 of the head
    // vectors and gains (a RoPE pair), the RoPE factors, then this lane's key row
    // (rows past pos clamped to pos: loaded, never used)
    const float qa = q[(size_t)h * HD + lane], qb = q[(size_t)h * HD + lane + half];
    const float ka = k[head_off + lane], kb = k[head_off + lane + half];
    const float qga = q_gain[lane], qgb = q_gain[lane + half], kga = k_gain[lane], kgb = k_gain[lane + half];
    const float c = cosv[lane], s = sinv[lane];
    float4 key[hd4];
    {
        const float4* row = reinterpret_cast<const float4*>(kc + (size_t)min(t, pos) * kv_dim + head_off);
#pragma unroll
        for (uint32_t i = 0; i < hd4; ++i)
            key[i] = row[i];
    }

    // head norms: both in-order sums over head_dim, interleaved, in every lane
    float* sq_q = reinterpret_cast<float*>(sq4[0]);
    float* sq_k = reinterpret_cast<float*>(sq4[1]);
    sq_q[lane] = qa * qa;
    sq_q[lane + half] = qb * qb;
    sq_k[lane] = ka * ka;
    sq_k[lane + half] = kb * kb;
    wave_lds_sync();
    float sum_q = 0.0f, sum_k = 0.0f;
#pragma unroll 8
    for (uint32_t i = 0; i < hd4; ++i) {
        const float4 a = sq4[0][i], b = sq4[1][i];
        sum_q = sum_q + a.x;
        sum_k = sum_k + b.x;
        sum_q = sum_q + a.y;
        sum_k = sum_k + b.y;
        sum_q = sum_q + a.z;
        sum_k = sum_k + b.z;
        sum_q = sum_q + a.w;
        sum_k = sum_k + b.w;
    }
    const float rq = sqrtf(sum_q / (float)HD + eps), rk = sqrtf(sum_k / (float)HD + eps);
    if (!isfinite(rq) || rq == 0.0f || !isfinite(rk) || rk == 0.0f) {
        if (lane == 0)
            set_error_first(err, code_base + 2);
        return;
    }
    // x / rms * gain, then the rotation of pair (lane, lane + 64)
    const float nqa = qa / rq * qga, nqb = qb / rq * qgb;
    const float nka = ka / rk * kga, nkb = kb / rk * kgb;
    float* qr = reinterpret_cast<float*>(qk4[0]);
    float* kr = reinterpret_cast<float*>(qk4[1]);
    qr[lane] = nqa * c - nqb * s;
    qr[lane + half] = nqa * s + nqb * c;
    const float rka = nka * c - nkb * s, rkb = nka * s + nkb * c;
    kr[lane] = rka;
    kr[lane + half] = rkb;
    if (row_owner) {
        kc[(size_t)pos * kv_dim + head_off + lane] = rka;
        kc[(size_t)pos * kv_dim + head_off + lane + half] = rkb;
        vc[(size_t)pos * kv_dim + head_off + lane] = v[head_off + lane];
        vc[(size_t)pos * kv_dim + head_off + lane + half] = v[head_off + lane + half];
    }
    wave_lds_sync();

    // the score of position t: in-order dot over head_dim (row pos: the new key)
    if (t == pos) {
#pragma unroll
        for (uint32_t i = 0; i < hd4; ++i)
            key[i] = qk4[1][i];
    }
    float dot = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < hd4; ++i) {
        const float4 qq = qk4[0][i];
        dot = dot + qq.x * key[i].x;
        dot = dot + qq.y * key[i].y;
        dot = dot + qq.z * key[i].z;
        dot = dot + qq.w * key[i].w;
    }
    if (t <= pos) {
        const float score = dot * scale;
        if (!isfinite(score))
            set_error_first(err, code_base + 3 + 2 * (int)h);
        scores[(size_t)h * n_ctx + t] = score;
    }
}

// 16 bytes per lane from global memory into LDS at lds_addr + 16 * lane (lds_addr is
// the wave's base, in M0).  Inline assembly: the wave waits for these loads itself
// (vmcnt(0)).  The s_nop covers the wait state between writing M0 and the LDS DMA
// reading it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_addr) : "memory");
}

// Attention of one query head in a single launch, for contexts of fewer than
// kAttnOneMax positions (pos < kAttnOneMax): workgroup h, four waves, the same
// operations in the same order as k_attn_scores + k_attn_pv.  Position t belongs to
// thread (t + 64) % 256: waves 1..3 hold positions 0..191 and wave 0 the rest, and wave 0
// requests its key rows only after its norms (loads complete in order: a wait for the
// head vectors would also wait for every row requested after them).  Then
//   wave 0: the head norms and RoPE of q and of the kv head's new key (the cache row
//   at pos stored by the kv head's first query head), while waves 1..3 load their
//   key rows and request the V rows of positions below pos into LDS by DMA;
//   the thread of position t <= pos: its score (in-order dot over head_dim; position
//   pos from the new key itself);
//   wave 0: the maximum, expf, the in-order sum and the probabilities;
//   all waves: the products p[t] * V[t][i] in place;
//   thread i < head_dim: value[i] = sum over t in order of the products, row pos from
//   the new value itself -- no workgroup reads a cache row that another is writing.
constexpr uint32_t kAttnOneMax = 256;

// Workgroup barrier for LDS data: waits for this wave's LDS accesses, not for its
// outstanding global loads and DMAs.
__device__ __forceinline__ void block_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The in-order sums below read their LDS operands in stages: a stage's reads are
// issued, then the previous stage's operands are declared ready (the compiler waits for
// those reads only, and the stage's additions cannot move above the declaration), and the
// additions run while the new stage's reads are in flight.  The memory clobber keeps the
// next stage's reads from being issued before the declaration.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_stage_ready(f32x4 (&r)[8]) {
    asm volatile("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
                 :
                 : "memory");
}
__device__ __forceinline__ void lds_stage_ready(float (&r)[16]) {
    asm volatile(""
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                   "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]), "+v"(r[12]), "+v"(r[13]), "+v"(r[14]),
                   "+v"(r[15])
                 :
                 : "memory");
}

__global__ __launch_bounds__(256) void k_attn_one(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, uint32_t kv_mul, float eps,
    const float* __restrict__ q_gain, const float* __restrict__ k_gain, const float* __restrict__ cosv,
    const float* __restrict__ sinv, float* __restrict__ kc, float* __restrict__ vc, uint32_t pos, uint32_t kv_dim,
    float scale, float* __restrict__ y, int* err, int code_base) {
    constexpr uint32_t HD = kAttnHD, hd4 = HD / 4, half = HD / 2;
    // V rows 0..pos-1 of the head (then their products), and 16 rows that the value sums'
    // last stage may read past row 255 (never added)
    __shared__ float4 vs4[(kAttnOneMax + 16u) * HD / 4];
    __shared__ float4 sq4[2][hd4];                 // the squares of q and k
    __shared__ float4 qk4[2][hd4];                 // q and k normalised and rotated
    __shared__ float4 p4[kAttnOneMax / 4];         // scores, then probabilities (+0 past pos)
    __shared__ uint64_t exp_tab[32];
    __shared__ int failed;
    float* p = reinterpret_cast<float*>(p4);
    const float* vs = reinterpret_cast<const float*>(vs4);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t h = blockIdx.x, t = (tid + 192u) & 255u;  // this thread's position
    const size_t head_off = (size_t)(h / kv_mul) * HD;

    float qa = 0.0f, qb = 0.0f, ka = 0.0f, kb = 0.0f, qga = 0.0f, qgb = 0.0f, kga = 0.0f, kgb = 0.0f, c = 0.0f, s = 0.0f;
    if (wave == 0) {
        qa = q[(size_t)h * HD + lane], qb = q[(size_t)h * HD + lane + half];
        ka = k[head_off + lane], kb = k[head_off + lane + half];
        qga = q_gain[lane], qgb = q_gain[lane + half], kga = k_gain[lane], kgb = k_gain[lane + half];
        c = cosv[lane], s = sinv[lane];
    }
    // this thread's key row (past position 192, wave 0 requests it after its norms)
    float4 key[hd4];
    const auto load_key = [&] {
        if (t < pos) {
            const float4* row = reinterpret_cast<const float4*>(kc + (size_t)t * kv_dim + head_off);
#pragma unroll
            for (uint32_t i = 0; i < hd4; ++i)
                key[i] = row[i];
        }
    };
    if (wave != 0) {
        load_key();
        // V rows 0..pos-1 (cache rows of earlier tokens) into LDS by DMA, behind the key
        // rows: 16-byte piece ci = 32 * row + part at byte 16 * ci of vs4; wave w > 0 issues
        // pieces (w - 1) * 64 + 192 * i + lane (pieces past the last row load row pos - 1
        // again into unused space).  They land during the head norms and the scores.
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)vs4;
        for (uint32_t c0 = (wave - 1u) * 64u; c0 < 32u * pos; c0 += 192u) {
            const uint32_t ci = c0 + lane, row = min(ci >> 5, pos - 1u);
            dma16(vc + (size_t)row * kv_dim + head_off + 4u * (ci & 31u), base + 16u * c0);
        }
    }
    if (wave == 1)  // not on the norms' path
        exp_table_fill(exp_tab, lane);
    if (wave == 0) {
        // head norms: both in-order sums over head_dim, interleaved, in every lane
        float* sq_q = reinterpret_cast<float*>(sq4[0]);
        float* sq_k = reinterpret_cast<float*>(sq4[1]);
        sq_q[lane] = qa * qa;
        sq_q[lane + half] = qb * qb;
        sq_k[lane] = ka * ka;
        sq_k[lane + half] = kb * kb;
        wave_lds_sync();
        // stages of 4 float4 of each sum, the next stage's reads in flight during the additions
        float sum_q = 0.0f, sum_k = 0.0f;
        const f32x4* sq_q4 = reinterpret_cast<const f32x4*>(sq4[0]);
        const f32x4* sq_k4 = reinterpret_cast<const f32x4*>(sq4[1]);
        f32x4 r[2][8];
#pragma unroll
        for (uint32_t c = 0; c < 4u; ++c) {
            r[0][c] = sq_q4[c];
            r[0][4u + c] = sq_k4[c];
        }
#pragma unroll
        for (uint32_t i = 0; i < hd4; i += 4u) {
            const uint32_t cur = (i / 4u) & 1u;
            if (i + 4u < hd4) {
#pragma unroll
                for (uint32_t c = 0; c < 4u; ++c) {
                    r[cur ^ 1u][c] = sq_q4[i + 4u + c];
                    r[cur ^ 1u][4u + c] = sq_k4[i + 4u + c];
                }
            }
            lds_stage_ready(r[cur]);
#pragma unroll
            for (uint32_t c = 0; c < 4u; ++c) {
                const f32x4 a = r[cur][c], b = r[cur][4u + c];
                sum_q = sum_q + a.x;
                sum_k = sum_k + b.x;
                sum_q = sum_q + a.y;
                sum_k = sum_k + b.y;
                sum_q = sum_q + a.z;
                sum_k = sum_k + b.z;
                sum_q = sum_q + a.w;
                sum_k = sum_k + b.w;
            }
        }
        const float rq = sqrtf(sum_q / (float)HD + eps), rk = sqrtf(sum_k / (float)HD + eps);
        const bool bad = !isfinite(rq) || rq == 0.0f || !isfinite(rk) || rk == 0.0f;
        if (bad) {
            if (lane == 0)
                set_error_first(err, code_base + 2);
        } else {
            // x / rms * gain, then the rotation of pair (lane, lane + 64)
            const float nqa = qa / rq * qga, nqb = qb / rq * qgb;
            const float nka = ka / rk * kga, nkb = kb / rk * kgb;
            float* qr = reinterpret_cast<float*>(qk4[0]);
            float* kr = reinterpret_cast<float*>(qk4[1]);
            qr[lane] = nqa * c - nqb * s;
            qr[lane + half] = nqa * s + nqb * c;
            const float rka = nka * c - nkb * s, rkb = nka * s + nkb * c;
            kr[lane] = rka;
            kr[lane + half] = rkb;
            if (h % kv_mul == 0) {
                kc[(size_t)pos * kv_dim + head_off + lane] = rka;
                kc[(size_t)pos * kv_dim + head_off + lane + half] = rkb;
                vc[(size_t)pos * kv_dim + head_off + lane] = v[head_off + lane];
                vc[(size_t)pos * kv_dim + head_off + lane + half] = v[head_off + lane + half];
            }
        }
        if (lane == 0)
            failed = bad;
        load_key();
    }
    block_lds_barrier();
    if (failed) {
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): no DMA still writing this workgroup's LDS
        return;                              // the whole workgroup
    }

    // the score of position t: in-order dot over head_dim (row pos: the new key)
    if (t <= pos) {
        if (t == pos) {
#pragma unroll
            for (uint32_t i = 0; i < hd4; ++i)
                key[i] = qk4[1][i];
        }
        // q in stages of 8 float4, the next stage's reads in flight during the additions
        float dot = 0.0f;
        const f32x4* q4 = reinterpret_cast<const f32x4*>(qk4[0]);
        f32x4 qs[2][8];
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c)
            qs[0][c] = q4[c];
#pragma unroll
        for (uint32_t i = 0; i < hd4; i += 8u) {
            const uint32_t cur = (i / 8u) & 1u;
            if (i + 8u < hd4) {
#pragma unroll
                for (uint32_t c = 0; c < 8u; ++c)
                    qs[cur ^ 1u][c] = q4[i + 8u + c];
            }
            lds_stage_ready(qs[cur]);
#pragma unroll
            for (uint32_t c = 0; c < 8u; ++c) {
                const f32x4 qq = qs[cur][c];
                dot = dot + qq.x * key[i + c].x;
                dot = dot + qq.y * key[i + c].y;
                dot = dot + qq.z * key[i + c].z;
                dot = dot + qq.w * key[i + c].w;
            }
        }
        const float score = dot * scale;
        if (!isfinite(score))
            set_error_first(err, code_base + 3 + 2 * (int)h);
        p[t] = score;
    }
    block_lds_barrier();

    // the maximum (order-free: finite or flagged), expf(score - max), their sum in
    // position order over a multiple of 64 terms (+0 pads), the probabilities
    if (wave == 0) {
        float mx = -INFINITY;
        for (uint32_t u = lane; u <= pos; u += 64u)
            mx = p[u] > mx ? p[u] : mx;
        const float maximum = __ockl_wfred_max_f32(mx);
        const uint32_t padded = (pos + 64u) & ~63u;
        for (uint32_t u = lane; u < padded; u += 64u)
            p[u] = u <= pos ? bnne_expf_libc(p[u] - maximum, exp_tab) : 0.0f;
        wave_lds_sync();
        const float sum = sum_lds_in_order(p, padded);
        if (!(sum > 0.0f) || !isfinite(sum)) {
            if (lane == 0)
                set_error_first(err, code_base + 4 + 2 * (int)h);
        }
        wave_lds_sync();
        for (uint32_t u = lane; u <= pos; u += 64u)
            p[u] = p[u] / sum;
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this wave's V rows are in LDS
    block_lds_barrier();                 // ... and every wave's, with the probabilities

    // the products p[t] * V[t][i] of rows t < pos, in place (each rounded once, as the
    // in-order loop forms them), by all four waves
    for (uint32_t ci = tid; ci < 32u * pos; ci += 256u) {
        const float pt = p[ci >> 5];
        float4 v4 = vs4[ci];
        v4.x = v4.x * pt;
        v4.y = v4.y * pt;
        v4.z = v4.z * pt;
        v4.w = v4.w * pt;
        vs4[ci] = v4;
    }
    block_lds_barrier();

    // value[i] = sum over t in position order of the products: stages of 16 rows, the next
    // stage's reads in flight during the current stage's additions (rows past pos - 1, at most
    // row 255 + 16, are read and not added)
    if (tid < HD) {
        const float* col = vs + tid;
        float acc = 0.0f;
        float ra[16], rb[16];
        const auto fetch = [&](float(&r)[16], uint32_t u) {
#pragma unroll
            for (uint32_t j = 0; j < 16u; ++j)
                r[j] = col[(u + j) * HD];
        };
        const auto add = [&](const float(&r)[16], uint32_t n) {
#pragma unroll
            for (uint32_t j = 0; j < 16u; ++j)
                if (j < n)
                    acc = acc + r[j];
        };
        uint32_t u = 0;
        fetch(ra, 0);
        for (; u + 32u <= pos; u += 32u) {
            fetch(rb, u + 16u);
            lds_stage_ready(ra);
            add(ra, 16u);
            fetch(ra, u + 32u);
            lds_stage_ready(rb);
            add(rb, 16u);
        }
        if (u + 16u <= pos) {
            fetch(rb, u + 16u);
            lds_stage_ready(ra);
            add(ra, 16u);
            lds_stage_ready(rb);
            add(rb, pos - u - 16u);
        } else {
            lds_stage_ready(ra);
            add(ra, pos - u);
        }
        acc = acc + p[pos] * v[head_off + tid];
        y[(size_t)h * HD + tid] = acc;
    }
}

constexpr uint32_t kPvRows = 1024;  // V slice rows in LDS per pass (128 KB)
constexpr uint32_t kPvPad = 16;     // rows / probabilities read past the end by the pipelined loop

__global__ __launch_bounds__(128) void k_attn_pv(const float* __restrict__ scores, const float* __restrict__ vc,
                                                 uint32_t kv_mul, uint32_t pos, uint32_t kv_dim, uint32_t n_ctx,
                                                 float* __restrict__ y, int* err, int code_base) {
    constexpr uint32_t HD = kAttnHD;
    constexpr uint32_t kBatch = 8;  // score loads per lane in flight
    __shared__ float4 vs4[(kPvRows + kPvPad) * kPvSlice / 4];
    __shared__ float4 p4[(kPvLdsPositions + 64u) / 4];  // probabilities (or one pass's), padded
    __shared__ uint64_t exp_tab[32];                      // the expf table: its lookups are per-lane gathers
    float* p = reinterpret_cast<float*>(p4);
    const float* vs = reinterpret_cast<const float*>(vs4);
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t h = blockIdx.x, d0 = blockIdx.y * kPvSlice;
    const size_t off = (size_t)(h / kv_mul) * HD + d0;
    const float* sc = scores + (size_t)h * n_ctx;
    const bool in_lds = pos < kPvLdsPositions;  // every probability in LDS, else per pass of V rows

    if (wave == 1) {
        // the V rows of each pass into LDS, 8 rows of 128 bytes per instruction (lane l:
        // piece l % 8 of row l / 8; rows past pos clamped), between the barriers that
        // hand the rows to wave 0 and take them back
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)vs4;
        for (uint32_t t0 = 0; t0 <= pos; t0 += kPvRows) {
            if (t0 > 0)
                __builtin_amdgcn_s_barrier();  // wave 0 is done with the previous rows
            const uint32_t rows = min(pos + 1u - t0, kPvRows);
            for (uint32_t r0 = 0; r0 < rows; r0 += 8u) {
                const uint32_t t = min(t0 + r0 + (lane >> 3), pos);
                dma16(vc + (size_t)t * kv_dim + off + 4u * (lane & 7u), base + r0 * kPvSlice * 4u);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __builtin_amdgcn_s_barrier();         // the rows are in LDS
        }
        return;
    }

    // wave 0: the scores into LDS when they fit, and their maximum (order-free: finite
    // or flagged)
    if (lane < 32u)
        exp_tab[lane] = kExp2Table[lane];
    float mx = -INFINITY;
    for (uint32_t t0 = 0; t0 <= pos; t0 += 64u * kBatch) {
        float x[kBatch];
#pragma unroll
        for (uint32_t c = 0; c < kBatch; ++c)
            x[c] = sc[min(t0 + 64u * c + lane, pos)];
#pragma unroll
        for (uint32_t c = 0; c < kBatch; ++c) {
            const uint32_t t = t0 + 64u * c + lane;
            if (t <= pos) {
                if (in_lds)
                    p[t] = x[c];
                mx = x[c] > mx ? x[c] : mx;
            }
        }
    }
    const float maximum = __ockl_wfred_max_f32(mx);
    wave_lds_sync();

    // expf(score - max) and their sum in position order; +0 pads the terms to a
    // multiple of 64 (adding +0 to this sum of non-negative terms changes nothing)
    float sum = 0.0f;
    if (in_lds) {
        const uint32_t padded = (pos + 64u) & ~63u;
        for (uint32_t t = lane; t < padded; t += 64u)
            p[t] = t <= pos ? bnne_expf_libc(p[t] - maximum, exp_tab) : 0.0f;
        wave_lds_sync();
        sum = sum_lds_in_order(p, padded);
    } else {
        for (uint32_t t0 = 0; t0 <= pos; t0 += 64u) {
            p[lane] = t0 + lane <= pos ? bnne_expf_libc(sc[t0 + lane] - maximum, exp_tab) : 0.0f;
            wave_lds_sync();
            sum = sum_lds_in_order(p, 64u, sum);
            wave_lds_sync();
        }
    }
    // a failed softmax is flagged; the wave still runs its barriers (y is then unused)
    if (!(sum > 0.0f) || !isfinite(sum)) {
        if (lane == 0)
            set_error_first(err, code_base + 4 + 2 * (int)h);
    }
    if (in_lds) {
        for (uint32_t t = lane; t <= pos; t += 64u)
            p[t] = p[t] / sum;
    }

    // value[i] = sum over t in order of p[t] * V[t][i] (lane i < 32 of the slice) per
    // pass of V rows; the next 8 rows' reads are issued before the current 8 are added
    float acc = 0.0f;
    for (uint32_t t0 = 0; t0 <= pos; t0 += kPvRows) {
        const uint32_t n = min(kPvRows, pos + 1u - t0);
        if (t0 > 0)
            __builtin_amdgcn_s_barrier();  // the previous rows are read: wave 1 may reload
        if (!in_lds) {                     // this pass's probabilities
            for (uint32_t r = lane; r < n; r += 64u)
                p[r] = bnne_expf_libc(sc[t0 + r] - maximum, exp_tab) / sum;
        }
        wave_lds_sync();
        __builtin_amdgcn_s_barrier();  // the rows are in LDS
        if (lane < kPvSlice) {
            const float4* pp = reinterpret_cast<const float4*>(in_lds ? p + t0 : p);
            const float* vl = vs + lane;
            float4 pa0 = pp[0], pa1 = pp[1];
            float va[8];
#pragma unroll
            for (uint32_t c = 0; c < 8; ++c)
                va[c] = vl[c * kPvSlice];
            uint32_t r = 0;
#pragma unroll 2
            for (; r + 8u <= n; r += 8u) {
                const float4 pb0 = pp[(r + 8u) / 4u], pb1 = pp[(r + 8u) / 4u + 1u];
                float vb[8];
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c)
                    vb[c] = vl[(r + 8u + c) * kPvSlice];
                acc = acc + pa0.x * va[0];
                acc = acc + pa0.y * va[1];
                acc = acc + pa0.z * va[2];
                acc = acc + pa0.w * va[3];
                acc = acc + pa1.x * va[4];
                acc = acc + pa1.y * va[5];
                acc = acc + pa1.z * va[6];
                acc = acc + pa1.w * va[7];
                pa0 = pb0;
                pa1 = pb1;
#pragma unroll
                for (uint32_t c = 0; c < 8; ++c)
                    va[c] = vb[c];
            }
            const float pr[8] = {pa0.x, pa0.y, pa0.z, pa0.w, pa1.x, pa1.y, pa1.z, pa1.w};
#pragma unroll
            for (uint32_t c = 0; c < 7; ++c)
                if (r + c < n)
                    acc = acc + pr[c] * va[c];
        }
    }
    if (lane < kPvSlice)
        y[(size_t)h * HD + d0 + lane] = acc;
}

// gate = gate / (1 + exp(-gate)) * up (qwen3.c:491-495).
__global__ __launch_bounds__(256) void k_silu_mul(float* __restrict__ gate, const float* __restrict__ up, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n)
        return;
    const float g = gate[i];
    const float silu = g / (1.0f + expf_libc(-g));
    gate[i] = silu * up[i];
}

}  // namespace

struct Resident {
    BNN_Device dev;
    hipStream_t stream;
    int ordinal;
    uint32_t C, H, Hk, HD, FF, L, V, kv_dim, n_ctx;
    float eps;
    // activations that linear layers read or write: accelerator buffers
    BNN_Buffer b_norm, b_q, b_k, b_v, b_y, b_o, b_gate, b_up, b_h, b_logits;
    float *norm, *q, *k, *v, *y, *o, *gate, *up, *h;  // h: SiLU(gate) * up (fused step)
    // everything else: this engine's device memory
    float *x, *x2, *kc, *vc, *scores, *gains, *rope_cos, *rope_sin;
    uint8_t* emb_bits;
    uint16_t* emb_scales;
    int* err;
    float* logits_dev;  // the lm_head's output (b_logits)
    // pinned host memory: V floats of logits, then the error word; both are copied back
    // on the stream behind a step's last launch, so the host waits once per step
    float* pinned;
    // greedy runs: two argmax keys (steps alternate), the logits-check flag, then the
    // tokens [n_ctx] (device); the tokens and the flag come back into pinned_tokens
    // [n_ctx + 1]
    unsigned long long* keys;
    int* logit_bad;
    int32_t* tokens_dev;
    int32_t* pinned_tokens;
    // fused: every linear layer is a fused batch (its input row produced and
    // quantised inside its one launch), else prepared batches plus this engine's
    // norm and SiLU kernels (models wider than a fused batch takes)
    bool allow_fused, fused;
    BNNX_Batch *qkv, *attn_out, *gate_up, *down;
    BNNX_Batch lm_head;
    const SignLinear** lin;  // [7 * L + 1]: per layer q, k, v, o, gate, up, down; then lm_head
    uint64_t jobs_per_token, macs_per_token, lm_jobs, lm_macs;
};

namespace {

BNNE_Status hip_error(hipError_t e, const char* what) {
    (void)hipGetLastError();
    return complain(e == hipErrorOutOfMemory ? BNNE_ENOMEM : BNNE_EIO, "%s: %s", what, hipGetErrorString(e));
}

BNNE_Status alloc_buffer(Resident* r, size_t floats, BNN_Buffer* b, float** ptr) {
    BNNE_Status st = accel_status(BNN_BufferAlloc(r->dev, floats * sizeof(float), b), "BNN_BufferAlloc");
    if (st == BNNE_OK)
        st = accel_status(BNNX_BufferDevicePointer(*b, reinterpret_cast<void**>(ptr)), "BNNX_BufferDevicePointer");
    return st;
}

template <class T>
BNNE_Status upload(T** dst, const void* src, size_t bytes) {
    hipError_t e = hipMalloc(reinterpret_cast<void**>(dst), bytes);
    if (e == hipSuccess && src)
        e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? BNNE_OK : hip_error(e, "device upload");
}

void add_jobs(const SignLinear* l, BNN_Buffer in, BNN_Buffer out, BNN_Job* jobs, uint32_t* n, uint64_t* macs) {
    for (uint32_t c = 0; c < (uint32_t)l->shards().size(); ++c) {
        BNN_Job& j = jobs[(*n)++];
        j = BNN_Job{};
        j.operation = BNN_OP_GEMV_F32;
        j.matrix = l->shards()[c].matrix;
        j.input.buffer = in;
        j.input.type = BNN_TYPE_F32;
        j.output.buffer = out;
        j.output.type = BNN_TYPE_F32;
        j.output.offset = (size_t)l->shards()[c].first * sizeof(float);
        j.rows = 1;
    }
    *macs += (uint64_t)l->in() * l->out();
}

BNNE_Status make_batch(Resident* r, std::initializer_list<std::pair<const SignLinear*, BNN_Buffer>> parts, BNN_Buffer in,
                       BNNX_Batch* out, uint64_t* jobs_total, uint64_t* macs) {
    uint32_t count = 0;
    for (const auto& p : parts)
        count += (uint32_t)p.first->shards().size();
    BNN_Job* jobs = static_cast<BNN_Job*>(std::calloc(count, sizeof(BNN_Job)));
    if (!jobs)
        return complain(BNNE_ENOMEM, "out of memory");
    uint32_t n = 0;
    for (const auto& p : parts)
        add_jobs(p.first, in, p.second, jobs, &n, macs);
    const BNNE_Status st = accel_status(BNNX_BatchCreate(r->dev, jobs, n, out), "BNNX_BatchCreate");
    std::free(jobs);
    *jobs_total += n;
    return st;
}

BNNE_Status make_fused(Resident* r, std::initializer_list<std::pair<const SignLinear*, BNN_Buffer>> parts, BNN_Buffer in,
                       const BNNX_PreOp& pre, BNNX_Batch* out, uint64_t* jobs_total, uint64_t* macs,
                       BNN_Status* refused, const BNNX_PostOp* post = nullptr) {
    uint32_t count = 0;
    for (const auto& p : parts)
        count += (uint32_t)p.first->shards().size();
    BNN_Job* jobs = static_cast<BNN_Job*>(std::calloc(count, sizeof(BNN_Job)));
    if (!jobs)
        return complain(BNNE_ENOMEM, "out of memory");
    uint32_t n = 0;
    for (const auto& p : parts)
        add_jobs(p.first, in, p.second, jobs, &n, macs);
    *refused = BNNX_BatchCreateFusedPost(r->dev, jobs, n, &pre, post, out);
    std::free(jobs);
    *jobs_total += n;
    return *refused == BNN_OK ? BNNE_OK : accel_status(*refused, "BNNX_BatchCreateFusedPost");
}

// Error codes of the fused step (see set_error_first).
int code_span(const Resident* r) { return 4 + 2 * (int)r->H; }

}  // namespace

namespace {

void destroy_batches(Resident* r) {
    for (uint32_t l = 0; l < r->L; ++l) {
        if (r->qkv) {
            BNNX_BatchDestroy(r->qkv[l]);
            r->qkv[l] = nullptr;
        }
        if (r->attn_out) {
            BNNX_BatchDestroy(r->attn_out[l]);
            r->attn_out[l] = nullptr;
        }
        if (r->gate_up) {
            BNNX_BatchDestroy(r->gate_up[l]);
            r->gate_up[l] = nullptr;
        }
        if (r->down) {
            BNNX_BatchDestroy(r->down[l]);
            r->down[l] = nullptr;
        }
    }
    BNNX_BatchDestroy(r->lm_head);
    r->lm_head = nullptr;
}

// Fused batches of every layer and of the lm_head:
//   qkv:    RMSNorm(x [+ o]) with attn_norm, the sum stored to x2   -> q, k, v
//   o:      the attention output row y                               -> o
//   gate/up RMSNorm(x2 + o) with ffn_norm, the sum stored to x       -> gate, up, h = SiLU(gate) * up
//   down:   the row h                                                -> o
//   lm_head RMSNorm(x + o) with final_norm                           -> logits
// so the residual stream alternates between x and x2 within a layer and is in x
// (plus the down output in o) between layers.  *refused is the backend's
// status of the first batch it refused.
BNNE_Status build_fused(Resident* r, BNN_Status* refused) {
    r->jobs_per_token = r->macs_per_token = r->lm_jobs = r->lm_macs = 0;
    *refused = BNN_OK;
    const uint32_t C = r->C;
    const float* attn_norm = r->gains;
    const float* ffn_norm = r->gains + (size_t)r->L * C;
    const float* final_norm = r->gains + 2 * (size_t)r->L * C + 2 * (size_t)r->L * r->HD;
    BNNE_Status st = BNNE_OK;
    for (uint32_t l = 0; st == BNNE_OK && l < r->L; ++l) {
        const SignLinear* const* p = r->lin + 7 * (size_t)l;
        const int base = (int)l * code_span(r);
        BNNX_PreOp pre{};
        pre.kind = BNNX_PRE_RMSNORM;
        pre.width = C;
        pre.a = r->x;
        pre.b = l ? r->o : nullptr;
        pre.gain = attn_norm + (size_t)l * C;
        pre.a_out = r->x2;
        pre.eps = r->eps;
        pre.err = r->err;
        pre.err_code = base + 1;
        st = make_fused(r, {{p[0], r->b_q}, {p[1], r->b_k}, {p[2], r->b_v}}, r->b_norm, pre, &r->qkv[l],
                        &r->jobs_per_token, &r->macs_per_token, refused);
        if (st == BNNE_OK) {
            BNNX_PreOp row{};
            row.kind = BNNX_PRE_ROW;
            row.width = C;
            st = make_fused(r, {{p[3], r->b_o}}, r->b_y, row, &r->attn_out[l], &r->jobs_per_token, &r->macs_per_token,
                            refused);
        }
        if (st == BNNE_OK) {
            pre.a = r->x2;
            pre.b = r->o;
            pre.gain = ffn_norm + (size_t)l * C;
            pre.a_out = r->x;
            pre.err_code = base + 3 + 2 * (int)r->H;
            // the chunks of gate and of up pair up (equal widths): SiLU(gate) * up -> h
            BNNX_PostOp silu{};
            silu.kind = BNNX_POST_SILU_MUL;
            silu.out = r->h;
            st = make_fused(r, {{p[4], r->b_gate}, {p[5], r->b_up}}, r->b_norm, pre, &r->gate_up[l], &r->jobs_per_token,
                            &r->macs_per_token, refused, &silu);
        }
        if (st == BNNE_OK) {
            BNNX_PreOp row{};
            row.kind = BNNX_PRE_ROW;
            row.width = r->FF;
            st = make_fused(r, {{p[6], r->b_o}}, r->b_h, row, &r->down[l], &r->jobs_per_token, &r->macs_per_token,
                            refused);
        }
    }
    if (st == BNNE_OK) {
        BNNX_PreOp pre{};
        pre.kind = BNNX_PRE_RMSNORM;
        pre.width = C;
        pre.a = r->x;
        pre.b = r->o;
        pre.gain = final_norm;
        pre.eps = r->eps;
        pre.err = r->err;
        pre.err_code = (int)r->L * code_span(r) + 1;
        st = make_fused(r, {{r->lin[7 * (size_t)r->L], r->b_logits}}, r->b_norm, pre, &r->lm_head, &r->lm_jobs,
                        &r->lm_macs, refused);
    }
    return st;
}

// The prepared batches of every layer and of the lm_head (fused where the backend
// takes them).  Rebuilt when the backend reports them stale (some other matrix or
// buffer of the device was destroyed since; this context's own objects are still
// alive).
BNNE_Status build_unfused(Resident* r);
BNNE_Status build_batches(Resident* r) {
    r->fused = false;
    if (!r->allow_fused || r->HD != kAttnHD)  // the fused step's attention kernel is built for one head_dim
        return build_unfused(r);
    BNN_Status accel = BNN_OK;
    BNNE_Status st = build_fused(r, &accel);
    r->fused = st == BNNE_OK;
    if (st == BNNE_OK || accel != BNN_ENOTSUP)
        return st;
    destroy_batches(r);
    return build_unfused(r);
}

BNNE_Status build_unfused(Resident* r) {
    r->jobs_per_token = r->macs_per_token = r->lm_jobs = r->lm_macs = 0;
    BNNE_Status st = BNNE_OK;
    for (uint32_t l = 0; st == BNNE_OK && l < r->L; ++l) {
        const SignLinear* const* p = r->lin + 7 * (size_t)l;
        st = make_batch(r, {{p[0], r->b_q}, {p[1], r->b_k}, {p[2], r->b_v}}, r->b_norm, &r->qkv[l], &r->jobs_per_token,
                        &r->macs_per_token);
        if (st == BNNE_OK)
            st = make_batch(r, {{p[3], r->b_o}}, r->b_y, &r->attn_out[l], &r->jobs_per_token, &r->macs_per_token);
        if (st == BNNE_OK)
            st = make_batch(r, {{p[4], r->b_gate}, {p[5], r->b_up}}, r->b_norm, &r->gate_up[l], &r->jobs_per_token,
                            &r->macs_per_token);
        if (st == BNNE_OK)
            st = make_batch(r, {{p[6], r->b_o}}, r->b_gate, &r->down[l], &r->jobs_per_token, &r->macs_per_token);
    }
    if (st == BNNE_OK)
        st = make_batch(r, {{r->lin[7 * (size_t)r->L], r->b_logits}}, r->b_norm, &r->lm_head, &r->lm_jobs, &r->lm_macs);
    return st;
}

}  // namespace

bool resident_fused(const Resident* r) { return r->fused; }

BNNE_Status resident_create(bnne_context* c, const ResidentModel& m, bool fused, Resident** out) {
    *out = nullptr;
    if (m.HD > kMaxHeadDim || m.HD % 4u != 0 || m.C > kMaxNormWidth)
        return complain(BNNE_ENOTSUP, "device-resident decode supports head_dim <= %u (a multiple of 4) and width <= %u",
                     kMaxHeadDim, kMaxNormWidth);
    Resident* r = static_cast<Resident*>(std::calloc(1, sizeof(Resident)));
    if (!r)
        return complain(BNNE_ENOMEM, "out of memory");
    r->dev = c->model->device;
    r->C = m.C, r->H = m.H, r->Hk = m.Hk, r->HD = m.HD, r->FF = m.FF, r->L = m.L, r->V = m.V;
    r->kv_dim = m.kv_dim, r->n_ctx = m.n_ctx, r->eps = m.eps;
    r->allow_fused = fused;
    BNNE_Status st = accel_status(BNNX_DeviceStream(r->dev, reinterpret_cast<void**>(&r->stream)), "BNNX_DeviceStream");
    hipError_t e = hipSuccess;
    if (st == BNNE_OK) {
        e = hipStreamGetDevice(r->stream, &r->ordinal);
        if (e == hipSuccess)
            e = hipSetDevice(r->ordinal);
        if (e != hipSuccess)
            st = hip_error(e, "device of the accelerator stream");
    }
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.C, &r->b_norm, &r->norm);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.C, &r->b_q, &r->q);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.kv_dim, &r->b_k, &r->k);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.kv_dim, &r->b_v, &r->v);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.C, &r->b_y, &r->y);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.C, &r->b_o, &r->o);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.FF, &r->b_gate, &r->gate);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.FF, &r->b_up, &r->up);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.FF, &r->b_h, &r->h);
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.V, &r->b_logits, &r->logits_dev);
    const size_t cache = (size_t)m.L * m.n_ctx * m.kv_dim * sizeof(float);
    if (st == BNNE_OK)
        st = upload(&r->x, nullptr, (size_t)m.C * sizeof(float));
    if (st == BNNE_OK)
        st = upload(&r->x2, nullptr, (size_t)m.C * sizeof(float));
    if (st == BNNE_OK)
        st = upload(&r->kc, nullptr, cache);
    if (st == BNNE_OK)
        st = upload(&r->vc, nullptr, cache);
    if (st == BNNE_OK)
        st = upload(&r->scores, nullptr, (size_t)m.H * m.n_ctx * sizeof(float));
    if (st == BNNE_OK) {
        // gains: attn_norm[L][C] | ffn_norm[L][C] | q_norm[L][HD] | k_norm[L][HD] | final[C]
        const size_t n = 2 * (size_t)m.L * m.C + 2 * (size_t)m.L * m.HD + m.C;
        float* host = static_cast<float*>(std::malloc(n * sizeof(float)));
        if (!host) {
            st = complain(BNNE_ENOMEM, "out of memory");
        } else {
            float* p = host;
            for (uint32_t l = 0; l < m.L; ++l, p += m.C)
                std::memcpy(p, m.attn_norm[l], m.C * sizeof(float));
            for (uint32_t l = 0; l < m.L; ++l, p += m.C)
                std::memcpy(p, m.ffn_norm[l], m.C * sizeof(float));
            for (uint32_t l = 0; l < m.L; ++l, p += m.HD)
                std::memcpy(p, m.q_norm[l], m.HD * sizeof(float));
            for (uint32_t l = 0; l < m.L; ++l, p += m.HD)
                std::memcpy(p, m.k_norm[l], m.HD * sizeof(float));
            std::memcpy(p, m.final_norm, m.C * sizeof(float));
            st = upload(&r->gains, host, n * sizeof(float));
            std::free(host);
        }
    }
    if (st == BNNE_OK)
        st = upload(&r->emb_bits, m.emb_bits, (size_t)m.V * (m.C / 8u));
    if (st == BNNE_OK)
        st = upload(&r->emb_scales, m.emb_scales, (size_t)m.V * (m.C / 128u) * sizeof(uint16_t));
    if (st == BNNE_OK)
        st = upload(&r->rope_cos, m.rope_cos, (size_t)m.n_ctx * (m.HD / 2u) * sizeof(float));
    if (st == BNNE_OK)
        st = upload(&r->rope_sin, m.rope_sin, (size_t)m.n_ctx * (m.HD / 2u) * sizeof(float));
    if (st == BNNE_OK) {
        st = upload(&r->err, nullptr, sizeof(int));
        if (st == BNNE_OK && (e = hipMemset(r->err, 0, sizeof(int))) != hipSuccess)
            st = hip_error(e, "hipMemset");
    }
    if (st == BNNE_OK &&
        (e = hipHostMalloc(reinterpret_cast<void**>(&r->pinned), ((size_t)m.V + 1u) * sizeof(float))) != hipSuccess) {
        r->pinned = nullptr;
        st = hip_error(e, "hipHostMalloc");
    }
    if (st == BNNE_OK) {
        st = upload(&r->keys, nullptr, 2 * sizeof(unsigned long long) + sizeof(int) * (2u + (size_t)m.n_ctx));
        if (st == BNNE_OK) {
            r->logit_bad = reinterpret_cast<int*>(r->keys + 2);
            r->tokens_dev = reinterpret_cast<int32_t*>(r->logit_bad + 2);
            if ((e = hipMemset(r->logit_bad, 0, sizeof(int))) != hipSuccess)
                st = hip_error(e, "hipMemset");
        }
    }
    if (st == BNNE_OK && (e = hipHostMalloc(reinterpret_cast<void**>(&r->pinned_tokens),
                                            ((size_t)m.n_ctx + 1u) * sizeof(int32_t))) != hipSuccess) {
        r->pinned_tokens = nullptr;
        st = hip_error(e, "hipHostMalloc");
    }
    if (st == BNNE_OK) {
        r->qkv = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->attn_out = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->gate_up = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->down = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->lin = static_cast<const SignLinear**>(std::calloc(7 * (size_t)m.L + 1, sizeof(SignLinear*)));
        if (!r->qkv || !r->attn_out || !r->gate_up || !r->down || !r->lin)
            st = complain(BNNE_ENOMEM, "out of memory");
    }
    if (st == BNNE_OK) {
        for (uint32_t l = 0; l < m.L; ++l) {
            const SignLinear** p = r->lin + 7 * (size_t)l;
            p[0] = m.wq[l], p[1] = m.wk[l], p[2] = m.wv[l], p[3] = m.wo[l];
            p[4] = m.gate[l], p[5] = m.up[l], p[6] = m.down[l];
        }
        r->lin[7 * (size_t)m.L] = m.lm_head;
        st = build_batches(r);
    }
    if (st != BNNE_OK) {
        resident_free(r);
        return st;
    }
    *out = r;
    return BNNE_OK;
}

void resident_free(Resident* r) {
    if (!r)
        return;
    if (r->stream)
        (void)hipStreamSynchronize(r->stream);
    destroy_batches(r);
    std::free(r->qkv);
    std::free(r->attn_out);
    std::free(r->gate_up);
    std::free(r->down);
    std::free(r->lin);
    for (BNN_Buffer b : {r->b_norm, r->b_q, r->b_k, r->b_v, r->b_y, r->b_o, r->b_gate, r->b_up, r->b_h, r->b_logits})
        BNN_BufferFree(b);
    for (void* p : {(void*)r->x, (void*)r->x2, (void*)r->kc, (void*)r->vc, (void*)r->scores, (void*)r->gains, (void*)r->rope_cos,
                    (void*)r->rope_sin, (void*)r->emb_bits, (void*)r->emb_scales, (void*)r->err, (void*)r->keys})
        if (p)
            (void)hipFree(p);
    if (r->pinned)
        (void)hipHostFree(r->pinned);
    if (r->pinned_tokens)
        (void)hipHostFree(r->pinned_tokens);
    std::free(r);
}

namespace {

// Stale prepared batches (any matrix or buffer of the device destroyed since: another
// context, another model) are rebuilt; nothing can be destroyed during a step, so
// checking one batch decides for all of them.
BNNE_Status ready_batches(Resident* r) {
    const BNN_Status valid = BNNX_BatchCheck(r->qkv[0]);
    if (valid == BNN_EINVAL) {
        destroy_batches(r);
        return build_batches(r);
    }
    return valid == BNN_OK ? BNNE_OK : accel_status(valid, "BNNX_BatchCheck");
}

// The launches of one token at position pos: its embedding row (of `token`, or of the
// token a greedy step's argmax left in *key_in, recorded in *tok_out, with *key_reset
// cleared), the layers, and the lm_head when `head`.  `first`: the call's first token,
// whose embedding launch clears the error word and the logits flag.
BNNE_Status enqueue_token(Resident* r, uint32_t pos, uint32_t token, const unsigned long long* key_in,
                          int32_t* tok_out, unsigned long long* key_reset, bool head, bool first) {
    const uint32_t C = r->C, HD = r->HD, half = HD / 2u;
    const float scale = 1.0f / sqrtf((float)HD);
    const float* attn_norm = r->gains;
    const float* ffn_norm = r->gains + (size_t)r->L * C;
    const float* q_norm = r->gains + 2 * (size_t)r->L * C;
    const float* k_norm = q_norm + (size_t)r->L * HD;
    const float* final_norm = k_norm + (size_t)r->L * HD;
    const size_t norm_lds = (size_t)C * sizeof(float);
    BNNE_Status st = BNNE_OK;
    auto launch = [&](BNNX_Batch b) {
        if (st == BNNE_OK)
            st = accel_status(BNNX_BatchLaunch(b), "BNNX_BatchLaunch");
    };
    hipLaunchKernelGGL(k_embed, dim3((C + 255u) / 256u), dim3(256), 0, r->stream, token, key_in, tok_out, key_reset,
                       first ? r->err : nullptr, first ? r->logit_bad : nullptr, r->emb_bits, r->emb_scales, C, r->x);
    for (uint32_t l = 0; l < r->L && st == BNNE_OK && r->fused; ++l) {
        const size_t cache_layer = (size_t)l * r->n_ctx * r->kv_dim;
        launch(r->qkv[l]);
        if (pos < kAttnOneMax) {
            hipLaunchKernelGGL(k_attn_one, dim3(r->H), dim3(256), 0, r->stream, r->q, r->k, r->v, r->H / r->Hk,
                               r->eps, q_norm + (size_t)l * HD, k_norm + (size_t)l * HD,
                               r->rope_cos + (size_t)pos * half, r->rope_sin + (size_t)pos * half,
                               r->kc + cache_layer, r->vc + cache_layer, pos, r->kv_dim, scale, r->y, r->err,
                               (int)l * code_span(r));
        } else {
            hipLaunchKernelGGL(k_attn_scores, dim3(r->H, pos / kScoreBlock + 1u), dim3(kScoreBlock), 0,
                               r->stream, r->q, r->k, r->v, r->H / r->Hk, r->eps, q_norm + (size_t)l * HD,
                               k_norm + (size_t)l * HD, r->rope_cos + (size_t)pos * half,
                               r->rope_sin + (size_t)pos * half, r->kc + cache_layer, r->vc + cache_layer, pos,
                               r->kv_dim, scale, r->scores, r->n_ctx, r->err, (int)l * code_span(r));
            hipLaunchKernelGGL(k_attn_pv, dim3(r->H, HD / kPvSlice), dim3(128), 0, r->stream, r->scores,
                               r->vc + cache_layer, r->H / r->Hk, pos, r->kv_dim, r->n_ctx, r->y, r->err,
                               (int)l * code_span(r));
        }
        launch(r->attn_out[l]);
        launch(r->gate_up[l]);
        launch(r->down[l]);
    }
    for (uint32_t l = 0; l < r->L && st == BNNE_OK && !r->fused; ++l) {
        const size_t cache_layer = (size_t)l * r->n_ctx * r->kv_dim;
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), norm_lds, r->stream, r->x, l ? r->o : nullptr, C,
                           r->eps, attn_norm + (size_t)l * C, r->norm, r->err);
        launch(r->qkv[l]);
        hipLaunchKernelGGL(k_head_norm_rope, dim3(r->H + r->Hk), dim3(64), 0, r->stream, r->q, r->k, r->v, r->H,
                           HD, r->eps, q_norm + (size_t)l * HD, k_norm + (size_t)l * HD,
                           r->rope_cos + (size_t)pos * half, r->rope_sin + (size_t)pos * half,
                           r->kc + cache_layer + (size_t)pos * r->kv_dim,
                           r->vc + cache_layer + (size_t)pos * r->kv_dim, r->err);
        hipLaunchKernelGGL(k_attention, dim3(r->H), dim3(256), 0, r->stream, r->q, r->kc + cache_layer,
                           r->vc + cache_layer, pos, r->kv_dim, HD, r->H / r->Hk, scale, r->scores, r->n_ctx,
                           r->y, r->err);
        launch(r->attn_out[l]);
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), norm_lds, r->stream, r->x, r->o, C, r->eps,
                           ffn_norm + (size_t)l * C, r->norm, r->err);
        launch(r->gate_up[l]);
        hipLaunchKernelGGL(k_silu_mul, dim3((r->FF + 255u) / 256u), dim3(256), 0, r->stream, r->gate, r->up, r->FF);
        launch(r->down[l]);
    }
    if (head && st == BNNE_OK && !r->fused)
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), norm_lds, r->stream, r->x, r->o, C, r->eps,
                           final_norm, r->norm, r->err);
    if (head)
        launch(r->lm_head);
    return st;
}

// The step's error word (read back into pinned memory), cleared on the device when set,
// as the engine's status.
BNNE_Status step_error(Resident* r, int err) {
    hipError_t e;
    if (err != kErrNone && (e = hipMemset(r->err, 0, sizeof(int))) != hipSuccess)
        return hip_error(e, "error word");
    int kind = err;
    if (r->fused && err != kErrNone) {
        const int p = err % code_span(r);  // 1: attention norm, 2: head norms, 3 + 2H: FFN norm
        kind = p == 1 || p == 2 || p == code_span(r) - 1 ? kErrNorm : ((p - 3) % 2 == 0 ? kErrScore : kErrSoftmax);
    }
    if (kind == kErrNorm)
        return complain(BNNE_ECOMPUTE, "RMSNorm divisor is zero or not finite");
    if (kind == kErrScore)
        return complain(BNNE_ECOMPUTE, "non-finite attention score");
    if (kind == kErrSoftmax)
        return complain(BNNE_ECOMPUTE, "softmax normaliser is zero or not finite");
    return BNNE_OK;
}

}  // namespace

BNNE_Status resident_step(bnne_context* c, Resident* r, const int32_t* tokens, uint32_t n, uint32_t pos0,
                          float* logits) {
    const bool stats = c->params.enable_stats != 0;
    hipError_t e = hipSetDevice(r->ordinal);
    if (e != hipSuccess)
        return hip_error(e, "hipSetDevice");
    BNNE_Status st = ready_batches(r);
    for (uint32_t i = 0; i < n && st == BNNE_OK; ++i)
        st = enqueue_token(r, pos0 + i, (uint32_t)tokens[i], nullptr, nullptr, nullptr, logits && i + 1 == n, i == 0);
    e = hipGetLastError();
    // the error word and the logits come back behind the last launch, into pinned memory
    int* const err_host = reinterpret_cast<int*>(r->pinned + r->V);
    if (st == BNNE_OK && e == hipSuccess)
        e = hipMemcpyAsync(err_host, r->err, sizeof(int), hipMemcpyDeviceToHost, r->stream);
    if (st == BNNE_OK && e == hipSuccess && logits)
        e = hipMemcpyAsync(r->pinned, r->logits_dev, (size_t)r->V * sizeof(float), hipMemcpyDeviceToHost, r->stream);
    const uint64_t t1 = stats ? clock_ns() : 0;
    const BNN_Status sync = BNNX_DeviceSynchronize(r->dev);
    const uint64_t t2 = stats ? clock_ns() : 0;
    if (st != BNNE_OK)
        return st;
    if (e != hipSuccess)
        return hip_error(e, "kernel launch");
    if (sync == BNN_EIO)
        return accel_status(sync, "BNN_Execute");
    st = step_error(r, *static_cast<volatile int*>(err_host));
    if (st != BNNE_OK)
        return st;
    st = accel_status(sync, "BNN_Execute");
    if (st != BNNE_OK)
        return st;
    if (logits) {
        // to the caller's buffer, checking on the way that every logit is finite
        // (BNNE_Decode's own check, made here in the same pass)
        // (the count and pointers in locals, restrict-qualified: the stores then cannot alias
        // them and the loop runs as vector copies -- a per-element reload of the count had kept
        // it scalar, tens of microseconds per token)
        const uint32_t V = r->V;
        const uint32_t* __restrict__ src = reinterpret_cast<const uint32_t*>(r->pinned);
        uint32_t* __restrict__ dst = reinterpret_cast<uint32_t*>(logits);
        uint32_t bad = 0;
        for (uint32_t i = 0; i < V; ++i) {
            const uint32_t u = src[i];
            dst[i] = u;
            bad |= (uint32_t)((u & 0x7F800000u) == 0x7F800000u);
        }
        if (bad)
            return complain(BNNE_ECOMPUTE, "the logits hold a NaN or infinity");
        c->logits_checked = true;
    }
    if (stats) {
        const uint64_t t3 = clock_ns();
        c->stats.execute_ns += t2 - t1;
        c->stats.transfer_ns += t3 - t2;
        const uint64_t lm = logits ? 1 : 0;
        c->stats.device_calls += n * r->jobs_per_token + lm * r->lm_jobs;
        c->stats.bytes_read += lm * r->V * sizeof(float);
        c->stats.logical_macs += n * r->macs_per_token + lm * r->lm_macs;
        c->stats.executed_macs += n * r->macs_per_token + lm * r->lm_macs;
    }
    return BNNE_OK;
}

BNNE_Status resident_greedy(bnne_context* c, Resident* r, int32_t token, uint32_t n, uint32_t pos0,
                            int32_t* out_tokens) {
    const bool stats = c->params.enable_stats != 0;
    hipError_t e = hipSetDevice(r->ordinal);
    if (e != hipSuccess)
        return hip_error(e, "hipSetDevice");
    BNNE_Status st = ready_batches(r);
    // step i embeds the token step i - 1's argmax left in keys[(i - 1) % 2] and clears
    // keys[i % 2] for its own argmax; nothing returns to the host until the last step
    const uint32_t argmax_grid = std::min<uint32_t>((r->V + 4u * kArgmaxThreads - 1u) / (4u * kArgmaxThreads), 1024u);
    for (uint32_t i = 0; i < n && st == BNNE_OK; ++i) {
        st = enqueue_token(r, pos0 + i, (uint32_t)token, i ? r->keys + ((i - 1u) & 1u) : nullptr,
                           i ? r->tokens_dev + (i - 1u) : nullptr, r->keys + (i & 1u), true, i == 0);
        if (st == BNNE_OK)
            hipLaunchKernelGGL(k_argmax, dim3(argmax_grid), dim3(kArgmaxThreads), 0, r->stream, r->logits_dev, r->V,
                               r->keys + (i & 1u), r->logit_bad);
    }
    if (st == BNNE_OK)
        hipLaunchKernelGGL(k_key_token, dim3(1), dim3(64), 0, r->stream, r->keys + ((n - 1u) & 1u),
                           r->tokens_dev + (n - 1u));
    e = hipGetLastError();
    // the error word, the logits flag and the tokens come back behind the last launch
    int* const err_host = reinterpret_cast<int*>(r->pinned + r->V);
    if (st == BNNE_OK && e == hipSuccess)
        e = hipMemcpyAsync(err_host, r->err, sizeof(int), hipMemcpyDeviceToHost, r->stream);
    if (st == BNNE_OK && e == hipSuccess)
        e = hipMemcpyAsync(r->pinned_tokens + n, r->logit_bad, sizeof(int), hipMemcpyDeviceToHost, r->stream);
    if (st == BNNE_OK && e == hipSuccess)
        e = hipMemcpyAsync(r->pinned_tokens, r->tokens_dev, (size_t)n * sizeof(int32_t), hipMemcpyDeviceToHost,
                           r->stream);
    const uint64_t t1 = stats ? clock_ns() : 0;
    const BNN_Status sync = BNNX_DeviceSynchronize(r->dev);
    const uint64_t t2 = stats ? clock_ns() : 0;
    if (st != BNNE_OK)
        return st;
    if (e != hipSuccess)
        return hip_error(e, "kernel launch");
    if (sync == BNN_EIO)
        return accel_status(sync, "BNN_Execute");
    st = step_error(r, *static_cast<volatile int*>(err_host));
    if (st != BNNE_OK)
        return st;
    st = accel_status(sync, "BNN_Execute");
    if (st != BNNE_OK)
        return st;
    if (*static_cast<volatile int32_t*>(r->pinned_tokens + n) != 0)  // cleared by the next call's first launch
        return complain(BNNE_ECOMPUTE, "the logits hold a NaN or infinity");
    std::memcpy(out_tokens, r->pinned_tokens, (size_t)n * sizeof(int32_t));
    if (stats) {
        c->stats.execute_ns += t2 - t1;
        c->stats.transfer_ns += clock_ns() - t2;
        c->stats.device_calls += n * (r->jobs_per_token + r->lm_jobs);
        c->stats.bytes_read += n * sizeof(int32_t);
        c->stats.logical_macs += n * (r->macs_per_token + r->lm_macs);
        c->stats.executed_macs += n * (r->macs_per_token + r->lm_macs);
    }
    return BNNE_OK;
}

}  // namespace bnne
