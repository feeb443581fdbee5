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

#include "bnn-accelerator-hip.h"
#include "resident.h"

#define BNNE_EXPF_QUALIFIER static __device__ __forceinline__
#include "libc_expf.h"

#pragma clang fp contract(off)

namespace bnne {
namespace {

constexpr uint32_t kMaxHeadDim = 512;
constexpr uint32_t kMaxNormWidth = 16384;
enum : int { kErrNone = 0, kErrNorm = 1, kErrScore = 2, kErrSoftmax = 3 };

// expf of the host C library, bit for bit (see libc_expf.h)
__constant__ uint64_t kExp2Table[32] = BNNE_EXP2_TABLE;

__device__ __forceinline__ float expf_libc(float x) { return bnne_expf_libc(x, kExp2Table); }

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

// The in-order sum of n floats held in LDS (16-byte aligned): 16-byte loads; the
// second half of each 64-value step is loading while the first half is added.
__device__ __forceinline__ float sum_lds_in_order(const float* p, uint32_t n) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    const uint32_t n4 = n / 4u;
    float sum = 0.0f;
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

// x[i] = +scale or -scale of the token's Q1_0 embedding row (qwen3.c:355-366).
__global__ __launch_bounds__(256) void k_embed(uint32_t token, const uint8_t* __restrict__ bits,
                                               const uint16_t* __restrict__ scales, uint32_t C,
                                               float* __restrict__ x) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= C)
        return;
    const float s = __half2float(__ushort_as_half(scales[(size_t)token * (C / 128u) + i / 128u]));
    const bool bit = (bits[(size_t)token * (C / 8u) + i / 8u] >> (i & 7u)) & 1u;
    x[i] = bit ? s : -s;
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

// Causal attention of one head against cache rows 0..pos (qwen3.c:441-478):
// scores (each dot sequential over head_dim), max, exp, the sum in position order,
// probabilities, and each output element's sum in position order.  Scores and
// probabilities live in LDS up to kLdsPositions positions, in `scores` beyond.
constexpr uint32_t kLdsPositions = 8192;

__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q, const float* __restrict__ kc,
                                                   const float* __restrict__ vc, uint32_t pos, uint32_t kv_dim,
                                                   uint32_t HD, uint32_t kv_mul, float scale,
                                                   float* __restrict__ scores, uint32_t n_ctx,
                                                   float* __restrict__ y, int* err) {
    __shared__ float qs[kMaxHeadDim];
    __shared__ float red[256];
    __shared__ float sum_s;
    __shared__ float4 lds_sc4[kLdsPositions / 4];
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
    // value[i] = sum_t p[t] * v[t][i]: lanes over i, positions in order, 8 rows of
    // V loaded ahead of their adds
    for (uint32_t i = tid; i < HD; i += 256u) {
        const float* col = vc + head_off + i;
        float acc = 0.0f;
        uint32_t t = 0;
        for (; t + 8u <= pos + 1u; t += 8u) {
            float vv[8];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                vv[c] = col[(size_t)(t + c) * kv_dim];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                acc = acc + sc[t + c] * vv[c];
        }
        for (; t <= pos; ++t)
            acc = acc + sc[t] * col[(size_t)t * kv_dim];
        y[(size_t)h * HD + i] = acc;
    }
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
    BNN_Buffer b_norm, b_q, b_k, b_v, b_y, b_o, b_gate, b_up, b_logits;
    float *norm, *q, *k, *v, *y, *o, *gate, *up;
    // everything else: this engine's device memory
    float *x, *kc, *vc, *scores, *gains, *rope_cos, *rope_sin;
    uint8_t* emb_bits;
    uint16_t* emb_scales;
    int* err;
    BNNX_Batch *qkv, *attn_out, *gate_up, *down;
    BNNX_Batch lm_head;
    const Linear** lin;  // [7 * L + 1]: per layer q, k, v, o, gate, up, down; then lm_head
    uint64_t jobs_per_token, macs_per_token, lm_jobs, lm_macs;
};

namespace {

BNNE_Status hip_error(hipError_t e, const char* what) {
    (void)hipGetLastError();
    return error(e == hipErrorOutOfMemory ? BNNE_ENOMEM : BNNE_EIO, "%s: %s", what, hipGetErrorString(e));
}

BNNE_Status alloc_buffer(Resident* r, size_t floats, BNN_Buffer* b, float** ptr) {
    BNNE_Status st = accel_error(BNN_BufferAlloc(r->dev, floats * sizeof(float), b), "BNN_BufferAlloc");
    if (st == BNNE_OK)
        st = accel_error(BNNX_BufferDevicePointer(*b, reinterpret_cast<void**>(ptr)), "BNNX_BufferDevicePointer");
    return st;
}

template <class T>
BNNE_Status upload(T** dst, const void* src, size_t bytes) {
    hipError_t e = hipMalloc(reinterpret_cast<void**>(dst), bytes);
    if (e == hipSuccess && src)
        e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? BNNE_OK : hip_error(e, "device upload");
}

void add_jobs(const Linear* l, BNN_Buffer in, BNN_Buffer out, BNN_Job* jobs, uint32_t* n, uint64_t* macs) {
    for (uint32_t c = 0; c < l->n_chunks; ++c) {
        BNN_Job& j = jobs[(*n)++];
        j = BNN_Job{};
        j.operation = BNN_OP_GEMV_F32;
        j.matrix = l->chunks[c].matrix;
        j.input.buffer = in;
        j.input.type = BNN_TYPE_F32;
        j.output.buffer = out;
        j.output.type = BNN_TYPE_F32;
        j.output.offset = (size_t)l->chunks[c].out_off * sizeof(float);
        j.rows = 1;
    }
    *macs += (uint64_t)l->in * l->out;
}

BNNE_Status make_batch(Resident* r, std::initializer_list<std::pair<const Linear*, BNN_Buffer>> parts, BNN_Buffer in,
                       BNNX_Batch* out, uint64_t* jobs_total, uint64_t* macs) {
    uint32_t count = 0;
    for (const auto& p : parts)
        count += p.first->n_chunks;
    BNN_Job* jobs = static_cast<BNN_Job*>(std::calloc(count, sizeof(BNN_Job)));
    if (!jobs)
        return error(BNNE_ENOMEM, "out of memory");
    uint32_t n = 0;
    for (const auto& p : parts)
        add_jobs(p.first, in, p.second, jobs, &n, macs);
    const BNNE_Status st = accel_error(BNNX_BatchCreate(r->dev, jobs, n, out), "BNNX_BatchCreate");
    std::free(jobs);
    *jobs_total += n;
    return st;
}

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

// The prepared batches of every layer and of the lm_head.  Rebuilt when the
// backend reports them stale (some other matrix or buffer of the device was
// destroyed since; this context's own objects are still alive).
BNNE_Status build_batches(Resident* r) {
    r->jobs_per_token = r->macs_per_token = r->lm_jobs = r->lm_macs = 0;
    BNNE_Status st = BNNE_OK;
    for (uint32_t l = 0; st == BNNE_OK && l < r->L; ++l) {
        const Linear* const* p = r->lin + 7 * (size_t)l;
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

BNNE_Status resident_create(bnne_context* c, const ResidentModel& m, Resident** out) {
    *out = nullptr;
    if (m.HD > kMaxHeadDim || m.C > kMaxNormWidth)
        return error(BNNE_ENOTSUP, "device-resident decode supports head_dim <= %u and width <= %u", kMaxHeadDim,
                     kMaxNormWidth);
    Resident* r = static_cast<Resident*>(std::calloc(1, sizeof(Resident)));
    if (!r)
        return error(BNNE_ENOMEM, "out of memory");
    r->dev = c->model->device;
    r->C = m.C, r->H = m.H, r->Hk = m.Hk, r->HD = m.HD, r->FF = m.FF, r->L = m.L, r->V = m.V;
    r->kv_dim = m.kv_dim, r->n_ctx = m.n_ctx, r->eps = m.eps;
    BNNE_Status st = accel_error(BNNX_DeviceStream(r->dev, reinterpret_cast<void**>(&r->stream)), "BNNX_DeviceStream");
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
    float* logits_dev = nullptr;
    if (st == BNNE_OK)
        st = alloc_buffer(r, m.V, &r->b_logits, &logits_dev);
    const size_t cache = (size_t)m.L * m.n_ctx * m.kv_dim * sizeof(float);
    if (st == BNNE_OK)
        st = upload(&r->x, nullptr, (size_t)m.C * sizeof(float));
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
            st = error(BNNE_ENOMEM, "out of memory");
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
    if (st == BNNE_OK) {
        r->qkv = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->attn_out = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->gate_up = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->down = static_cast<BNNX_Batch*>(std::calloc(m.L, sizeof(BNNX_Batch)));
        r->lin = static_cast<const Linear**>(std::calloc(7 * (size_t)m.L + 1, sizeof(Linear*)));
        if (!r->qkv || !r->attn_out || !r->gate_up || !r->down || !r->lin)
            st = error(BNNE_ENOMEM, "out of memory");
    }
    if (st == BNNE_OK) {
        for (uint32_t l = 0; l < m.L; ++l) {
            const Linear** p = r->lin + 7 * (size_t)l;
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
    for (BNN_Buffer b : {r->b_norm, r->b_q, r->b_k, r->b_v, r->b_y, r->b_o, r->b_gate, r->b_up, r->b_logits})
        BNN_BufferFree(b);
    for (void* p : {(void*)r->x, (void*)r->kc, (void*)r->vc, (void*)r->scores, (void*)r->gains, (void*)r->rope_cos,
                    (void*)r->rope_sin, (void*)r->emb_bits, (void*)r->emb_scales, (void*)r->err})
        if (p)
            (void)hipFree(p);
    std::free(r);
}

BNNE_Status resident_step(bnne_context* c, Resident* r, const int32_t* tokens, uint32_t n, uint32_t pos0,
                          float* logits) {
    const bool stats = c->params.enable_stats != 0;
    const uint64_t t0 = stats ? now_ns() : 0;
    hipError_t e = hipSetDevice(r->ordinal);
    if (e != hipSuccess)
        return hip_error(e, "hipSetDevice");
    const uint32_t C = r->C, HD = r->HD, half = HD / 2u;
    const float scale = 1.0f / sqrtf((float)HD);
    const float* attn_norm = r->gains;
    const float* ffn_norm = r->gains + (size_t)r->L * C;
    const float* q_norm = r->gains + 2 * (size_t)r->L * C;
    const float* k_norm = q_norm + (size_t)r->L * HD;
    const float* final_norm = k_norm + (size_t)r->L * HD;
    const size_t norm_lds = (size_t)C * sizeof(float);
    BNNE_Status st = BNNE_OK;
    // Prepared batches go stale when any matrix or buffer of the device is destroyed
    // (another context, another model); nothing can be destroyed during a step, so
    // checking one batch decides for all of them.
    const BNN_Status valid = BNNX_BatchCheck(r->qkv[0]);
    if (valid == BNN_EINVAL) {
        destroy_batches(r);
        st = build_batches(r);
        if (st != BNNE_OK)
            return st;
    } else if (valid != BNN_OK) {
        return accel_error(valid, "BNNX_BatchCheck");
    }
    auto launch = [&](BNNX_Batch b) {
        if (st == BNNE_OK)
            st = accel_error(BNNX_BatchLaunch(b), "BNNX_BatchLaunch");
    };
    for (uint32_t i = 0; i < n && st == BNNE_OK; ++i) {
        const uint32_t pos = pos0 + i;
        hipLaunchKernelGGL(k_embed, dim3((C + 255u) / 256u), dim3(256), 0, r->stream, (uint32_t)tokens[i],
                           r->emb_bits, r->emb_scales, C, r->x);
        for (uint32_t l = 0; l < r->L && st == BNNE_OK; ++l) {
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
        if (logits && i + 1 == n) {
            hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), norm_lds, r->stream, r->x, r->o, C, r->eps, final_norm,
                               r->norm, r->err);
            launch(r->lm_head);
        }
    }
    e = hipGetLastError();
    const uint64_t t1 = stats ? now_ns() : 0;
    const BNN_Status sync = BNNX_DeviceSynchronize(r->dev);
    const uint64_t t2 = stats ? now_ns() : 0;
    if (st != BNNE_OK)
        return st;
    if (e != hipSuccess)
        return hip_error(e, "kernel launch");
    int err = 0;
    e = hipMemcpy(&err, r->err, sizeof err, hipMemcpyDeviceToHost);
    if (e == hipSuccess && err != kErrNone)
        e = hipMemset(r->err, 0, sizeof(int));
    if (e != hipSuccess)
        return hip_error(e, "error word");
    if (err == kErrNorm)
        return error(BNNE_ECOMPUTE, "Qwen3 RMSNorm produced a non-finite divisor");
    if (err == kErrScore)
        return error(BNNE_ECOMPUTE, "Qwen3 attention score is not finite");
    if (err == kErrSoftmax)
        return error(BNNE_ECOMPUTE, "Qwen3 attention softmax failed");
    st = accel_error(sync, "BNN_Execute");
    if (st != BNNE_OK)
        return st;
    if (logits) {
        st = accel_error(BNN_BufferRead(r->b_logits, 0, logits, (size_t)r->V * sizeof(float)), "BNN_BufferRead");
        if (st != BNNE_OK)
            return st;
    }
    if (stats) {
        const uint64_t t3 = now_ns();
        c->stats.execute_ns += t2 - t1;
        c->stats.transfer_ns += t3 - t2;
        const uint64_t lm = logits ? 1 : 0;
        c->stats.device_calls += n * r->jobs_per_token + lm * r->lm_jobs;
        c->stats.bytes_read += lm * r->V * sizeof(float);
        c->stats.logical_macs += n * r->macs_per_token + lm * r->lm_macs;
        c->stats.executed_macs += n * r->macs_per_token + lm * r->lm_macs;
        (void)t0;
    }
    return BNNE_OK;
}

}  // namespace bnne
