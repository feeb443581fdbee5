// Host side of the HIP backend: the eleven BNN_* entry points of the BNN
// accelerator API v2 (reference bnn-accelerator/bnn-accelerator.h:171-207),
// plus the BNNX_* extensions of include/bnn-accelerator-hip.h.
//
// Argument validation follows the reference soft backend's order and status
// codes exactly (bnn-accelerator/soft-bnn-accelerator.c:310-603), because the
// reference's contract test pins both.  Input-value validation (-128, NaN/Inf)
// happens on the GPU: the prep kernel raises a per-device flag with the job's
// sequence number, every later kernel of the job checks it before writing, and
// the host learns the outcome from a pinned status word after the one
// synchronisation of the call.  So an illegal input leaves the output untouched.
#include <fenv.h>
#include <float.h>
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "bnn-accelerator-hip.h"
#include "bnn-accelerator.h"
#include "bnn_internal.h"

using namespace bnnhip;

#define EXPORT extern "C" __attribute__((visibility("default")))

namespace {

constexpr size_t kPinnedCap = size_t(8) << 20;       // largest transfer staged through pinned memory
constexpr size_t kWriteRingBytes = size_t(1) << 20;  // pinned ring for small writes
constexpr size_t kAsyncWriteMax = size_t(64) << 10;  // writes up to this size return before the copy ends
constexpr size_t kScratchRowsCap = 4096;              // rows per launch chunk
constexpr size_t kExecuteScratchBytes = size_t(32) << 20;  // allocated with the device

bool mul_size(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a)
        return false;
    *out = a * b;
    return true;
}

bool span_fits(size_t capacity, size_t offset, size_t bytes) {
    return offset <= capacity && bytes <= capacity - offset;
}

// (soft-bnn-accelerator.c:65-77) last logical row inside the buffer, overflow-free.
bool rows_fit(size_t capacity, size_t offset, size_t stride, size_t row_bytes, uint32_t rows) {
    if (rows == 0 || row_bytes == 0 || stride < row_bytes || offset > capacity)
        return false;
    size_t room = capacity - offset;
    if (row_bytes > room)
        return false;
    return (uintmax_t)(rows - 1u) <= (uintmax_t)((room - row_bytes) / stride);
}

BNN_Status hip_status(hipError_t e) {
    if (e == hipSuccess)
        return BNN_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return BNN_ENOMEM;
    return BNN_EIO;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

BNN_Status ensure_scratch(BNN_Device d, size_t bytes) {
    if (bytes <= d->scratch_bytes)
        return BNN_OK;
    if (d->scratch) {
        (void)hipFree(d->scratch);
        d->scratch = nullptr;
        d->scratch_bytes = 0;
    }
    size_t want = round_up(bytes, size_t(1) << 20);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_ENOMEM;
    }
    d->scratch = static_cast<unsigned char*>(p);
    d->scratch_bytes = want;
    d->generation++;
    return BNN_OK;
}

BNN_Status ensure_pinned(BNN_Device d, size_t bytes) {
    if (bytes <= d->pinned_bytes)
        return BNN_OK;
    if (d->pinned) {
        (void)hipHostFree(d->pinned);
        d->pinned = nullptr;
        d->pinned_bytes = 0;
    }
    size_t want = round_up(bytes, size_t(1) << 16);
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_ENOMEM;
    }
    d->pinned = static_cast<unsigned char*>(p);
    d->pinned_bytes = want;
    return BNN_OK;
}

BNN_Status ensure_mirror(BNN_Device d) {
    if (d->mirror)
        return BNN_OK;
    void* p = nullptr;
    if (hipHostMalloc(&p, sizeof(float) * kMaxFeatures, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return BNN_ENOMEM;
    }
    d->mirror = static_cast<float*>(p);
    return BNN_OK;
}

// Adds the elapsed time of every recorded event pair; the stream must be idle.
hipError_t resolve_timing(BNN_Device d) {
    hipError_t result = hipSuccess;
    for (int i = 0; i < d->ev_used; ++i) {
        float ms = 0.0f;
        hipError_t e = hipEventElapsedTime(&ms, d->ev_begin[i], d->ev_end[i]);
        if (e != hipSuccess) {
            result = e;
            continue;
        }
        d->kernel_ms[d->ev_kind[i]] += ms;
        d->kernel_launches[d->ev_kind[i]] += 1;
    }
    d->ev_used = 0;
    return result;
}

void destroy_events(BNN_Device d) {
    for (int i = 0; i < bnn_accel_device::kTimingSlots; ++i) {
        if (d->ev_begin[i])
            (void)hipEventDestroy(d->ev_begin[i]);
        if (d->ev_end[i])
            (void)hipEventDestroy(d->ev_end[i]);
        d->ev_begin[i] = d->ev_end[i] = nullptr;
    }
    d->events_created = false;
}

// The timing event pairs, created on the first BNNX_KernelTiming(device, 1).
BNN_Status ensure_events(BNN_Device d) {
    if (d->events_created)
        return BNN_OK;
    if (hipSetDevice(d->ordinal) != hipSuccess)
        return BNN_EIO;
    hipError_t e = hipSuccess;
    for (int i = 0; e == hipSuccess && i < bnn_accel_device::kTimingSlots; ++i) {
        e = hipEventCreate(&d->ev_begin[i]);
        if (e == hipSuccess)
            e = hipEventCreate(&d->ev_end[i]);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        destroy_events(d);
        return hip_status(e);
    }
    d->events_created = true;
    return BNN_OK;
}

}  // namespace

namespace bnnhip {
thread_local LaunchEvents t_launch_events = {nullptr, nullptr};
}  // namespace bnnhip

namespace {

// Launch helper: when timing is on, the kernel that `launch` enqueues records its own
// start and end into an event pair (hipExtLaunchKernel: timestamps of the dispatch
// itself, no marker packets between kernels; no synchronisation unless the slots run out).
template <typename F>
hipError_t timed(BNN_Device d, int kind, F&& launch) {
    if (!d->timing)
        return launch();
    if (d->ev_used == bnn_accel_device::kTimingSlots) {
        hipError_t e = hipStreamSynchronize(d->stream);
        if (e == hipSuccess)
            e = resolve_timing(d);
        if (e != hipSuccess)
            return e;
    }
    const int slot = d->ev_used;
    t_launch_events = LaunchEvents{d->ev_begin[slot], d->ev_end[slot]};
    hipError_t e = launch();
    t_launch_events = LaunchEvents{nullptr, nullptr};
    if (e == hipSuccess) {
        d->ev_kind[slot] = kind;
        d->ev_used = slot + 1;
    }
    return e;
}

BNN_Status op_types(BNN_Operation op, BNN_Type* in, BNN_Type* out) {
    switch (op) {
    case BNN_OP_GEMV:
    case BNN_OP_GEMM:
        *in = BNN_TYPE_I8;
        *out = BNN_TYPE_F32;
        return BNN_OK;
    case BNN_OP_DOT_GROUPS:
        *in = BNN_TYPE_I8;
        *out = BNN_TYPE_I16;
        return BNN_OK;
    case BNN_OP_GEMV_F32:
    case BNN_OP_GEMM_F32:
        *in = BNN_TYPE_F32;
        *out = BNN_TYPE_F32;
        return BNN_OK;
    default:
        return BNN_ENOTSUP;
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Devices (soft-bnn-accelerator.c:310-356)
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Fixed device scratch of BNNX_ExecuteNoAlloc: one copy per GPU, resident until the
// process ends.  Host code never passes the symbol itself to a kernel (on the host it
// is only a stand-in for the device variable): open_device resolves each GPU's copy
// once with hipGetSymbolAddress, and every later use goes through that address.
// ---------------------------------------------------------------------------
constexpr size_t kStaticScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

constexpr int kMaxOrdinals = 64;
pthread_mutex_t g_static_lock = PTHREAD_MUTEX_INITIALIZER;
unsigned char* g_static_scratch[kMaxOrdinals];  // per HIP ordinal, null until resolved
// Held by BNNX_ExecuteNoAlloc while it uses its GPU's `scratch` (the call is synchronous):
// devices are independent (bnn-accelerator.h:166-168) even when several handles share a GPU.
std::mutex g_static_use[kMaxOrdinals];

// The current device's copy of `scratch` (the caller has made `ordinal` current).
hipError_t resolve_static_scratch(int ordinal, unsigned char** out) {
    *out = nullptr;
    if (ordinal < 0 || ordinal >= kMaxOrdinals)
        return hipErrorInvalidDevice;
    pthread_mutex_lock(&g_static_lock);
    hipError_t e = hipSuccess;
    if (g_static_scratch[ordinal] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess && p == nullptr)
            e = hipErrorInvalidSymbol;
        if (e == hipSuccess)
            g_static_scratch[ordinal] = static_cast<unsigned char*>(p);
    }
    *out = g_static_scratch[ordinal];
    pthread_mutex_unlock(&g_static_lock);
    return e;
}

// Opens HIP device `ordinal` (BNN_DeviceOpen: 0; BNNX_DeviceOpenOrdinal: any).
BNN_Status open_device(int ordinal, BNN_Device* out_device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return BNN_ENOTSUP;
    }
    if (ordinal < 0 || ordinal >= count || ordinal >= kMaxOrdinals)
        return BNN_ENOTSUP;
    float one = 1.0f;
    uint32_t one_bits;
    memcpy(&one_bits, &one, sizeof one_bits);
    if (one_bits != 0x3f800000u)
        return BNN_ENOTSUP;

    BNN_Device d = static_cast<BNN_Device>(calloc(1, sizeof(bnn_accel_device)));
    if (d == nullptr)
        return BNN_ENOMEM;
    d->ordinal = ordinal;
    hipError_t e = hipSetDevice(d->ordinal);
    if (e == hipSuccess)
        e = resolve_static_scratch(d->ordinal, &d->static_scratch);
    int cus = 0;
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d->ordinal);
    d->cu_count = cus > 0 ? (uint32_t)cus : 256u;
    if (e == hipSuccess)
        e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e == hipSuccess)
        e = hipMalloc(reinterpret_cast<void**>(&d->flag_dev), 256);
    if (e == hipSuccess) {  // BNN_Execute's scratch: quantised rows (and staging rows) of a chunk of rows
        e = hipMalloc(reinterpret_cast<void**>(&d->scratch), kExecuteScratchBytes);
        d->scratch_bytes = e == hipSuccess ? kExecuteScratchBytes : 0;
    }
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&d->status_host), kStatusHostBytes, hipHostMallocCoherent);
    if (e == hipSuccess) {
        memset(d->status_host, 0, kStatusHostBytes);
        static const uint64_t zero = 0;  // the illegal-input flag
        e = hipMemcpyAsync(d->flag_dev, &zero, sizeof zero, hipMemcpyHostToDevice, d->stream);
        if (e == hipSuccess)
            e = hipStreamSynchronize(d->stream);
    }
    if (e != hipSuccess) {
        BNN_Status st = hip_status(e);
        (void)hipGetLastError();
        if (d->status_host)
            (void)hipHostFree(d->status_host);
        if (d->flag_dev)
            (void)hipFree(d->flag_dev);
        if (d->scratch)
            (void)hipFree(d->scratch);
        if (d->stream)
            (void)hipStreamDestroy(d->stream);
        free(d);
        return st == BNN_ENOMEM ? BNN_ENOMEM : BNN_EIO;
    }
    *out_device = d;
    return BNN_OK;
}

}  // namespace

// (soft-bnn-accelerator.c:309-325) index 0 only; it names the process's first visible
// HIP device.  Other GPUs of a host: BNNX_DeviceOpenOrdinal.
EXPORT BNN_Status BNN_DeviceOpen(uint32_t device_index, BNN_Device* out_device) {
    if (out_device == nullptr)
        return BNN_EINVAL;
    *out_device = nullptr;
    if (device_index != 0)
        return BNN_ENOTSUP;
    return open_device(0, out_device);
}

EXPORT BNN_Status BNNX_DeviceOpenOrdinal(uint32_t hip_ordinal, BNN_Device* out_device) {
    if (out_device == nullptr)
        return BNN_EINVAL;
    *out_device = nullptr;
    if (hip_ordinal > (uint32_t)INT32_MAX)
        return BNN_ENOTSUP;
    return open_device((int)hip_ordinal, out_device);
}

EXPORT BNN_Status BNN_DeviceClose(BNN_Device device) {
    if (device == nullptr)
        return BNN_EINVAL;
    if (device->live_matrices != 0 || device->live_buffers != 0 || device->live_batches != 0)
        return BNN_EBUSY;
    (void)hipSetDevice(device->ordinal);
    (void)hipStreamSynchronize(device->stream);
    if (device->scratch)
        (void)hipFree(device->scratch);
    if (device->pinned)
        (void)hipHostFree(device->pinned);
    if (device->wring)
        (void)hipHostFree(device->wring);
    if (device->mirror)
        (void)hipHostFree(device->mirror);
    if (device->table_host)
        (void)hipHostFree(device->table_host);
    if (device->table_dev)
        (void)hipFree(device->table_dev);
    free(device->batch_jobs);
    destroy_events(device);
    (void)hipHostFree(device->status_host);
    (void)hipFree(device->flag_dev);
    (void)hipStreamDestroy(device->stream);
    free(device);
    return BNN_OK;
}

EXPORT BNN_Status BNN_DeviceGetCaps(BNN_Device device, BNN_Caps* out_caps) {
    if (device == nullptr || out_caps == nullptr)
        return BNN_EINVAL;
    memset(out_caps, 0, sizeof *out_caps);
    out_caps->api_version = BNN_API_VERSION;
    out_caps->max_in_features = kMaxFeatures;
    out_caps->max_out_features = kMaxFeatures;
    out_caps->max_rows = UINT32_MAX;
    out_caps->group_size = kGroup;
    out_caps->supported_ops =
        BNN_CAP_GEMV | BNN_CAP_GEMM | BNN_CAP_DOT_GROUPS | BNN_CAP_GEMV_F32 | BNN_CAP_GEMM_F32;
    return BNN_OK;
}

// ---------------------------------------------------------------------------
// Matrices (soft-bnn-accelerator.c:358-440): validate, repack to the tile
// layout of bnn_internal.h on the host, upload once, keep resident.
// ---------------------------------------------------------------------------

EXPORT BNN_Status BNN_MatrixCreate(BNN_Device device, const BNN_MatrixDesc* desc, BNN_Matrix* out_matrix) {
    if (out_matrix == nullptr)
        return BNN_EINVAL;
    *out_matrix = nullptr;
    if (device == nullptr || desc == nullptr)
        return BNN_EINVAL;
    if (desc->in_features == 0 || desc->out_features == 0 || desc->group_size == 0 || desc->group_size > 256u ||
        desc->group_size % 8u != 0)
        return BNN_EINVAL;
    if (desc->in_features > kMaxFeatures || desc->out_features > kMaxFeatures || desc->group_size != kGroup)
        return BNN_ENOTSUP;
    if (desc->in_features % kGroup != 0)
        return BNN_EINVAL;
    size_t bits_bytes, scale_count, scale_bytes;
    if (!mul_size(desc->out_features, desc->in_features / 8u, &bits_bytes) ||
        !mul_size(desc->out_features, desc->in_features / kGroup, &scale_count) ||
        !mul_size(scale_count, sizeof(uint16_t), &scale_bytes))
        return BNN_ERANGE;
    if (desc->weight_bits == nullptr || desc->scale_fp16 == nullptr || desc->weight_bytes != bits_bytes ||
        desc->scale_count != scale_count)
        return BNN_EINVAL;
    for (size_t i = 0; i < scale_count; ++i)
        if ((desc->scale_fp16[i] & 0x7c00u) == 0x7c00u)
            return BNN_EINVAL;
    if (device->live_matrices == SIZE_MAX)
        return BNN_ERANGE;

    const uint32_t k = desc->in_features, n = desc->out_features, groups = k / kGroup;
    const uint32_t tiles = (n + kTile - 1) / kTile;
    const size_t wbits_bytes = (size_t)tiles * groups * kTile * 16u;
    const size_t wscale_bytes = (size_t)tiles * kTile * groups * 2u;
    const size_t total = wbits_bytes + round_up(wscale_bytes, 256);

    BNN_Matrix m = static_cast<BNN_Matrix>(calloc(1, sizeof(bnn_accel_matrix)));
    if (m == nullptr)
        return BNN_ENOMEM;
    unsigned char* host = static_cast<unsigned char*>(malloc(total));
    if (host == nullptr) {
        free(m);
        return BNN_ENOMEM;
    }
    // repack: wbits[t][g][lane] <- row n = 64t + lane, bytes 16g..16g+15
    const size_t row_bytes = k / 8u;
    uint8_t* hb = host;
    for (uint32_t t = 0; t < tiles; ++t)
        for (uint32_t g = 0; g < groups; ++g)
            for (uint32_t l = 0; l < kTile; ++l) {
                const uint32_t nn = t * kTile + l;
                uint8_t* dst = hb + (((size_t)t * groups + g) * kTile + l) * 16u;
                if (nn < n)
                    memcpy(dst, desc->weight_bits + (size_t)nn * row_bytes + (size_t)g * 16u, 16);
                else
                    memset(dst, 0, 16);
            }
    // wscale[t][g][lane] <- scale of (n = 64t + lane, g)
    uint16_t* hs = reinterpret_cast<uint16_t*>(host + wbits_bytes);
    for (uint32_t t = 0; t < tiles; ++t)
        for (uint32_t g = 0; g < groups; ++g)
            for (uint32_t l = 0; l < kTile; ++l) {
                const uint32_t nn = t * kTile + l;
                hs[((size_t)t * groups + g) * kTile + l] = nn < n ? desc->scale_fp16[(size_t)nn * groups + g] : 0;
            }

    hipError_t e = hipSetDevice(device->ordinal);
    void* dev = nullptr;
    if (e == hipSuccess)
        e = hipMalloc(&dev, total);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dev, host, total, hipMemcpyHostToDevice, device->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(device->stream);
    free(host);
    if (e != hipSuccess) {
        BNN_Status st = hip_status(e);
        (void)hipGetLastError();
        if (dev)
            (void)hipFree(dev);
        free(m);
        return st;
    }
    m->device = device;
    m->k = k;
    m->n = n;
    m->groups = groups;
    m->tiles = tiles;
    m->wbits = static_cast<uint4*>(dev);
    m->wscale = reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(dev) + wbits_bytes);
    device->live_matrices++;
    device->generation++;
    *out_matrix = m;
    return BNN_OK;
}

EXPORT void BNN_MatrixDestroy(BNN_Matrix matrix) {
    if (matrix == nullptr)
        return;
    (void)hipSetDevice(matrix->device->ordinal);
    (void)hipStreamSynchronize(matrix->device->stream);
    (void)hipFree(matrix->wbits);
    matrix->device->live_matrices--;
    matrix->device->generation++;
    matrix->device->retired++;
    free(matrix);
}

// ---------------------------------------------------------------------------
// Buffers (soft-bnn-accelerator.c:442-511): device memory, synchronous copies.
// ---------------------------------------------------------------------------

EXPORT BNN_Status BNN_BufferAlloc(BNN_Device device, size_t bytes, BNN_Buffer* out_buffer) {
    if (out_buffer == nullptr)
        return BNN_EINVAL;
    *out_buffer = nullptr;
    if (device == nullptr || bytes == 0)
        return BNN_EINVAL;
    if (device->live_buffers == SIZE_MAX)
        return BNN_ERANGE;
    BNN_Buffer b = static_cast<BNN_Buffer>(calloc(1, sizeof(bnn_accel_buffer)));
    if (b == nullptr)
        return BNN_ENOMEM;
    void* p = nullptr;
    hipError_t e = hipSetDevice(device->ordinal);
    if (e == hipSuccess)
        e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        free(b);
        return BNN_ENOMEM;
    }
    b->device = device;
    b->size = bytes;
    b->dev = static_cast<unsigned char*>(p);
    device->live_buffers++;
    device->generation++;
    *out_buffer = b;
    return BNN_OK;
}

EXPORT void BNN_BufferFree(BNN_Buffer buffer) {
    if (buffer == nullptr)
        return;
    (void)hipSetDevice(buffer->device->ordinal);
    (void)hipStreamSynchronize(buffer->device->stream);
    if (buffer->device->mirror_buf == buffer)
        buffer->device->mirror_buf = nullptr;
    (void)hipFree(buffer->dev);
    buffer->device->live_buffers--;
    buffer->device->generation++;
    buffer->device->retired++;
    free(buffer);
}

EXPORT BNN_Status BNN_BufferWrite(BNN_Buffer buffer, size_t offset, const void* src, size_t bytes) {
    if (buffer == nullptr || (bytes != 0 && src == nullptr))
        return BNN_EINVAL;
    if (!span_fits(buffer->size, offset, bytes))
        return BNN_ERANGE;
    if (bytes == 0)
        return BNN_OK;
    BNN_Device d = buffer->device;
    d->mirror_buf = nullptr;
    hipError_t e = hipSetDevice(d->ordinal);
    if (e != hipSuccess)
        return BNN_EIO;
    if (bytes <= kAsyncWriteMax) {
        // Small writes (a linear's input row: linear.c:169-175): the bytes are copied into
        // the pinned ring and the host->device copy is queued on the device stream, which
        // orders it before every later kernel, read or write of this device.  The caller's
        // memory is free on return; the ring restarts after a synchronisation.
        if (d->wring == nullptr) {
            void* p = nullptr;
            if (hipHostMalloc(&p, kWriteRingBytes, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                return BNN_ENOMEM;
            }
            d->wring = static_cast<unsigned char*>(p);
            d->wring_off = 0;
        }
        if (d->wring_off + bytes > kWriteRingBytes) {
            if (hipStreamSynchronize(d->stream) != hipSuccess) {
                (void)hipGetLastError();
                return BNN_EIO;
            }
            d->wring_off = 0;
        }
        unsigned char* slot = d->wring + d->wring_off;
        memcpy(slot, src, bytes);
        e = hipMemcpyAsync(buffer->dev + offset, slot, bytes, hipMemcpyHostToDevice, d->stream);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return BNN_EIO;
        }
        d->wring_off += round_up(bytes, 256);
        return BNN_OK;
    }
    if (bytes <= kPinnedCap && ensure_pinned(d, bytes) == BNN_OK) {
        memcpy(d->pinned, src, bytes);
        e = hipMemcpyAsync(buffer->dev + offset, d->pinned, bytes, hipMemcpyHostToDevice, d->stream);
    } else {
        e = hipMemcpyAsync(buffer->dev + offset, src, bytes, hipMemcpyHostToDevice, d->stream);
    }
    if (e == hipSuccess)
        e = hipStreamSynchronize(d->stream);
    return e == hipSuccess ? BNN_OK : BNN_EIO;
}

EXPORT BNN_Status BNN_BufferRead(BNN_Buffer buffer, size_t offset, void* dst, size_t bytes) {
    if (buffer == nullptr || (bytes != 0 && dst == nullptr))
        return BNN_EINVAL;
    if (!span_fits(buffer->size, offset, bytes))
        return BNN_ERANGE;
    if (bytes == 0)
        return BNN_OK;
    BNN_Device d = buffer->device;
    if (d->mirror_buf == buffer && offset >= d->mirror_off && bytes <= d->mirror_bytes &&
        offset - d->mirror_off <= d->mirror_bytes - bytes) {
        // the last BNN_Execute's output, already in host memory (the call synchronised)
        memcpy(dst, reinterpret_cast<const unsigned char*>(d->mirror) + (offset - d->mirror_off), bytes);
        return BNN_OK;
    }
    hipError_t e = hipSetDevice(d->ordinal);
    if (e != hipSuccess)
        return BNN_EIO;
    if (bytes <= kPinnedCap && ensure_pinned(d, bytes) == BNN_OK) {
        e = hipMemcpyAsync(d->pinned, buffer->dev + offset, bytes, hipMemcpyDeviceToHost, d->stream);
        if (e == hipSuccess)
            e = hipStreamSynchronize(d->stream);
        if (e == hipSuccess)
            memcpy(dst, d->pinned, bytes);
    } else {
        e = hipMemcpyAsync(dst, buffer->dev + offset, bytes, hipMemcpyDeviceToHost, d->stream);
        if (e == hipSuccess)
            e = hipStreamSynchronize(d->stream);
    }
    return e == hipSuccess ? BNN_OK : BNN_EIO;
}

// ---------------------------------------------------------------------------
// Execute (soft-bnn-accelerator.c:513-603)
// ---------------------------------------------------------------------------

namespace {

// Everything Execute derives from a job before touching the device.
struct JobPlan {
    BNN_Matrix m;
    bool f32_in, dot_out;
    size_t in_row, out_row, in_stride, out_stride;
    const unsigned char* in_base;
    unsigned char* out_base;
    bool in_aligned, out_aligned;
    DotMode mode;
};

// Argument checks in the reference's order with its status codes
// (soft-bnn-accelerator.c:527-573).
BNN_Status plan_job(BNN_Device device, const BNN_Job* job, JobPlan* p) {
    if (device == nullptr || job == nullptr || job->matrix == nullptr || job->input.buffer == nullptr ||
        job->output.buffer == nullptr || job->rows == 0)
        return BNN_EINVAL;
    BNN_Type in_type, out_type;
    BNN_Status st = op_types(job->operation, &in_type, &out_type);
    if (st != BNN_OK)
        return st;
    if ((job->operation == BNN_OP_GEMV || job->operation == BNN_OP_GEMV_F32) && job->rows != 1)
        return BNN_EINVAL;
    if (job->input.type != in_type || job->output.type != out_type)
        return BNN_EINVAL;
    const BNN_Matrix m = job->matrix;
    if (m->device != device || job->input.buffer->device != device || job->output.buffer->device != device ||
        job->input.buffer == job->output.buffer)
        return BNN_EINVAL;
    p->m = m;
    p->f32_in = in_type == BNN_TYPE_F32;
    p->dot_out = job->operation == BNN_OP_DOT_GROUPS;
    size_t out_count;
    if (!mul_size(m->k, p->f32_in ? 4u : 1u, &p->in_row))
        return BNN_ERANGE;
    if (p->dot_out) {
        if (!mul_size(m->n, m->groups, &out_count) || !mul_size(out_count, 2u, &p->out_row))
            return BNN_ERANGE;
    } else if (!mul_size(m->n, 4u, &p->out_row)) {
        return BNN_ERANGE;
    }
    p->in_stride = job->input.row_stride ? job->input.row_stride : p->in_row;
    p->out_stride = job->output.row_stride ? job->output.row_stride : p->out_row;
    if (p->in_stride < p->in_row || p->out_stride < p->out_row)
        return BNN_EINVAL;
    if (!rows_fit(job->input.buffer->size, job->input.offset, p->in_stride, p->in_row, job->rows) ||
        !rows_fit(job->output.buffer->size, job->output.offset, p->out_stride, p->out_row, job->rows))
        return BNN_ERANGE;
    if (!p->dot_out && fegetround() != FE_TONEAREST)
        return BNN_ENOTSUP;
    p->in_base = job->input.buffer->dev + job->input.offset;
    p->out_base = job->output.buffer->dev + job->output.offset;
    p->in_aligned = !p->f32_in || (((uintptr_t)p->in_base | p->in_stride) & 3u) == 0;
    const size_t out_align = p->dot_out ? 2u : 4u;
    p->out_aligned = (((uintptr_t)p->out_base | p->out_stride) & (out_align - 1u)) == 0;
    p->mode = p->dot_out ? MODE_DOT_I16 : (p->f32_in ? MODE_SUM_SCALED : MODE_SUM);
    return BNN_OK;
}

// Scratch per block of rows: planes | sums | rscale | (matrix-core jobs) Q rows.
size_t row_scratch_bytes(const JobPlan& p, size_t rows, size_t* planes, size_t* sums, size_t* rscale,
                         size_t* q = nullptr, bool with_q = false) {
    *planes = round_up(rows * p.m->groups * kPlaneWords * 4u, 256);
    *sums = round_up(rows * p.m->groups * 4u, 256);
    *rscale = round_up(rows * 4u, 256);
    const size_t qb = with_q ? round_up(rows * p.m->k, 256) : 0;
    if (q)
        *q = qb;
    return *planes + *sums + *rscale + qb;
}

PrepJob make_prep(const JobPlan& p, const unsigned char* in, uint32_t rows, unsigned char* scratch,
                  bool with_q = false) {
    size_t planes, sums, rscale;
    row_scratch_bytes(p, rows, &planes, &sums, &rscale);
    PrepJob j = {};
    j.in = in;
    j.in_stride = p.in_stride;
    j.planes = reinterpret_cast<uint32_t*>(scratch);
    j.sums = reinterpret_cast<int32_t*>(scratch + planes);
    j.rscale = reinterpret_cast<float*>(scratch + planes + sums);
    j.q = with_q ? reinterpret_cast<int8_t*>(scratch + planes + sums + rscale) : nullptr;
    if (with_q) {  // the matrix-core path reads Q rows only
        j.planes = nullptr;
        j.sums = nullptr;
    }
    j.k = p.m->k;
    j.rows = rows;
    j.f32 = p.f32_in;
    j.aligned = p.in_aligned;
    return j;
}

DotJob make_dot(const JobPlan& p, const PrepJob& pj, unsigned char* out, size_t out_stride) {
    DotJob j = {};
    j.wbits = p.m->wbits;
    j.wscale = p.m->wscale;
    j.planes = pj.planes;
    j.sums = pj.sums;
    j.rscale = pj.rscale;
    j.out = out;
    j.out_stride = out_stride;
    j.n = p.m->n;
    j.groups = p.m->groups;
    j.tiles = p.m->tiles;
    j.rows = pj.rows;
    j.mode = p.mode;
    return j;
}

GemmJob make_gemm(const JobPlan& p, const PrepJob& pj, unsigned char* out, size_t out_stride) {
    GemmJob j = {};
    j.wbits = p.m->wbits;
    j.wscale = p.m->wscale;
    j.q = pj.q;
    j.rscale = pj.rscale;
    j.out = out;
    j.out_stride = out_stride;
    j.n = p.m->n;
    j.k = p.m->k;
    j.groups = p.m->groups;
    j.tiles = p.m->tiles;
    j.rows = pj.rows;
    j.mode = p.mode;
    return j;
}

// Completion of a single-row launch whose `grid` workgroups each store seq into their own
// pinned word (status_host from kDoneFlagWord) once their results are visible to the host:
// spin on those instead of waiting for the end of the kernel, which the runtime reports
// several microseconds later.  Past a bound far above any single-row kernel (or with
// kernel timing on, whose events are resolved at a stream synchronisation) the ordinary
// stream wait takes over; it also reports device errors.
BNN_Status finish(BNN_Device device, hipError_t e, uint64_t seq);

BNN_Status finish_signalled(BNN_Device device, hipError_t e, uint64_t seq, uint32_t grid) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_EIO;
    }
    if (!device->timing) {
        const uint64_t* const done = device->status_host + kDoneFlagWord;
        const uint64_t t0 = __builtin_readcyclecounter();
        uint32_t seen = 0;  // workgroups 0 .. seen-1 have signalled
        for (uint32_t i = 0;; ++i) {
            while (seen < grid && __atomic_load_n(&done[seen], __ATOMIC_ACQUIRE) == seq)
                ++seen;
            if (seen == grid)
                return __atomic_load_n(&device->status_host[0], __ATOMIC_ACQUIRE) == seq ? BNN_ERANGE : BNN_OK;
            // ~2 ms at a few GHz of time-stamp counter
            if ((i & 1023u) == 1023u && __builtin_readcyclecounter() - t0 > 8000000ull)
                break;
            __builtin_ia32_pause();
        }
    }
    return finish(device, hipSuccess, seq);
}

BNN_Status finish(BNN_Device device, hipError_t e, uint64_t seq) {
    if (e == hipSuccess)
        e = hipStreamSynchronize(device->stream);
    if (e == hipSuccess && device->ev_used)
        e = resolve_timing(device);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_EIO;
    }
    if (__atomic_load_n(&device->status_host[0], __ATOMIC_ACQUIRE) == seq)
        return BNN_ERANGE;
    return BNN_OK;
}

}  // namespace

namespace {

// Rows per launch chunk of a multi-row job and the scratch bytes of one chunk's
// quantised rows, for a scratch of `cap` bytes that also holds the chunk's staging
// rows when the output view is not naturally aligned.  chunk = 0: not even one row fits.
void chunk_rows(const JobPlan& p, uint32_t rows, bool mfma, size_t cap, size_t* chunk_out, size_t* rows_bytes) {
    size_t a, b, c;
    // planes + group sums + row scale (+ Q rows) (+ staging), unrounded
    const size_t per_row = (size_t)p.m->groups * (kPlaneWords * 4u + 4u) + 4u + (mfma ? p.m->k : 0u) +
                           (p.out_aligned ? 0u : p.out_row);
    // each of the (at most five) regions is rounded up to 256 bytes once per chunk
    const size_t slack = 5 * 256;
    size_t chunk = rows < kScratchRowsCap ? rows : kScratchRowsCap;
    const size_t fit = cap > slack ? (cap - slack) / per_row : 0;
    if (chunk > fit)
        chunk = fit;
    *chunk_out = chunk;
    *rows_bytes = chunk ? row_scratch_bytes(p, chunk, &a, &b, &c, nullptr, mfma) : 0;
}

// One row, aligned views, K <= kFusedMaxWidth: check, quantisation and dots in one
// launch of the fused kernel, read straight from the input view -- no scratch.
// `mirror`: also write an F32 output row into the device's pinned host mirror.
BNN_Status run_single_row(BNN_Device device, const BNN_Job* job, const JobPlan& p, bool allow_mirror) {
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    FusedArgs fa = {};
    fa.jobs = nullptr;
    fa.njobs = 1;
    fa.kind = p.f32_in ? PRE_ROW : PRE_ROW_I8;
    fa.dot_out = p.dot_out ? 1 : 0;
    fa.width = p.m->k;
    fa.row = reinterpret_cast<const float*>(p.in_base);
    fa.post = POST_NONE;
    fa.inl[0] = FusedJob{p.m->wbits, p.m->wscale, reinterpret_cast<float*>(p.out_base), p.m->n, p.m->tiles, 0, 0};
    fa.inline_jobs = 1;
    // F32 outputs of buffers whose device address was never handed out are mirrored
    // into pinned host memory by the same kernel
    const bool mirror =
        allow_mirror && !p.dot_out && !job->output.buffer->exposed && ensure_mirror(device) == BNN_OK;
    fa.mirror = mirror ? device->mirror : nullptr;
    // one workgroup per tile up to one per CU (a CU holds one 1024-thread workgroup of
    // the kernel at a time); beyond that workgroups loop over tiles
    const uint32_t cus = device->cu_count ? device->cu_count : 256u;
    const uint32_t grid = p.m->tiles < cus ? p.m->tiles : cus;
    const uint64_t seq = ++device->seq;
    fa.done_flags = grid <= kDoneFlagSlots ? device->status_host + kDoneFlagWord : nullptr;
    const hipError_t e = timed(device, KK_DOT, [&] {
        return launch_fused(device->stream, fa, p.m->tiles, grid, seq, device->flag_dev, device->status_host);
    });
    const BNN_Status result =
        fa.done_flags ? finish_signalled(device, e, seq, grid) : finish(device, e, seq);
    if (result == BNN_OK && mirror) {
        device->mirror_buf = job->output.buffer;
        device->mirror_off = job->output.offset;
        device->mirror_bytes = p.out_row;
    }
    return result;
}

// A multi-row job (or a single row the fused kernel does not take) in chunks of
// `chunk` rows whose quantised forms occupy the first `rows_bytes` of `scratch`,
// followed by the chunk's staging rows when the output view is not aligned.
// mfma: the rows run on the matrix cores (the matrix's +1/-1 copy must exist).
BNN_Status run_rows(BNN_Device device, const BNN_Job* job, const JobPlan& p, bool mfma, unsigned char* scratch,
                    size_t chunk, size_t rows_bytes, hipError_t e) {
    const uint32_t rows = job->rows;
    unsigned char* staging = scratch + rows_bytes;
    const uint64_t seq = ++device->seq;
    if (e == hipSuccess && chunk < rows) {
        // every row is checked before any chunk writes output
        const PrepJob all = make_prep(p, p.in_base, rows, scratch);
        e = timed(device, KK_PREP, [&] {
            return launch_prep(device->stream, all, true, seq, device->flag_dev, device->status_host);
        });
    }
    for (size_t r0 = 0; e == hipSuccess && r0 < rows; r0 += chunk) {
        const uint32_t rc = (uint32_t)((rows - r0) < chunk ? (rows - r0) : chunk);
        const PrepJob pj = make_prep(p, p.in_base + r0 * p.in_stride, rc, scratch, mfma);
        e = timed(device, KK_PREP, [&] {
            return launch_prep(device->stream, pj, false, seq, device->flag_dev, device->status_host);
        });
        if (e != hipSuccess)
            break;
        unsigned char* dst = p.out_aligned ? p.out_base + r0 * p.out_stride : staging;
        const size_t dst_stride = p.out_aligned ? p.out_stride : p.out_row;
        if (mfma) {
            const GemmJob gj = make_gemm(p, pj, dst, dst_stride);
            e = timed(device, KK_GEMM,
                      [&] { return launch_gemm(device->stream, gj, device->cu_count, seq, device->flag_dev); });
        } else {
            const DotJob dj = make_dot(p, pj, dst, dst_stride);
            e = timed(device, KK_DOT,
                      [&] { return launch_dot(device->stream, dj, device->cu_count, seq, device->flag_dev); });
        }
        if (e == hipSuccess && !p.out_aligned)
            e = timed(device, KK_SCATTER, [&] {
                return launch_scatter(device->stream, staging, p.out_row, p.out_base + r0 * p.out_stride,
                                      p.out_stride, p.out_row, rc, seq, device->flag_dev);
            });
    }
    return finish(device, e, seq);
}

bool single_row_path(const BNN_Job* job, const JobPlan& p) {
    return job->rows == 1 && p.in_aligned && p.out_aligned && p.m->k <= kFusedMaxWidth && p.m->k % kGroup == 0;
}

}  // namespace

EXPORT BNN_Status BNN_Execute(BNN_Device device, const BNN_Job* job) {
    if (device != nullptr)
        device->mirror_buf = nullptr;
    JobPlan p;
    BNN_Status st = plan_job(device, job, &p);
    if (st != BNN_OK)
        return st;
    // one row of GEMV_F32 (the reference engine's only call, linear.c:169-200), GEMV or DOT_GROUPS
    if (single_row_path(job, p))
        return run_single_row(device, job, p, true);

    // rows in chunks that fit the device's scratch (allocated with the device)
    const bool mfma = job->rows >= kMfmaMinRows;
    size_t chunk = 0, rows_bytes = 0;
    chunk_rows(p, job->rows, mfma, device->scratch_bytes, &chunk, &rows_bytes);
    if (chunk == 0)
        return BNN_ENOMEM;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    return run_rows(device, job, p, mfma, device->scratch, chunk, rows_bytes, hipSuccess);
}

// BNN_Execute without any allocation: the quantised rows (and staging rows for
// unaligned output views) live in this GPU's fixed `scratch` array, multi-row jobs
// run on the bit-plane kernels in chunks that fit it, and single-row outputs are
// not mirrored into host memory.
EXPORT BNN_Status BNNX_ExecuteNoAlloc(BNN_Device device, const BNN_Job* job) {
    if (device != nullptr)
        device->mirror_buf = nullptr;
    JobPlan p;
    BNN_Status st = plan_job(device, job, &p);
    if (st != BNN_OK)
        return st;
    if (single_row_path(job, p))
        return run_single_row(device, job, p, false);
    size_t chunk = 0, rows_bytes = 0;
    chunk_rows(p, job->rows, false, kStaticScratchBytes, &chunk, &rows_bytes);
    if (chunk == 0 || device->static_scratch == nullptr)
        return BNN_ENOMEM;  // one row's quantised form and staging exceed the fixed scratch
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    // every handle on this GPU shares the array: one call at a time uses it
    const std::lock_guard<std::mutex> hold(g_static_use[device->ordinal]);
    return run_rows(device, job, p, false, device->static_scratch, chunk, rows_bytes, hipSuccess);
}

// ---------------------------------------------------------------------------
// Batch extension (include/bnn-accelerator-hip.h; no reference counterpart)
// ---------------------------------------------------------------------------

namespace {

struct Extent {
    const void* buffer;
    size_t begin, end;
};

bool extent_less(const Extent& a, const Extent& b) {
    return a.buffer != b.buffer ? (uintptr_t)a.buffer < (uintptr_t)b.buffer : a.begin < b.begin;
}

// Grow-only pinned + device memory for the batch job tables.
BNN_Status ensure_tables(BNN_Device d, size_t bytes) {
    if (bytes > d->table_dev_bytes) {
        if (d->table_dev)
            (void)hipFree(d->table_dev);
        d->table_dev = nullptr;
        d->table_dev_bytes = 0;
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return BNN_ENOMEM;
        }
        d->table_dev = static_cast<unsigned char*>(p);
        d->table_dev_bytes = bytes;
        d->generation++;
    }
    if (bytes > d->table_host_bytes) {
        if (d->table_host)
            (void)hipHostFree(d->table_host);
        d->table_host = nullptr;
        d->table_host_bytes = 0;
        void* p = nullptr;
        if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return BNN_ENOMEM;
        }
        d->table_host = static_cast<unsigned char*>(p);
        d->table_host_bytes = bytes;
    }
    return BNN_OK;
}

// All checks of a batch (per job as BNN_Execute, then the batch rules) and the
// sizes of its scratch and job tables.
struct BatchPlan {
    JobPlan* plans = nullptr;
    uint32_t count = 0;
    bool needs_nearest = false, uniform = true;
    uint64_t prep_blocks = 0, dot_items_total = 0;
    size_t scratch_bytes = 0;
    uint32_t max_groups = 0;
    // tables: PrepJob[count] | DotJob[count] | prep block->job (unless one row per job) |
    // dot item->job (non-uniform only)
    size_t prep_tab = 0, dot_tab = 0, prep_map = 0, dot_map = 0, tables = 0;
    ~BatchPlan() { free(plans); }
};

BNN_Status plan_batch(BNN_Device device, const BNN_Job* jobs, uint32_t count, BatchPlan* bp) {
    bp->plans = static_cast<JobPlan*>(malloc(sizeof(JobPlan) * count));
    bp->count = count;
    Extent* outs = static_cast<Extent*>(malloc(sizeof(Extent) * count));
    const void** ins = static_cast<const void**>(malloc(sizeof(void*) * count));
    BNN_Status st = bp->plans && outs && ins ? BNN_OK : BNN_ENOMEM;
    for (uint32_t i = 0; st == BNN_OK && i < count; ++i) {
        st = plan_job(device, &jobs[i], &bp->plans[i]);
        if (st != BNN_OK)
            break;
        const JobPlan& p = bp->plans[i];
        if (!p.in_aligned || !p.out_aligned || jobs[i].rows > kScratchRowsCap) {
            st = BNN_ENOTSUP;
            break;
        }
        bp->needs_nearest = bp->needs_nearest || !p.dot_out;
        size_t a, b, c;
        bp->scratch_bytes += row_scratch_bytes(p, jobs[i].rows, &a, &b, &c);
        bp->prep_blocks += jobs[i].rows;
        bp->max_groups = p.m->groups > bp->max_groups ? p.m->groups : bp->max_groups;
        outs[i].buffer = jobs[i].output.buffer;
        outs[i].begin = jobs[i].output.offset;
        outs[i].end = jobs[i].output.offset + (size_t)(jobs[i].rows - 1) * p.out_stride + p.out_row;
        ins[i] = jobs[i].input.buffer;
    }
    // work items per job depend on the batch's largest group count
    for (uint32_t i = 0; st == BNN_OK && i < count; ++i) {
        const uint64_t items = dot_items(bp->plans[i].m->tiles, jobs[i].rows, bp->max_groups);
        bp->uniform = bp->uniform && items == dot_items(bp->plans[0].m->tiles, jobs[0].rows, bp->max_groups);
        bp->dot_items_total += items;
    }
    // the jobs run concurrently: no output buffer may be an input buffer, and
    // outputs sharing a buffer may not overlap
    if (st == BNN_OK) {
        std::sort(ins, ins + count);
        std::sort(outs, outs + count, extent_less);
        for (uint32_t i = 0; st == BNN_OK && i < count; ++i) {
            if (std::binary_search(ins, ins + count, outs[i].buffer))
                st = BNN_EINVAL;
            else if (i > 0 && outs[i].buffer == outs[i - 1].buffer && outs[i].begin < outs[i - 1].end)
                st = BNN_EINVAL;
        }
        if (st == BNN_OK && (bp->prep_blocks > 0x7fffffffu || bp->dot_items_total > 0x7fffffffu))
            st = BNN_ENOTSUP;
    }
    free(outs);
    free(ins);
    if (st == BNN_OK) {
        bp->prep_tab = round_up(sizeof(PrepJob) * count, 256);
        bp->dot_tab = round_up(sizeof(DotJob) * count, 256);
        bp->prep_map = bp->prep_blocks == count ? 0 : round_up(4u * bp->prep_blocks, 256);
        bp->dot_map = bp->uniform ? 0 : round_up(4u * bp->dot_items_total, 256);
        bp->tables = bp->prep_tab + bp->dot_tab + bp->prep_map + bp->dot_map;
    }
    return st;
}

// Writes the job tables of a planned batch into host memory, with the rows'
// quantised forms placed consecutively from 'scratch' (a device address).
void fill_batch_tables(const BatchPlan& bp, const BNN_Job* jobs, unsigned char* scratch, unsigned char* host) {
    PrepJob* hp = reinterpret_cast<PrepJob*>(host);
    DotJob* hd = reinterpret_cast<DotJob*>(host + bp.prep_tab);
    uint32_t* hpm = reinterpret_cast<uint32_t*>(host + bp.prep_tab + bp.dot_tab);
    uint32_t* hdm = reinterpret_cast<uint32_t*>(host + bp.prep_tab + bp.dot_tab + bp.prep_map);
    size_t soff = 0;
    uint32_t pb = 0, di = 0;
    for (uint32_t i = 0; i < bp.count; ++i) {
        const JobPlan& p = bp.plans[i];
        const uint32_t rows = jobs[i].rows;
        size_t a, b, c;
        hp[i] = make_prep(p, p.in_base, rows, scratch + soff);
        hp[i].first_block = pb;
        soff += row_scratch_bytes(p, rows, &a, &b, &c);
        hd[i] = make_dot(p, hp[i], p.out_base, p.out_stride);
        hd[i].first_block = di;
        for (uint32_t r = 0; r < rows; ++r, ++pb)
            if (bp.prep_map)
                hpm[pb] = i;
        const uint32_t items = dot_items(p.m->tiles, rows, bp.max_groups);
        if (!bp.uniform)
            for (uint32_t r = 0; r < items; ++r)
                hdm[di + r] = i;
        di += items;
    }
}

// The two launches of a batch whose tables start at 'tables' on the device.
hipError_t launch_batch(BNN_Device device, const unsigned char* tables, size_t prep_tab, size_t dot_tab,
                        size_t prep_map, uint32_t prep_blocks, uint32_t items, uint32_t uniform_items,
                        uint32_t max_groups, bool scales, uint64_t seq, uint64_t* status) {
    const PrepJob* dp = reinterpret_cast<const PrepJob*>(tables);
    const DotJob* dd = reinterpret_cast<const DotJob*>(tables + prep_tab);
    // no map (prep_map == 0) when every job has one row: prep block b is job b
    const uint32_t* dpm = prep_map ? reinterpret_cast<const uint32_t*>(tables + prep_tab + dot_tab) : nullptr;
    const uint32_t* ddm =
        uniform_items ? nullptr : reinterpret_cast<const uint32_t*>(tables + prep_tab + dot_tab + prep_map);
    hipError_t e = timed(device, KK_PREP, [&] {
        return launch_prep_batch(device->stream, dp, dpm, prep_blocks, max_groups, seq, device->flag_dev, status);
    });
    if (e == hipSuccess)
        e = timed(device, KK_DOT, [&] {
            return launch_dot_batch(device->stream, dd, ddm, items, uniform_items, max_groups, scales,
                                    device->cu_count, seq, device->flag_dev);
        });
    return e;
}

}  // namespace

static BNN_Status run_cached_batch(BNN_Device device);

EXPORT BNN_Status BNNX_ExecuteBatch(BNN_Device device, const BNN_Job* jobs, uint32_t count) {
    if (device != nullptr)
        device->mirror_buf = nullptr;
    if (device == nullptr || jobs == nullptr || count == 0)
        return BNN_EINVAL;
    // An identical job array of the same resource generation reuses the tables
    // already on the device.  Its per-job checks depend only on the job bytes
    // (identical), on matrix/buffer objects (immutable while the generation is
    // unchanged) and on the host rounding mode, so only the latter is re-checked.
    const bool cached = device->batch_jobs != nullptr && device->batch_count == count &&
                        device->batch_generation == device->generation &&
                        memcmp(device->batch_jobs, jobs, sizeof(BNN_Job) * count) == 0;
    if (cached) {
        if (device->batch_needs_nearest && fegetround() != FE_TONEAREST) {
            // same outcome as the full checks: the first job that is not DOT_GROUPS fails
            for (uint32_t i = 0; i < count; ++i) {
                JobPlan p;
                const BNN_Status st = plan_job(device, &jobs[i], &p);
                if (st != BNN_OK)
                    return st;
            }
        }
        if (hipSetDevice(device->ordinal) != hipSuccess)
            return BNN_EIO;
        return run_cached_batch(device);
    }
    BatchPlan bp;
    BNN_Status st = plan_batch(device, jobs, count, &bp);
    if (st != BNN_OK)
        return st;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    st = ensure_scratch(device, bp.scratch_bytes);
    if (st == BNN_OK)
        st = ensure_tables(device, bp.tables);
    if (st == BNN_OK && count > device->batch_cap) {
        BNN_Job* copy = static_cast<BNN_Job*>(realloc(device->batch_jobs, sizeof(BNN_Job) * count));
        if (copy == nullptr) {
            st = BNN_ENOMEM;
        } else {
            device->batch_jobs = copy;
            device->batch_cap = count;
        }
    }
    if (st != BNN_OK) {
        device->batch_count = 0;
        return st;
    }
    fill_batch_tables(bp, jobs, device->scratch, device->table_host);
    if (hipMemcpyAsync(device->table_dev, device->table_host, bp.tables, hipMemcpyHostToDevice, device->stream) !=
        hipSuccess) {
        (void)hipGetLastError();
        device->batch_count = 0;
        return BNN_EIO;
    }
    memcpy(device->batch_jobs, jobs, sizeof(BNN_Job) * count);
    device->batch_count = count;
    device->batch_generation = device->generation;
    device->batch_prep_blocks = (uint32_t)bp.prep_blocks;
    device->batch_items = (uint32_t)bp.dot_items_total;
    device->batch_uniform_items = bp.uniform ? dot_items(bp.plans[0].m->tiles, jobs[0].rows, bp.max_groups) : 0u;
    device->batch_max_groups = bp.max_groups;
    device->batch_prep_tab = bp.prep_tab;
    device->batch_dot_tab = bp.dot_tab;
    device->batch_prep_map = bp.prep_map;
    device->batch_tables = bp.tables;
    device->batch_needs_nearest = bp.needs_nearest;
    return run_cached_batch(device);
}

// Launches the batch whose tables are on the device (the last one built).
static BNN_Status run_cached_batch(BNN_Device device) {
    const uint64_t seq = ++device->seq;
    const hipError_t e = launch_batch(device, device->table_dev, device->batch_prep_tab, device->batch_dot_tab,
                                      device->batch_prep_map, device->batch_prep_blocks, device->batch_items,
                                      device->batch_uniform_items, device->batch_max_groups,
                                      device->batch_needs_nearest, seq, device->status_host);
    if (e != hipSuccess)
        device->batch_count = 0;
    return finish(device, e, seq);
}

// ---------------------------------------------------------------------------
// Prepared batches (asynchronous launches) and device pointers of buffers
// ---------------------------------------------------------------------------

EXPORT BNN_Status BNNX_BatchCreate(BNN_Device device, const BNN_Job* jobs, uint32_t count, BNNX_Batch* out_batch) {
    if (out_batch == nullptr)
        return BNN_EINVAL;
    *out_batch = nullptr;
    if (device == nullptr || jobs == nullptr || count == 0)
        return BNN_EINVAL;
    BatchPlan bp;
    BNN_Status st = plan_batch(device, jobs, count, &bp);
    if (st != BNN_OK)
        return st;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    BNNX_Batch b = static_cast<BNNX_Batch>(calloc(1, sizeof(bnnx_batch)));
    unsigned char* host = static_cast<unsigned char*>(malloc(bp.tables));
    if (b == nullptr || host == nullptr) {
        free(b);
        free(host);
        return BNN_ENOMEM;
    }
    const size_t scratch_at = round_up(bp.tables, 256);
    void* mem = nullptr;
    if (hipMalloc(&mem, scratch_at + bp.scratch_bytes) != hipSuccess) {
        (void)hipGetLastError();
        free(b);
        free(host);
        return BNN_ENOMEM;
    }
    b->mem = static_cast<unsigned char*>(mem);
    fill_batch_tables(bp, jobs, b->mem + scratch_at, host);
    hipError_t e = hipMemcpy(b->mem, host, bp.tables, hipMemcpyHostToDevice);
    free(host);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(b->mem);
        free(b);
        return BNN_EIO;
    }
    b->device = device;
    b->retired = device->retired;
    b->prep_blocks = (uint32_t)bp.prep_blocks;
    b->items = (uint32_t)bp.dot_items_total;
    b->uniform_items = bp.uniform ? dot_items(bp.plans[0].m->tiles, jobs[0].rows, bp.max_groups) : 0u;
    b->max_groups = bp.max_groups;
    b->prep_tab = bp.prep_tab;
    b->dot_tab = bp.dot_tab;
    b->prep_map = bp.prep_map;
    b->needs_nearest = bp.needs_nearest;
    device->live_batches++;
    *out_batch = b;
    return BNN_OK;
}

namespace {
struct Span {
    uintptr_t begin, end;
};
bool spans_overlap(const Span& x, const Span& y) { return x.begin < y.end && y.begin < x.end; }
Span span_of(const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    return Span{a, p ? a + bytes : a};
}
}  // namespace

EXPORT BNN_Status BNNX_BatchCreateFusedPost(BNN_Device device, const BNN_Job* jobs, uint32_t count,
                                            const BNNX_PreOp* pre, const BNNX_PostOp* post, BNNX_Batch* out_batch) {
    if (out_batch == nullptr)
        return BNN_EINVAL;
    *out_batch = nullptr;
    if (device == nullptr || jobs == nullptr || count == 0 || pre == nullptr)
        return BNN_EINVAL;
    if (pre->kind != BNNX_PRE_ROW && pre->kind != BNNX_PRE_RMSNORM && pre->kind != BNNX_PRE_SILU_MUL)
        return BNN_EINVAL;
    const int32_t post_kind = post ? post->kind : BNNX_POST_NONE;
    if (post_kind != BNNX_POST_NONE && post_kind != BNNX_POST_SILU_MUL)
        return BNN_EINVAL;
    const bool paired = post_kind == BNNX_POST_SILU_MUL;
    if (paired && (count % 2u != 0 || post->out == nullptr))
        return BNN_EINVAL;
    const uint32_t width = pre->width;
    if (width == 0 || width % kGroup != 0)
        return BNN_EINVAL;
    if ((pre->kind == BNNX_PRE_RMSNORM && (pre->a == nullptr || pre->gain == nullptr)) ||
        (pre->kind == BNNX_PRE_SILU_MUL && (pre->a == nullptr || pre->b == nullptr)))
        return BNN_EINVAL;
    const size_t row_bytes = (size_t)width * 4u;
    // everything the workgroups read while others write
    Span reads[5];
    uint32_t nreads = 0;
    if (pre->kind != BNNX_PRE_ROW) {
        reads[nreads++] = span_of(pre->a, row_bytes);
        if (pre->b)
            reads[nreads++] = span_of(pre->b, row_bytes);
        if (pre->kind == BNNX_PRE_RMSNORM)
            reads[nreads++] = span_of(pre->gain, row_bytes);
    }
    const float* a_out = pre->kind == BNNX_PRE_RMSNORM ? pre->a_out : nullptr;
    if (a_out) {
        const Span w = span_of(a_out, row_bytes);
        for (uint32_t r = 0; r < nreads; ++r)
            if (spans_overlap(w, reads[r]))
                return BNN_EINVAL;
    }
    Span* outs = static_cast<Span*>(malloc(sizeof(Span) * (count + 2u)));
    FusedJob* table = static_cast<FusedJob*>(malloc(sizeof(FusedJob) * count));
    BNN_Status st = outs && table ? BNN_OK : BNN_ENOMEM;
    uint32_t tiles = 0;
    const unsigned char* row = nullptr;
    for (uint32_t i = 0; st == BNN_OK && i < count; ++i) {
        JobPlan p;
        st = plan_job(device, &jobs[i], &p);
        if (st != BNN_OK)
            break;
        if (jobs[i].operation != BNN_OP_GEMV_F32 || !p.out_aligned || p.m->k > kFusedMaxWidth) {
            st = BNN_ENOTSUP;
            break;
        }
        if (p.m->k != width) {
            st = BNN_EINVAL;
            break;
        }
        if (pre->kind == BNNX_PRE_ROW) {
            if (!p.in_aligned) {
                st = BNN_ENOTSUP;
                break;
            }
            if (i == 0) {
                row = p.in_base;
                reads[nreads++] = span_of(row, row_bytes);
            } else if (p.in_base != row) {
                st = BNN_EINVAL;
                break;
            }
        }
        outs[i] = span_of(p.out_base, p.out_row);
        table[i] = FusedJob{p.m->wbits, p.m->wscale, reinterpret_cast<float*>(p.out_base), p.m->n, p.m->tiles, tiles, 0};
        tiles += p.m->tiles;
    }
    uint32_t post_n = 0;
    if (st == BNN_OK && paired) {
        // pairs (p, m + p) of equal length; tiles count half-tiles of the pairs
        const uint32_t m = count / 2u;
        tiles = 0;
        for (uint32_t q = 0; st == BNN_OK && q < m; ++q) {
            if (table[q].n != table[m + q].n) {
                st = BNN_EINVAL;
                break;
            }
            table[q].first_tile = tiles;
            table[q].post_off = post_n;
            tiles += 2u * table[q].tiles;
            post_n += table[q].n;
        }
    }
    if (st == BNN_OK) {
        uint32_t nouts = count;
        if (a_out)
            outs[nouts++] = span_of(a_out, row_bytes);
        if (paired)
            outs[nouts++] = span_of(post->out, (size_t)post_n * 4u);
        std::sort(outs, outs + nouts, [](const Span& x, const Span& y) { return x.begin < y.begin; });
        for (uint32_t i = 0; st == BNN_OK && i < nouts; ++i) {
            if (i > 0 && outs[i].begin < outs[i - 1].end)
                st = BNN_EINVAL;
            for (uint32_t r = 0; st == BNN_OK && r < nreads; ++r)
                if (spans_overlap(outs[i], reads[r]))
                    st = BNN_EINVAL;
        }
    }
    free(outs);
    if (st == BNN_OK && hipSetDevice(device->ordinal) != hipSuccess)
        st = BNN_EIO;
    BNNX_Batch b = nullptr;
    if (st == BNN_OK) {
        b = static_cast<BNNX_Batch>(calloc(1, sizeof(bnnx_batch)));
        void* mem = nullptr;
        if (b == nullptr || hipMalloc(&mem, sizeof(FusedJob) * count) != hipSuccess) {
            (void)hipGetLastError();
            st = BNN_ENOMEM;
        } else if (hipMemcpy(mem, table, sizeof(FusedJob) * count, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(mem);
            st = BNN_EIO;
        } else {
            b->mem = static_cast<unsigned char*>(mem);
        }
    }
    // the job of a tile in one step when the jobs (pairs) start at multiples of a power of two
    uint32_t walk_shift = 32;
    if (st == BNN_OK) {
        const uint32_t nwalk = paired ? count / 2u : count;
        for (uint32_t sh = 0; sh < 31u && walk_shift == 32u; ++sh) {
            bool fits = true;
            for (uint32_t i = 0; fits && i < nwalk; ++i)
                fits = (uint64_t)table[i].first_tile == ((uint64_t)i << sh);
            if (fits)
                walk_shift = sh;
        }
    }
    FusedJob inl[kFusedInline] = {};
    const bool inline_jobs = count <= kFusedInline;
    for (uint32_t i = 0; st == BNN_OK && inline_jobs && i < count; ++i)
        inl[i] = table[i];
    free(table);
    if (st != BNN_OK) {
        free(b);
        return st;
    }
    b->device = device;
    b->retired = device->retired;
    b->needs_nearest = true;
    b->fused = true;
    b->fused_tiles = tiles;
    // one workgroup per tile up to one per CU (a CU holds one 1024-thread workgroup of the
    // kernel at a time: a second one per CU would start only as the first ends); beyond
    // that workgroups loop over tiles (each produces the row once)
    const uint32_t cus = device->cu_count ? device->cu_count : 256u;
    b->fused_grid = tiles < cus ? tiles : cus;
    FusedArgs& fa = b->fused_args;
    fa.jobs = reinterpret_cast<const FusedJob*>(b->mem);
    fa.njobs = count;
    fa.kind = pre->kind;
    fa.width = width;
    fa.eps = pre->eps;
    fa.a = pre->kind == BNNX_PRE_ROW ? nullptr : pre->a;
    fa.b = pre->kind == BNNX_PRE_ROW ? nullptr : pre->b;
    fa.gain = pre->kind == BNNX_PRE_RMSNORM ? pre->gain : nullptr;
    fa.a_out = const_cast<float*>(a_out);
    fa.row = reinterpret_cast<const float*>(row);
    fa.err = pre->kind == BNNX_PRE_RMSNORM ? pre->err : nullptr;
    fa.err_code = pre->err_code;
    fa.post = paired ? POST_SILU_MUL : POST_NONE;
    fa.post_out = paired ? post->out : nullptr;
    fa.walk_shift = walk_shift;
    for (uint32_t i = 0; i < kFusedInline; ++i)
        fa.inl[i] = inl[i];
    fa.inline_jobs = inline_jobs ? 1u : 0u;
    device->live_batches++;
    *out_batch = b;
    return BNN_OK;
}

EXPORT BNN_Status BNNX_BatchCreateFused(BNN_Device device, const BNN_Job* jobs, uint32_t count, const BNNX_PreOp* pre,
                                        BNNX_Batch* out_batch) {
    return BNNX_BatchCreateFusedPost(device, jobs, count, pre, nullptr, out_batch);
}

EXPORT BNN_Status BNNX_BatchCheck(BNNX_Batch batch) {
    if (batch == nullptr || batch->retired != batch->device->retired)  // a matrix or buffer it uses may be gone
        return BNN_EINVAL;
    if (batch->needs_nearest && fegetround() != FE_TONEAREST)
        return BNN_ENOTSUP;
    return BNN_OK;
}

EXPORT BNN_Status BNNX_BatchLaunch(BNNX_Batch batch) {
    const BNN_Status st = BNNX_BatchCheck(batch);
    if (st != BNN_OK)
        return st;
    BNN_Device device = batch->device;
    device->mirror_buf = nullptr;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    const uint64_t seq = ++device->seq;
    if (device->async_first_seq == 0)
        device->async_first_seq = seq;
    const hipError_t e =
        batch->chain ? timed(device, KK_DOT,
                             [&] { return launch_chain(device->stream, batch->chain_args, seq, device->flag_dev,
                                                       device->status_host + 1); })
        : batch->fused ? timed(device, KK_DOT,
                             [&] {
                                 return launch_fused(device->stream, batch->fused_args, batch->fused_tiles,
                                                     batch->fused_grid, seq, device->flag_dev,
                                                     device->status_host + 1);
                             })
                     : launch_batch(device, batch->mem, batch->prep_tab, batch->dot_tab, batch->prep_map,
                                    batch->prep_blocks, batch->items, batch->uniform_items, batch->max_groups,
                                    batch->needs_nearest, seq, device->status_host + 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_EIO;
    }
    return BNN_OK;
}

EXPORT void BNNX_BatchDestroy(BNNX_Batch batch) {
    if (batch == nullptr)
        return;
    (void)hipSetDevice(batch->device->ordinal);
    (void)hipStreamSynchronize(batch->device->stream);
    (void)hipFree(batch->mem);
    batch->device->live_batches--;
    free(batch);
}

EXPORT BNN_Status BNNX_DeviceSynchronize(BNN_Device device) {
    if (device == nullptr)
        return BNN_EINVAL;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    hipError_t e = hipStreamSynchronize(device->stream);
    if (e == hipSuccess && device->ev_used)
        e = resolve_timing(device);
    const uint64_t first = device->async_first_seq;
    device->async_first_seq = 0;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return BNN_EIO;
    }
    if (first != 0 && __atomic_load_n(&device->status_host[1], __ATOMIC_ACQUIRE) >= first)
        return BNN_ERANGE;
    return BNN_OK;
}

namespace {
// An F32 view of `rows` rows of `width` values for a chained batch: on the device, in
// bounds, rows 4-byte aligned.
BNN_Status chain_view(BNN_Device device, const BNN_BufferView& v, uint32_t width, uint32_t rows,
                      unsigned char** base, uint64_t* stride) {
    if (v.buffer == nullptr || v.buffer->device != device || v.type != BNN_TYPE_F32)
        return BNN_EINVAL;
    const size_t row = (size_t)width * 4u;
    const size_t st = v.row_stride ? v.row_stride : row;
    if (st < row)
        return BNN_EINVAL;
    if (!rows_fit(v.buffer->size, v.offset, st, row, rows))
        return BNN_ERANGE;
    *base = v.buffer->dev + v.offset;
    *stride = st;
    return (((uintptr_t)*base | st) & 3u) == 0 ? BNN_OK : BNN_ENOTSUP;
}
}  // namespace

EXPORT BNN_Status BNNX_BatchCreateChain(BNN_Device device, const BNNX_ChainLayer* layers, uint32_t count,
                                        BNN_BufferView input, BNN_BufferView output, uint32_t rows,
                                        BNNX_Batch* out_batch) {
    if (out_batch == nullptr)
        return BNN_EINVAL;
    *out_batch = nullptr;
    if (device == nullptr || layers == nullptr || count == 0 || rows == 0)
        return BNN_EINVAL;
    if (count > kChainMaxLayers || rows > kChainMaxRows)
        return BNN_ENOTSUP;
    ChainLayer table[kChainMaxLayers] = {};
    for (uint32_t i = 0; i < count; ++i) {
        const BNN_Matrix m = layers[i].matrix;
        if (m == nullptr || m->device != device || (layers[i].post_scale == nullptr) != (layers[i].post_bias == nullptr))
            return BNN_EINVAL;
        if (i > 0 && m->k != layers[i - 1].matrix->n)  // each layer reads the previous one's outputs
            return BNN_EINVAL;
        if (m->k > kChainMaxWidth || m->n > kChainMaxWidth)
            return BNN_ENOTSUP;
        table[i] = ChainLayer{m->wbits, m->wscale, layers[i].post_scale, layers[i].post_bias,
                              m->k, m->n, m->groups, m->tiles, layers[i].relu != 0, 0u};
    }
    if (input.buffer != nullptr && input.buffer == output.buffer)
        return BNN_EINVAL;
    ChainArgs args = {};
    unsigned char* in_base = nullptr;
    BNN_Status st = chain_view(device, input, layers[0].matrix->k, rows, &in_base, &args.in_stride);
    args.in = in_base;
    if (st == BNN_OK)
        st = chain_view(device, output, layers[count - 1].matrix->n, rows, &args.out, &args.out_stride);
    if (st != BNN_OK)
        return st;
    if (fegetround() != FE_TONEAREST)
        return BNN_ENOTSUP;
    if (hipSetDevice(device->ordinal) != hipSuccess)
        return BNN_EIO;
    BNNX_Batch b = static_cast<BNNX_Batch>(calloc(1, sizeof(bnnx_batch)));
    if (b == nullptr)
        return BNN_ENOMEM;
    void* mem = nullptr;
    if (hipMalloc(&mem, sizeof(ChainLayer) * count) != hipSuccess) {
        (void)hipGetLastError();
        free(b);
        return BNN_ENOMEM;
    }
    if (hipMemcpy(mem, table, sizeof(ChainLayer) * count, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(mem);
        free(b);
        return BNN_EIO;
    }
    b->mem = static_cast<unsigned char*>(mem);
    b->device = device;
    b->retired = device->retired;
    b->needs_nearest = true;
    b->chain = true;
    args.layers = static_cast<const ChainLayer*>(mem);
    args.count = count;
    args.rows = rows;
    args.k0 = layers[0].matrix->k;
    b->chain_args = args;
    device->live_batches++;
    *out_batch = b;
    return BNN_OK;
}

EXPORT BNN_Status BNNX_BufferDevicePointer(BNN_Buffer buffer, void** out_pointer) {
    if (out_pointer == nullptr)
        return BNN_EINVAL;
    *out_pointer = nullptr;
    if (buffer == nullptr)
        return BNN_EINVAL;
    buffer->exposed = true;
    if (buffer->device->mirror_buf == buffer)
        buffer->device->mirror_buf = nullptr;
    *out_pointer = buffer->dev;
    return BNN_OK;
}

EXPORT const char* BNN_StatusString(BNN_Status status) {
    switch (status) {
    case BNN_OK:
        return "success";
    case BNN_EINVAL:
        return "invalid argument";
    case BNN_ENOMEM:
        return "out of memory";
    case BNN_ENOTSUP:
        return "unsupported operation or configuration";
    case BNN_ERANGE:
        return "buffer or input range error";
    case BNN_EBUSY:
        return "device still owns resources";
    case BNN_EIO:
        return "device I/O error";
    case BNN_ETIMEOUT:
        return "device timeout";
    default:
        return "unknown status";
    }
}

// ---------------------------------------------------------------------------
// Extensions (include/bnn-accelerator-hip.h); no reference counterpart.
// ---------------------------------------------------------------------------

EXPORT BNN_Status BNNX_DeviceStream(BNN_Device device, void** out_stream) {
    if (device == nullptr || out_stream == nullptr)
        return BNN_EINVAL;
    *out_stream = device->stream;
    return BNN_OK;
}

EXPORT BNN_Status BNNX_KernelTiming(BNN_Device device, int enable) {
    if (device == nullptr)
        return BNN_EINVAL;
    if (enable) {
        const BNN_Status st = ensure_events(device);
        if (st != BNN_OK)
            return st;
    }
    device->timing = enable != 0;
    device->ev_used = 0;
    for (int i = 0; i < KK_COUNT; ++i) {
        device->kernel_ms[i] = 0.0;
        device->kernel_launches[i] = 0;
    }
    return BNN_OK;
}

EXPORT BNN_Status BNNX_KernelTimingRead(BNN_Device device, uint32_t kind, double* total_ms, uint64_t* launches) {
    if (device == nullptr || kind >= (uint32_t)KK_COUNT)
        return BNN_EINVAL;
    if (total_ms)
        *total_ms = device->kernel_ms[kind];
    if (launches)
        *launches = device->kernel_launches[kind];
    return BNN_OK;
}

EXPORT BNN_Status BNNX_DeviceName(BNN_Device device, char* name, size_t name_bytes, char* arch, size_t arch_bytes) {
    if (device == nullptr)
        return BNN_EINVAL;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device->ordinal) != hipSuccess)
        return BNN_EIO;
    if (name && name_bytes) {
        strncpy(name, prop.name, name_bytes - 1);
        name[name_bytes - 1] = 0;
    }
    if (arch && arch_bytes) {
        strncpy(arch, prop.gcnArchName, arch_bytes - 1);
        arch[arch_bytes - 1] = 0;
    }
    return BNN_OK;
}
