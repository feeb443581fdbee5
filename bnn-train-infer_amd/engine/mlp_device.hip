// Device-resident bnn-mlp classification (mlp_device.h).  The reference engine runs a
// sample through the blocks as one synchronous GEMV_F32 per block, with the block's
// post_scale / post_bias / ReLU on the host in between (bnn-sw-v2/bnn-mlp/bnn-mlp.c:173-198);
// here a chunk's rows stay on the device from the first block to the last.
#include "mlp_device.h"

#include "bnn-accelerator-hip.h"

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <vector>

namespace bnne {
namespace {

// y = post_scale * y + post_bias for every output column o, then "negative -> 0" when the
// block has ReLU: mlp.cpp's host loop, product and sum rounded separately (no contraction).
__global__ __launch_bounds__(256) void k_mlp_post(float* __restrict__ y, uint32_t n, uint32_t width,
                                                  const float* __restrict__ scale, const float* __restrict__ bias,
                                                  int relu) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n)
        return;
    const uint32_t o = i % width;
    const float scaled = scale[o] * y[i];
    const float v = scaled + bias[o];
    y[i] = relu && v < 0.0f ? 0.0f : v;
}

BNNE_Status hip_failure(hipError_t e, const char* what) {
    (void)hipGetLastError();
    return complain(e == hipErrorOutOfMemory ? BNNE_ENOMEM : BNNE_EIO, "%s: %s", what, hipGetErrorString(e));
}

// Prepared batches kept per chunk size: a call pattern uses one or two (the full chunk
// and the last, shorter one).
constexpr size_t kMaxPlans = 4;

}  // namespace

struct MlpDevice {
    struct Block {
        const SignLinear* weight;
        uint32_t in, out;
        bool relu;
        const float* scale;  // device: post_scale, then post_bias at scale + out
    };
    struct Plan {
        uint32_t rows;
        std::vector<BNNX_Batch> batches;  // one chained batch, or one batch per block
        uint64_t jobs;                    // the GEMM_F32 jobs the host call pattern would run
        bool chain;
    };

    BNN_Device dev = nullptr;
    hipStream_t stream = nullptr;
    int ordinal = 0;
    uint32_t inputs = 0, classes = 0, rows = 0, widest = 0;
    std::vector<Block> blocks;
    float* params = nullptr;  // device: every block's post_scale and post_bias
    // accelerator buffers: the chunk's input rows, the hidden activations (blocks
    // alternate between the two) and the last block's outputs
    BNN_Buffer b_in = nullptr, b_act[2] = {nullptr, nullptr}, b_out = nullptr;
    float *in = nullptr, *act[2] = {nullptr, nullptr}, *out = nullptr;
    float *pinned_in = nullptr, *pinned_out = nullptr;  // host staging of the two copies
    std::vector<Plan> plans;                             // the most recently used last

    ~MlpDevice() {
        drop_plans();
        if (params)
            (void)hipFree(params);
        BNN_BufferFree(b_in);
        BNN_BufferFree(b_act[0]);
        BNN_BufferFree(b_act[1]);
        BNN_BufferFree(b_out);
        if (pinned_in)
            (void)hipHostFree(pinned_in);
        if (pinned_out)
            (void)hipHostFree(pinned_out);
    }
    void drop_plans() {
        for (Plan& p : plans)
            for (BNNX_Batch b : p.batches)
                BNNX_BatchDestroy(b);
        plans.clear();
    }
    // block i reads the chunk's rows (i = 0) or the previous block's outputs and writes
    // the next activation buffer (the logits for the last block)
    BNN_Buffer input_of(size_t i) const { return i == 0 ? b_in : b_act[(i - 1) % 2]; }
    BNN_Buffer output_of(size_t i) const { return i + 1 == blocks.size() ? b_out : b_act[i % 2]; }
    float* output_ptr(size_t i) const { return i + 1 == blocks.size() ? out : act[i % 2]; }

    BNNE_Status alloc(size_t floats, BNN_Buffer* b, float** ptr) {
        BNNE_Status st = accel_status(BNN_BufferAlloc(dev, floats * sizeof(float), b), "BNN_BufferAlloc");
        if (st == BNNE_OK)
            st = accel_status(BNNX_BufferDevicePointer(*b, reinterpret_cast<void**>(ptr)), "BNNX_BufferDevicePointer");
        return st;
    }

    // The batches of a chunk of n rows: one chained batch (every block and its mapping in
    // one launch) where the backend takes it, else per block GEMM_F32 jobs over consecutive
    // rows of at most the backend's max_rows each (as SignLinear::apply_rows splits them)
    // and this engine's post-operation kernel.
    BNNE_Status build_plan(uint32_t n, uint32_t max_rows, Plan* plan) {
        plan->rows = n;
        plan->jobs = 0;
        plan->chain = false;
        const uint32_t job_rows = max_rows ? (max_rows < n ? max_rows : n) : 1u;
        const uint64_t jobs_per_block = (n + job_rows - 1u) / job_rows;
        std::vector<BNNX_ChainLayer> layers;
        for (const Block& b : blocks)
            layers.push_back(BNNX_ChainLayer{b.weight->shards()[0].matrix, b.scale, b.scale + b.out, b.relu ? 1 : 0});
        BNNX_Batch chain = nullptr;
        const BNN_Status cs = BNNX_BatchCreateChain(dev, layers.data(), (uint32_t)layers.size(),
                                                    BNN_BufferView{b_in, BNN_TYPE_F32, 0, 0},
                                                    BNN_BufferView{b_out, BNN_TYPE_F32, 0, 0}, n, &chain);
        if (cs == BNN_OK) {
            plan->batches.push_back(chain);
            plan->jobs = jobs_per_block * blocks.size();
            plan->chain = true;
            return BNNE_OK;
        }
        if (cs != BNN_ENOTSUP)
            return accel_status(cs, "BNNX_BatchCreateChain");
        std::vector<BNN_Job> jobs;
        for (size_t i = 0; i < blocks.size(); ++i) {
            const Block& b = blocks[i];
            jobs.clear();
            for (uint32_t r0 = 0; r0 < n; r0 += job_rows) {
                BNN_Job j{};
                j.operation = BNN_OP_GEMM_F32;
                j.matrix = b.weight->shards()[0].matrix;
                j.input = BNN_BufferView{input_of(i), BNN_TYPE_F32, (size_t)r0 * b.in * sizeof(float), 0};
                j.output = BNN_BufferView{output_of(i), BNN_TYPE_F32, (size_t)r0 * b.out * sizeof(float), 0};
                j.rows = n - r0 < job_rows ? n - r0 : job_rows;
                jobs.push_back(j);
            }
            BNNX_Batch batch = nullptr;
            const BNNE_Status st =
                accel_status(BNNX_BatchCreate(dev, jobs.data(), (uint32_t)jobs.size(), &batch), "BNNX_BatchCreate");
            if (st != BNNE_OK)
                return st;
            plan->batches.push_back(batch);
            plan->jobs += jobs.size();
        }
        return BNNE_OK;
    }
};

BNNE_Status mlp_device_create(bnne_context* c, const MlpDeviceBlock* blocks, uint32_t count, uint32_t inputs,
                              uint32_t rows, MlpDevice** out) {
    *out = nullptr;
    if (count == 0 || rows == 0)
        return complain(BNNE_ENOTSUP, "device classify needs at least one block and one row");
    for (uint32_t i = 0; i < count; ++i)
        if (blocks[i].weight->shards().size() != 1)
            return complain(BNNE_ENOTSUP, "device classify takes blocks of one shard (block %u has %zu)", i,
                            blocks[i].weight->shards().size());
    MlpDevice* d = new (std::nothrow) MlpDevice;
    if (!d)
        return complain(BNNE_ENOMEM, "out of memory");
    d->dev = c->model->device;
    d->inputs = inputs;
    d->rows = rows;
    BNNE_Status st = accel_status(BNNX_DeviceStream(d->dev, reinterpret_cast<void**>(&d->stream)), "BNNX_DeviceStream");
    hipError_t e = hipSuccess;
    if (st == BNNE_OK) {
        e = hipStreamGetDevice(d->stream, &d->ordinal);
        if (e == hipSuccess)
            e = hipSetDevice(d->ordinal);
        if (e != hipSuccess)
            st = hip_failure(e, "device of the accelerator stream");
    }
    // post_scale and post_bias of every block, one upload
    size_t param_floats = 0;
    for (uint32_t i = 0; i < count; ++i)
        param_floats += 2 * (size_t)blocks[i].weight->out();
    std::vector<float> host(param_floats);
    size_t at = 0;
    for (uint32_t i = 0; i < count && st == BNNE_OK; ++i) {
        const MlpDeviceBlock& b = blocks[i];
        const uint32_t n_out = b.weight->out();
        std::memcpy(host.data() + at, b.post_scale, n_out * sizeof(float));
        std::memcpy(host.data() + at + n_out, b.post_bias, n_out * sizeof(float));
        d->blocks.push_back(MlpDevice::Block{b.weight, b.weight->in(), n_out, b.relu, nullptr});
        at += 2 * (size_t)n_out;
        if (i + 1 < count && n_out > d->widest)
            d->widest = n_out;
    }
    if (st == BNNE_OK) {
        d->classes = d->blocks.back().out;
        e = hipMalloc(reinterpret_cast<void**>(&d->params), param_floats * sizeof(float));
        if (e == hipSuccess)
            e = hipMemcpy(d->params, host.data(), param_floats * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess)
            st = hip_failure(e, "post-operation parameters");
        at = 0;
        for (MlpDevice::Block& b : d->blocks) {
            b.scale = d->params + at;
            at += 2 * (size_t)b.out;
        }
    }
    if (st == BNNE_OK)
        st = d->alloc((size_t)rows * inputs, &d->b_in, &d->in);
    for (int k = 0; k < 2 && st == BNNE_OK && d->widest > 0; ++k)
        st = d->alloc((size_t)rows * d->widest, &d->b_act[k], &d->act[k]);
    if (st == BNNE_OK)
        st = d->alloc((size_t)rows * d->classes, &d->b_out, &d->out);
    if (st == BNNE_OK) {
        e = hipHostMalloc(reinterpret_cast<void**>(&d->pinned_in), (size_t)rows * inputs * sizeof(float),
                          hipHostMallocDefault);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void**>(&d->pinned_out), (size_t)rows * d->classes * sizeof(float),
                              hipHostMallocDefault);
        if (e != hipSuccess)
            st = hip_failure(e, "pinned staging");
    }
    if (st != BNNE_OK) {
        delete d;
        return st;
    }
    *out = d;
    return BNNE_OK;
}

BNNE_Status mlp_device_classify(bnne_context* c, MlpDevice* d, const float* input, uint32_t rows, float* logits) {
    if (rows == 0 || rows > d->rows)
        return complain(BNNE_EINVAL, "%u rows at once; the device path stages %u", rows, d->rows);
    hipError_t e = hipSetDevice(d->ordinal);
    if (e != hipSuccess)
        return hip_failure(e, "hipSetDevice");
    // a plan for this chunk size; every plan is rebuilt once the backend reports the
    // batches stale (a matrix or buffer of the device destroyed since they were built)
    if (!d->plans.empty() && BNNX_BatchCheck(d->plans.back().batches[0]) == BNN_EINVAL)
        d->drop_plans();
    size_t found = d->plans.size();
    for (size_t i = 0; i < d->plans.size(); ++i)
        if (d->plans[i].rows == rows)
            found = i;
    if (found == d->plans.size()) {
        if (d->plans.size() == kMaxPlans) {
            for (BNNX_Batch b : d->plans.front().batches)
                BNNX_BatchDestroy(b);
            d->plans.erase(d->plans.begin());
        }
        MlpDevice::Plan plan;
        const BNNE_Status st = d->build_plan(rows, c->model->caps.max_rows, &plan);
        if (st != BNNE_OK) {
            for (BNNX_Batch b : plan.batches)
                BNNX_BatchDestroy(b);
            return st;
        }
        d->plans.push_back(std::move(plan));
    } else if (found + 1 != d->plans.size()) {
        MlpDevice::Plan plan = std::move(d->plans[found]);
        d->plans.erase(d->plans.begin() + (ptrdiff_t)found);
        d->plans.push_back(std::move(plan));
    }
    const MlpDevice::Plan& plan = d->plans.back();

    const bool stats = c->params.enable_stats != 0;
    const size_t in_bytes = (size_t)rows * d->inputs * sizeof(float);
    const size_t out_bytes = (size_t)rows * d->classes * sizeof(float);
    const uint64_t t0 = stats ? clock_ns() : 0;
    std::memcpy(d->pinned_in, input, in_bytes);
    e = hipMemcpyAsync(d->in, d->pinned_in, in_bytes, hipMemcpyHostToDevice, d->stream);
    BNNE_Status st = e == hipSuccess ? BNNE_OK : hip_failure(e, "input rows to the device");
    const uint64_t t_in = stats ? clock_ns() : 0;
    if (st == BNNE_OK && plan.chain)
        st = accel_status(BNNX_BatchLaunch(plan.batches[0]), "BNNX_BatchLaunch");
    for (size_t i = 0; i < d->blocks.size() && st == BNNE_OK && !plan.chain; ++i) {
        const MlpDevice::Block& b = d->blocks[i];
        st = accel_status(BNNX_BatchLaunch(plan.batches[i]), "BNNX_BatchLaunch");
        if (st != BNNE_OK)
            break;
        const uint32_t n = rows * b.out;
        hipLaunchKernelGGL(k_mlp_post, dim3((n + 255u) / 256u), dim3(256), 0, d->stream, d->output_ptr(i), n, b.out,
                           b.scale, b.scale + b.out, b.relu ? 1 : 0);
        e = hipGetLastError();
        if (e != hipSuccess)
            st = hip_failure(e, "post-operation launch");
    }
    if (st == BNNE_OK) {
        e = hipMemcpyAsync(d->pinned_out, d->out, out_bytes, hipMemcpyDeviceToHost, d->stream);
        if (e != hipSuccess)
            st = hip_failure(e, "logits to the host");
    }
    const uint64_t t1 = stats ? clock_ns() : 0;
    const BNN_Status sync = BNNX_DeviceSynchronize(d->dev);
    const uint64_t t2 = stats ? clock_ns() : 0;
    if (st != BNNE_OK)
        return st;
    // an illegal row (a non-finite value) is reported here as BNN_Execute reports it
    st = accel_status(sync, "BNN_Execute");
    if (st != BNNE_OK)
        return st;
    std::memcpy(logits, d->pinned_out, out_bytes);
    if (stats) {
        const uint64_t t3 = clock_ns();
        c->stats.transfer_ns += (t_in - t0) + (t3 - t2);  // the enqueues in between count as host time
        c->stats.execute_ns += t2 - t1;
        c->stats.device_calls += plan.jobs;
        c->stats.bytes_written += in_bytes;
        c->stats.bytes_read += out_bytes;
        uint64_t macs = 0;
        for (const MlpDevice::Block& b : d->blocks)
            macs += (uint64_t)rows * b.in * b.out;
        c->stats.logical_macs += macs;
        c->stats.executed_macs += macs;
    }
    return BNNE_OK;
}

void mlp_device_free(MlpDevice* d) { delete d; }

}  // namespace bnne
