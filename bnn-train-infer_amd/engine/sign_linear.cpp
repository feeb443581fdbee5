// Q1_0 tensors and the linear layers built from them.
//
// Q1_0 on disk (bnn-sw-v2/linear.c:26-62, gguf.c:358-379): a tensor [in, out] is out
// rows of in / 128 blocks; a block is 18 bytes, the little-endian fp16 scale and then
// the 128 sign bits of the group, bit j % 8 of byte j / 8 for weight j (1 = +1).
// Blocks are stored row-major, which is also the order of the accelerator's
// scales[out][in / 128] and of the 16-byte groups of its bits[out][in / 8]: splitting
// is one pass over the blocks.
//
// A layer wider than the device's max_out_features is split into shards of at most
// that many outputs (linear.c:104-125), each its own BNN_Matrix.  apply() is the call
// sequence of the reference engine's linear layer (linear.c:161-216) with the same
// statistics: the input row written once, then per shard one BNN_Execute of
// GEMV_F32 at rows = 1 and one read of its outputs.  apply_rows() is the same sequence
// for a block of rows, with GEMM_F32 over all of them in place of one GEMV_F32 per row.
#include "engine.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace bnne {

SignWeights read_sign_weights(const GgufFile& file, std::string_view name) {
    const TensorRef* t = file.tensor(name);
    if (!t || t->type != kQ1_0 || t->rank != 2)
        raise(BNNE_EFORMAT, "no Q1_0 [in, out] tensor '%.*s'", (int)name.size(), name.data());
    if (t->dims[0] > UINT32_MAX || t->dims[1] > UINT32_MAX)
        raise(BNNE_EFORMAT, "tensor '%.*s' is too wide", (int)name.size(), name.data());
    SignWeights w;
    w.in = (uint32_t)t->dims[0];
    w.out = (uint32_t)t->dims[1];
    const size_t blocks = (size_t)w.out * (w.in / kGroup);
    w.bits.resize(blocks * 16);
    w.scales.resize(blocks);
    const uint8_t* block = t->data;
    for (size_t b = 0; b < blocks; ++b, block += 18) {
        const uint16_t scale = (uint16_t)(block[0] | block[1] << 8);
        if (!half_is_finite(scale))
            raise(BNNE_EFORMAT, "tensor '%.*s' has a NaN or infinite scale", (int)name.size(), name.data());
        w.scales[b] = scale;
        std::memcpy(&w.bits[b * 16], block + 2, 16);
    }
    return w;
}

SignWeights read_sign_weights(const GgufFile& file, std::string_view name, uint32_t in, uint32_t out) {
    SignWeights w = read_sign_weights(file, name);
    if (w.in != in || w.out != out)
        raise(BNNE_EFORMAT, "tensor '%.*s' maps %u -> %u values where %u -> %u belong", (int)name.size(), name.data(),
              w.in, w.out, in, out);
    return w;
}

SignLinear::~SignLinear() {
    for (const Shard& s : shards_)
        BNN_MatrixDestroy(s.matrix);
}

void SignLinear::upload(bnne_model& model, const SignWeights& w) {
    const BNN_Caps& caps = model.caps;
    if (caps.group_size != kGroup || !(caps.supported_ops & BNN_CAP_GEMV_F32))
        raise(BNNE_ENOTSUP, "Q1_0 layers need an accelerator with 128-weight groups and GEMV_F32");
    if (caps.max_in_features == 0 || caps.max_out_features == 0)
        raise(BNNE_ENOTSUP, "the accelerator reports no matrix size limits");
    if (w.in > caps.max_in_features)
        raise(BNNE_ENOTSUP, "a layer reads %u values; the accelerator takes at most %u", w.in, caps.max_in_features);
    in_ = w.in;
    out_ = w.out;
    const size_t row_bits = w.in / 8u, row_scales = w.in / kGroup;
    for (uint32_t first = 0; first < w.out; first += caps.max_out_features) {
        const uint32_t count = w.out - first < caps.max_out_features ? w.out - first : caps.max_out_features;
        BNN_MatrixDesc desc{};
        desc.in_features = w.in;
        desc.out_features = count;
        desc.group_size = kGroup;
        desc.weight_bits = w.bits.data() + first * row_bits;
        desc.weight_bytes = count * row_bits;
        desc.scale_fp16 = w.scales.data() + first * row_scales;
        desc.scale_count = count * row_scales;
        BNN_Matrix m = nullptr;
        require(BNN_MatrixCreate(model.device, &desc, &m), "BNN_MatrixCreate");
        shards_.push_back(Shard{first, count, m});
        if (count > model.widest_shard)
            model.widest_shard = count;
    }
    if (w.in > model.widest_in)
        model.widest_in = w.in;
}

void SignLinear::apply(bnne_context& ctx, const float* x, float* y) const {
    const size_t in_bytes = (size_t)in_ * sizeof(float);
    {
        Span busy(ctx.counter(&BNNE_Stats::transfer_ns));
        const BNN_Status st = BNN_BufferWrite(ctx.stage_in, 0, x, in_bytes);
        ctx.count(&BNNE_Stats::bytes_written, in_bytes);
        require(st, "BNN_BufferWrite");
    }
    for (const Shard& s : shards_) {
        BNN_Job job{};
        job.operation = BNN_OP_GEMV_F32;
        job.matrix = s.matrix;
        job.input = BNN_BufferView{ctx.stage_in, BNN_TYPE_F32, 0, 0};
        job.output = BNN_BufferView{ctx.stage_out, BNN_TYPE_F32, 0, 0};
        job.rows = 1;
        {
            Span busy(ctx.counter(&BNNE_Stats::execute_ns));
            require(BNN_Execute(ctx.model->device, &job), "BNN_Execute");
        }
        const size_t out_bytes = (size_t)s.count * sizeof(float);
        Span busy(ctx.counter(&BNNE_Stats::transfer_ns));
        const BNN_Status st = BNN_BufferRead(ctx.stage_out, 0, y + s.first, out_bytes);
        ctx.count(&BNNE_Stats::device_calls, 1);
        ctx.count(&BNNE_Stats::bytes_read, out_bytes);
        require(st, "BNN_BufferRead");
    }
    const uint64_t macs = (uint64_t)in_ * out_;
    ctx.count(&BNNE_Stats::logical_macs, macs);
    ctx.count(&BNNE_Stats::executed_macs, macs);
}

void SignLinear::apply_rows(bnne_context& ctx, const float* x, uint32_t rows, float* y) const {
    if (rows > ctx.stage_rows)
        raise(BNNE_EINVAL, "%u rows at once; the context stages %u", rows, ctx.stage_rows);
    if (rows <= 1 || !(ctx.model->caps.supported_ops & BNN_CAP_GEMM_F32)) {
        for (uint32_t r = 0; r < rows; ++r)
            apply(ctx, x + (size_t)r * in_, y + (size_t)r * out_);
        return;
    }
    const size_t in_bytes = (size_t)rows * in_ * sizeof(float);
    {
        Span busy(ctx.counter(&BNNE_Stats::transfer_ns));
        const BNN_Status st = BNN_BufferWrite(ctx.stage_in, 0, x, in_bytes);
        ctx.count(&BNNE_Stats::bytes_written, in_bytes);
        require(st, "BNN_BufferWrite");
    }
    // a layer of one shard reads its rows straight into y; a sharded one reads each
    // shard's block of rows and places it at the shard's columns.  A job holds at most
    // the backend's max_rows rows (the remote backend's limit is 128): larger blocks run
    // as several jobs over consecutive rows of the staged input and output.
    const uint32_t job_rows = std::max(1u, std::min(rows, ctx.model->caps.max_rows));
    std::vector<float> block(shards_.size() > 1 ? (size_t)rows * shards_.front().count : 0);
    for (const Shard& s : shards_) {
        for (uint32_t r0 = 0; r0 < rows; r0 += job_rows) {
            BNN_Job job{};
            job.operation = BNN_OP_GEMM_F32;
            job.matrix = s.matrix;
            job.input = BNN_BufferView{ctx.stage_in, BNN_TYPE_F32, (size_t)r0 * in_ * sizeof(float), 0};
            job.output = BNN_BufferView{ctx.stage_out, BNN_TYPE_F32, (size_t)r0 * s.count * sizeof(float), 0};
            job.rows = std::min(job_rows, rows - r0);
            Span busy(ctx.counter(&BNNE_Stats::execute_ns));
            require(BNN_Execute(ctx.model->device, &job), "BNN_Execute");
            ctx.count(&BNNE_Stats::device_calls, 1);
        }
        const size_t out_bytes = (size_t)rows * s.count * sizeof(float);
        float* dst = shards_.size() > 1 ? block.data() : y;
        {
            Span busy(ctx.counter(&BNNE_Stats::transfer_ns));
            const BNN_Status st = BNN_BufferRead(ctx.stage_out, 0, dst, out_bytes);
            ctx.count(&BNNE_Stats::bytes_read, out_bytes);
            require(st, "BNN_BufferRead");
        }
        if (shards_.size() > 1)
            for (uint32_t r = 0; r < rows; ++r)
                std::memcpy(y + (size_t)r * out_ + s.first, block.data() + (size_t)r * s.count,
                            s.count * sizeof(float));
    }
    const uint64_t macs = (uint64_t)rows * in_ * out_;
    ctx.count(&BNNE_Stats::logical_macs, macs);
    ctx.count(&BNNE_Stats::executed_macs, macs);
}

}  // namespace bnne
