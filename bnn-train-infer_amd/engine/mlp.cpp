// bnn-mlp classifiers (general.architecture "bnn-mlp"), the model of the reference's
// MNIST tooling (bnn-sw-v2/bnn-mlp/bnn-mlp.c:61-198 reads the same files).
//
// A stack of Q1_0 blocks: block i maps its input through blk.<i>.weight on the
// accelerator, then every output becomes post_scale * y + post_bias (the product and
// the sum rounded separately) and, when the block's activation is ReLU, max(., 0)
// written as "negative -> 0".  Metadata: bnn-mlp.block_count (1..64),
// bnn-mlp.input_features (a multiple of 128), bnn-mlp.class_count (the last block's
// width), bnn-mlp.input_std (> 0), bnn-mlp.input_pixels (at most input_features when
// present), bnn-mlp.block.<i>.activation ("relu" or "none"; absent: ReLU on every
// block but the last).
//
// A context classifies on one of two paths with the same logits: the device path
// (mlp_device.hip: a chunk's rows stay on the device through every block, one host wait
// per chunk; the default where the backend and the shapes allow it) or the reference's
// call pattern below (per block one write, GEMM_F32 jobs and one read, the post-operation
// on the host).
#include "engine.hpp"
#include "mlp_device.h"

#include <cstdio>
#include <string>

namespace bnne {
namespace {

constexpr uint64_t kMaxBlocks = 64;

struct MlpBlock {
    SignLinear weight;
    std::vector<float> post_scale, post_bias;
    bool relu = false;
};

class MlpModel final : public bnne_model {
public:
    void load() override;
    bnne_context* new_context(const BNNE_ContextParams& p) override;

    std::vector<std::unique_ptr<MlpBlock>> blocks;
    uint32_t inputs = 0, classes = 0;
    uint32_t widest = 0;  // the widest activation row (input or block output)
};

// Samples run through the blocks in chunks of up to kChunkRows: one GEMM_F32 job per
// block and chunk (each row of it is that sample's GEMV_F32), so a classify call of n
// samples makes ceil(n / kChunkRows) accelerator calls per block instead of n.
constexpr uint32_t kChunkRows = 256;

class MlpContext final : public bnne_context {
public:
    MlpContext(MlpModel& net, const BNNE_ContextParams& p) : bnne_context(net, p), net_(net) {
        stage_rows = p.n_batch < kChunkRows ? (p.n_batch ? p.n_batch : 1u) : kChunkRows;
        for (std::vector<float>& r : rows_)
            r.resize((size_t)stage_rows * net.widest);
        // the device path where the backend and the shapes allow it, else the host pattern
        const BNNE_Status st = open_device(&device_);
        if (st == BNNE_ENOTSUP)
            forget_message();
        else if (st != BNNE_OK)
            throw Failure{st};
    }
    ~MlpContext() override { mlp_device_free(device_); }
    void classify(const float* input, uint32_t n, float* logits) override;
    // 0 the host call pattern, 2 the device path (prepared batches; there is no fused form,
    // so asking for 1 selects it too).  The path may change between calls.
    int path() const override { return device_ ? 2 : 0; }
    void select_path(int path) override;

private:
    BNNE_Status open_device(MlpDevice** out);

    MlpModel& net_;
    std::vector<float> rows_[2];  // the hidden activations of a chunk alternate between these
    MlpDevice* device_ = nullptr;
};

std::string block_key(uint32_t i, const char* what) {
    char name[64];
    std::snprintf(name, sizeof name, "blk.%u.%s", i, what);
    return name;
}

void MlpModel::load() {
    const GgufFile& f = *file;
    const uint64_t n_blocks = f.integer("bnn-mlp.block_count").value_or(0);
    const uint64_t n_inputs = f.integer("bnn-mlp.input_features").value_or(0);
    const uint64_t n_classes = f.integer("bnn-mlp.class_count").value_or(0);
    const uint64_t pixels = f.integer("bnn-mlp.input_pixels").value_or(0);
    const float spread = f.real("bnn-mlp.input_std").value_or(0.0f);
    if (n_blocks == 0 || n_blocks > kMaxBlocks || n_inputs == 0 || n_inputs > UINT32_MAX || n_inputs % kGroup != 0 ||
        n_classes == 0 || n_classes > UINT32_MAX || pixels > n_inputs || !(spread > 0.0f))
        raise(BNNE_EFORMAT, "bnn-mlp metadata out of range (blocks %llu, inputs %llu, classes %llu)",
              (unsigned long long)n_blocks, (unsigned long long)n_inputs, (unsigned long long)n_classes);
    inputs = (uint32_t)n_inputs;
    classes = (uint32_t)n_classes;
    widest = inputs;

    uint32_t width = inputs;  // the current block's input width
    for (uint32_t i = 0; i < (uint32_t)n_blocks; ++i) {
        std::unique_ptr<MlpBlock> b(new MlpBlock);
        const SignWeights w = read_sign_weights(f, block_key(i, "weight"));
        if (w.in != width)
            raise(BNNE_EFORMAT, "bnn-mlp block %u reads %u values but receives %u", i, w.in, width);
        b->weight.upload(*this, w);
        b->post_scale = read_floats(f, block_key(i, "post_scale"), w.out);
        b->post_bias = read_floats(f, block_key(i, "post_bias"), w.out);
        char key[64];
        std::snprintf(key, sizeof key, "bnn-mlp.block.%u.activation", i);
        const std::optional<std::string_view> act = f.text(key);
        if (!act)
            b->relu = i + 1 < (uint32_t)n_blocks;
        else if (*act == "relu" || *act == "none")
            b->relu = *act == "relu";
        else
            raise(BNNE_EFORMAT, "bnn-mlp block %u has activation '%.*s' (relu or none)", i, (int)act->size(),
                  act->data());
        width = w.out;
        if (width > widest)
            widest = width;
        blocks.push_back(std::move(b));
    }
    if (width != classes)
        raise(BNNE_EFORMAT, "the last bnn-mlp block gives %u values for %u classes", width, classes);
    info.input_rank = 1;
    info.input_dims[0] = inputs;
    info.input_size = inputs;
    info.n_classes = classes;
}

bnne_context* MlpModel::new_context(const BNNE_ContextParams& p) { return new MlpContext(*this, p); }

BNNE_Status MlpContext::open_device(MlpDevice** out) {
    std::vector<MlpDeviceBlock> blocks;
    for (const auto& b : net_.blocks)
        blocks.push_back(MlpDeviceBlock{&b->weight, b->post_scale.data(), b->post_bias.data(), b->relu});
    return mlp_device_create(this, blocks.data(), (uint32_t)blocks.size(), net_.inputs, stage_rows, out);
}

void MlpContext::select_path(int path) {
    if (path < 0 || path > 2)
        raise(BNNE_EINVAL, "classify path %d (0 host, 1 or 2 device)", path);
    if ((path == 0) == (device_ == nullptr))
        return;
    if (path == 0) {
        mlp_device_free(device_);
        device_ = nullptr;
        return;
    }
    const BNNE_Status st = open_device(&device_);
    if (st != BNNE_OK)
        throw Failure{st};
}

void MlpContext::classify(const float* input, uint32_t n, float* logits) {
    if (device_) {
        for (uint32_t s0 = 0; s0 < n; s0 += stage_rows) {
            const uint32_t rows = n - s0 < stage_rows ? n - s0 : stage_rows;
            const BNNE_Status st = mlp_device_classify(this, device_, input + (size_t)s0 * net_.inputs, rows,
                                                       logits + (size_t)s0 * net_.classes);
            if (st != BNNE_OK)
                throw Failure{st};
        }
        return;
    }
    const size_t count = net_.blocks.size();
    for (uint32_t s0 = 0; s0 < n; s0 += stage_rows) {
        const uint32_t rows = n - s0 < stage_rows ? n - s0 : stage_rows;
        const float* x = input + (size_t)s0 * net_.inputs;
        for (size_t i = 0; i < count; ++i) {
            const MlpBlock& b = *net_.blocks[i];
            const uint32_t out = b.weight.out();
            float* y = i + 1 == count ? logits + (size_t)s0 * net_.classes : rows_[i % 2].data();
            b.weight.apply_rows(*this, x, rows, y);
            for (uint32_t r = 0; r < rows; ++r) {
                float* yr = y + (size_t)r * out;
                for (uint32_t o = 0; o < out; ++o) {
                    const float scaled = b.post_scale[o] * yr[o];
                    const float v = scaled + b.post_bias[o];
                    yr[o] = b.relu && v < 0.0f ? 0.0f : v;
                }
            }
            x = y;
        }
    }
}

}  // namespace

bnne_model* make_bnn_mlp() { return new MlpModel; }

}  // namespace bnne
