// bnn-mlp classifier (architecture "bnn-mlp"): a stack of Q1_0 linear blocks, each
// followed by an F32 affine y = post_scale * y + post_bias (two roundings, no FMA)
// and an optional ReLU (bnn-sw-v2/bnn-mlp/bnn-mlp.c:61-198).
//
// Metadata: bnn-mlp.block_count (1..64), input_features (multiple of 128),
// class_count, input_std > 0, input_pixels <= input_features; per block
// blk.<i>.weight (Q1_0), blk.<i>.post_scale / post_bias (F32 or F16, out_features
// long) and bnn-mlp.block.<i>.activation ("relu", "none", or absent = ReLU on all
// but the last block).
#include "engine_internal.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace bnne {
namespace {

constexpr uint32_t kMaxLayers = 64;

struct Layer {
    Linear weight;
    float *post_scale, *post_bias;
    uint32_t in, out;
    bool relu;
};

struct Model {
    uint32_t layer_count, input_features, class_count, max_dim;
    Layer* layers;
};

struct State {
    float* work[2];
};

void unload(void* impl) {
    Model* m = static_cast<Model*>(impl);
    if (!m)
        return;
    if (m->layers)
        for (uint32_t i = 0; i < m->layer_count; ++i) {
            linear_free(&m->layers[i].weight);
            std::free(m->layers[i].post_scale);
            std::free(m->layers[i].post_bias);
        }
    std::free(m->layers);
    std::free(m);
}

BNNE_Status read_vector(const Gguf* g, const char* name, uint32_t count, float** out) {
    float* data = nullptr;
    size_t n = 0;
    const BNNE_Status st = tensor_f32(g, name, &data, &n);
    if (st != BNNE_OK)
        return st;
    if (n != count) {
        std::free(data);
        return error(BNNE_EFORMAT, "tensor '%s' has %zu elements, expected %u", name, n, count);
    }
    *out = data;
    return BNNE_OK;
}

BNNE_Status load(bnne_model* mm, const Gguf* g, void** out_impl) {
    *out_impl = nullptr;
    if (g->mlp_block_count == 0 || g->mlp_block_count > kMaxLayers || g->mlp_input_features == 0 ||
        g->mlp_input_features > UINT32_MAX || g->mlp_input_features % 128 != 0 || g->mlp_class_count == 0 ||
        g->mlp_class_count > UINT32_MAX || (g->mlp_input_pixels && g->mlp_input_pixels > g->mlp_input_features) ||
        !(g->mlp_input_std > 0.0f))
        return error(BNNE_EFORMAT, "unsupported bnn-mlp metadata");
    Model* m = static_cast<Model*>(std::calloc(1, sizeof(Model)));
    if (!m)
        return error(BNNE_ENOMEM, "out of memory");
    m->layer_count = (uint32_t)g->mlp_block_count;
    m->input_features = (uint32_t)g->mlp_input_features;
    m->class_count = (uint32_t)g->mlp_class_count;
    m->max_dim = m->input_features;
    m->layers = static_cast<Layer*>(std::calloc(m->layer_count, sizeof(Layer)));
    if (!m->layers) {
        unload(m);
        return error(BNNE_ENOMEM, "out of memory");
    }
    uint32_t expected_in = m->input_features;
    BNNE_Status st = BNNE_OK;
    char name[64];
    for (uint32_t i = 0; i < m->layer_count && st == BNNE_OK; ++i) {
        Layer& L = m->layers[i];
        std::snprintf(name, sizeof name, "blk.%u.weight", i);
        st = linear_load(mm, g, name, &L.weight);
        if (st != BNNE_OK)
            break;
        if (L.weight.in != expected_in) {
            st = error(BNNE_EFORMAT, "layer %u input width %u does not match previous output %u", i, L.weight.in,
                       expected_in);
            break;
        }
        L.in = L.weight.in;
        L.out = L.weight.out;
        std::snprintf(name, sizeof name, "blk.%u.post_scale", i);
        st = read_vector(g, name, L.out, &L.post_scale);
        if (st != BNNE_OK)
            break;
        std::snprintf(name, sizeof name, "blk.%u.post_bias", i);
        st = read_vector(g, name, L.out, &L.post_bias);
        if (st != BNNE_OK)
            break;
        const char* act = i < g->mlp_activation_count ? g->mlp_activations[i] : "";
        if (!act[0])
            L.relu = i + 1 < m->layer_count;
        else if (std::strcmp(act, "relu") == 0)
            L.relu = true;
        else if (std::strcmp(act, "none") == 0)
            L.relu = false;
        else
            st = error(BNNE_EFORMAT, "invalid activation for bnn-mlp block %u", i);
        if (L.out > m->max_dim)
            m->max_dim = L.out;
        expected_in = L.out;
    }
    if (st == BNNE_OK && expected_in != m->class_count)
        st = error(BNNE_EFORMAT, "last bnn-mlp layer width %u does not match class_count %u", expected_in,
                   m->class_count);
    if (st != BNNE_OK) {
        unload(m);
        return st;
    }
    mm->info.input_rank = 1;
    mm->info.input_dims[0] = m->input_features;
    mm->info.input_size = m->input_features;
    mm->info.n_classes = m->class_count;
    *out_impl = m;
    return BNNE_OK;
}

void ctx_free(void* state) {
    State* s = static_cast<State*>(state);
    if (!s)
        return;
    std::free(s->work[0]);
    std::free(s->work[1]);
    std::free(s);
}

BNNE_Status ctx_init(bnne_context* c, void** out_state) {
    const Model* m = static_cast<const Model*>(c->model->impl);
    State* s = static_cast<State*>(std::calloc(1, sizeof(State)));
    if (!s)
        return error(BNNE_ENOMEM, "out of memory");
    s->work[0] = static_cast<float*>(std::malloc((size_t)m->max_dim * sizeof(float)));
    s->work[1] = static_cast<float*>(std::malloc((size_t)m->max_dim * sizeof(float)));
    if (!s->work[0] || !s->work[1]) {
        ctx_free(s);
        return error(BNNE_ENOMEM, "out of memory");
    }
    *out_state = s;
    return BNNE_OK;
}

BNNE_Status classify(bnne_context* c, const float* input, uint32_t n, float* logits) {
    const Model* m = static_cast<const Model*>(c->model->impl);
    State* s = static_cast<State*>(c->state);
    for (uint32_t sample = 0; sample < n; ++sample) {
        const float* x = input + (size_t)sample * m->input_features;
        for (uint32_t i = 0; i < m->layer_count; ++i) {
            const Layer& L = m->layers[i];
            float* y = i + 1 == m->layer_count ? logits + (size_t)sample * m->class_count : s->work[i & 1];
            const BNNE_Status st = linear_forward(c, &L.weight, x, y);
            if (st != BNNE_OK)
                return st;
            for (uint32_t o = 0; o < L.out; ++o) {
                float v = L.post_scale[o] * y[o] + L.post_bias[o];
                if (L.relu && v < 0.0f)
                    v = 0.0f;
                y[o] = v;
            }
            x = y;
        }
    }
    return BNNE_OK;
}

}  // namespace

const Arch kArchBnnMlp = {"bnn-mlp", BNNE_TASK_CLASSIFY, load, unload, ctx_init, ctx_free, classify, nullptr, nullptr};

}  // namespace bnne
