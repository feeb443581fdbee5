// Qwen3 decoders (general.architecture "qwen3"), the model of the reference's LLM path.
//
// Weights: token_embd.weight is Q1_0 [C, V]: a token's row is its embedding (+scale
// where the sign bit is 1, -scale where it is 0) and the same matrix is the output
// layer (tied embeddings); per layer blk.<l>.attn_norm, ffn_norm (C values),
// attn_q_norm, attn_k_norm (head_dim values) as F32/F16 and the Q1_0 projections
// attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down; output_norm.
//
// A context decodes on one of two paths with the same results: the device path
// (resident.hip: everything on the GPU, the linear layers as fused batches) or the
// host step below, which runs every linear layer through SignLinear::apply (one
// BNN_Execute per shard) and the rest on the host.  The host step performs the
// floating-point operations of the reference's qwen3_step
// (bnn-sw-v2/qwen3/qwen3.c:342-512) in the same order -- sequential sums, RMSNorm as
// x / rms * gain, softmax as exp(s - max) / sum, SiLU as g / (1 + exp(-g)) * u --
// compiled without contraction and with the same libm, so equal linear results
// give equal logits.
#include "engine.hpp"
#include "resident.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <math.h>
#include <string>

#include "host_expf.h"

namespace bnne {
namespace {

constexpr uint64_t kMaxLayers = 128, kMaxHeads = 256, kMaxVocab = 1u << 20;
constexpr double kPi = 3.14159265358979323846;

struct Shape {
    uint32_t layers = 0, width = 0, ffn = 0, heads = 0, kv_heads = 0, head_dim = 0, vocab = 0, kv_width = 0;
    uint32_t trained_ctx = 0;
    float eps = 0, rope_base = 0;
    // RoPE scaling: frequencies times freq_scale; YaRN ramps between scaled and
    // unscaled frequencies over the pairs [ramp_lo, ramp_hi] and multiplies by mscale
    float freq_scale = 1.0f, mscale = 1.0f;
    int32_t ramp_lo = 0, ramp_hi = 0;
    bool yarn = false;
};

struct Layer {
    std::vector<float> attn_norm, ffn_norm, q_norm, k_norm;
    SignLinear q, k, v, o, gate, up, down;
};

class Qwen3Model final : public bnne_model {
public:
    void load() override;
    bnne_context* new_context(const BNNE_ContextParams& p) override;

    Shape shape;
    SignWeights embedding;  // token rows (and the output layer's weights)
    SignLinear lm_head;
    std::vector<float> final_norm;
    std::vector<std::unique_ptr<Layer>> layers;

private:
    void read_shape();
};

uint32_t bounded(const GgufFile& f, const char* key, uint64_t max) {
    const uint64_t v = f.integer(key).value_or(0);
    if (v == 0 || v > max)
        raise(BNNE_EFORMAT, "Qwen3 metadata %s = %llu is outside 1..%llu", key, (unsigned long long)v,
              (unsigned long long)max);
    return (uint32_t)v;
}

int32_t clamp_pair(double v, int32_t lo, int32_t hi) { return v <= (double)lo ? lo : v >= (double)hi ? hi : (int32_t)v; }

void Qwen3Model::read_shape() {
    const GgufFile& f = *file;
    Shape& s = shape;
    const TensorRef* emb = f.tensor("token_embd.weight");
    if (!emb || emb->type != kQ1_0 || emb->rank != 2)
        raise(BNNE_EFORMAT, "no Q1_0 token_embd.weight");
    s.layers = bounded(f, "qwen3.block_count", kMaxLayers);
    s.width = bounded(f, "qwen3.embedding_length", UINT32_MAX);
    s.ffn = bounded(f, "qwen3.feed_forward_length", UINT32_MAX);
    s.heads = bounded(f, "qwen3.attention.head_count", kMaxHeads);
    s.kv_heads = bounded(f, "qwen3.attention.head_count_kv", kMaxHeads);
    s.head_dim = bounded(f, "qwen3.attention.key_length", UINT32_MAX);
    if (f.integer("qwen3.attention.value_length").value_or(0) != s.head_dim)
        raise(BNNE_EFORMAT, "Qwen3 value heads differ from key heads");
    s.trained_ctx = bounded(f, "qwen3.context_length", UINT32_MAX);
    s.eps = f.real("qwen3.attention.layer_norm_rms_epsilon").value_or(0.0f);
    s.rope_base = f.real("qwen3.rope.freq_base").value_or(0.0f);
    if (!(s.eps > 0.0f) || !(s.rope_base > 0.0f))
        raise(BNNE_EFORMAT, "Qwen3 RMSNorm epsilon and RoPE base must be positive");
    if (emb->dims[0] != s.width || emb->dims[1] == 0 || emb->dims[1] > kMaxVocab)
        raise(BNNE_EFORMAT, "token_embd.weight is not [%u, vocabulary <= 2^20]", s.width);
    s.vocab = (uint32_t)emb->dims[1];
    if (s.head_dim > s.width || (uint64_t)s.heads * s.head_dim != s.width || s.heads % s.kv_heads != 0 ||
        s.width % kGroup != 0 || s.ffn % kGroup != 0 || s.head_dim % 2 != 0)
        raise(BNNE_EFORMAT, "Qwen3 widths do not fit together (heads x head_dim = width, groups of 128)");
    s.kv_width = s.kv_heads * s.head_dim;
    if (s.kv_width % kGroup != 0)
        raise(BNNE_EFORMAT, "Qwen3 key/value width %u is not a multiple of 128", s.kv_width);
    if (caps.group_size != kGroup || !(caps.supported_ops & BNN_CAP_GEMV_F32))
        raise(BNNE_ENOTSUP, "Qwen3 layers need an accelerator with 128-weight groups and GEMV_F32");

    // RoPE scaling (YaRN when qwen3.rope.scaling.type is "yarn")
    // a factor <= 0 (or none) means 1; a NaN factor stays NaN and is rejected below (gguf.c:483-484)
    const float factor = f.real("qwen3.rope.scaling.factor").value_or(0.0f);
    s.freq_scale = 1.0f / (factor <= 0.0f ? 1.0f : factor);
    s.yarn = f.text("qwen3.rope.scaling.type").value_or("") == "yarn";
    s.ramp_lo = 0;
    s.ramp_hi = (int32_t)s.head_dim - 1;
    uint64_t original = f.integer("qwen3.rope.scaling.original_context_length").value_or(0);
    if (original == 0)
        original = s.trained_ctx;
    if (s.yarn && original) {
        // the pairs whose wavelength spans 32 and 1 rotations of the original context
        const double dims = (double)s.head_dim, log_base2 = 2.0 * std::log((double)s.rope_base);
        const double lo = std::floor(dims * std::log((double)original / (32.0 * 2.0 * kPi)) / log_base2);
        const double hi = std::ceil(dims * std::log((double)original / (2.0 * kPi)) / log_base2);
        s.ramp_lo = clamp_pair(lo, 0, (int32_t)s.head_dim - 1);
        s.ramp_hi = clamp_pair(hi, 0, (int32_t)s.head_dim - 1);
        s.mscale = 1.0f + 0.1f * logf(1.0f / s.freq_scale);
    }
    if (!(s.freq_scale > 0.0f) || !std::isfinite(s.mscale))
        raise(BNNE_EFORMAT, "Qwen3 RoPE scaling gives no usable frequencies");
}

std::string layer_key(uint32_t l, const char* what) {
    char name[80];
    std::snprintf(name, sizeof name, "blk.%u.%s.weight", l, what);
    return name;
}

void Qwen3Model::load() {
    read_shape();
    const Shape& s = shape;
    const GgufFile& f = *file;
    final_norm = read_floats(f, "output_norm.weight", s.width);
    for (uint32_t l = 0; l < s.layers; ++l) {
        std::unique_ptr<Layer> layer(new Layer);
        layer->attn_norm = read_floats(f, layer_key(l, "attn_norm"), s.width);
        layer->ffn_norm = read_floats(f, layer_key(l, "ffn_norm"), s.width);
        layer->q_norm = read_floats(f, layer_key(l, "attn_q_norm"), s.head_dim);
        layer->k_norm = read_floats(f, layer_key(l, "attn_k_norm"), s.head_dim);
        layers.push_back(std::move(layer));
    }
    embedding = read_sign_weights(f, "token_embd.weight", s.width, s.vocab);
    lm_head.upload(*this, embedding);
    for (uint32_t l = 0; l < s.layers; ++l) {
        Layer& L = *layers[l];
        const struct {
            const char* name;
            uint32_t in, out;
            SignLinear* dst;
        } projections[] = {
            {"attn_q", s.width, s.width, &L.q},     {"attn_k", s.width, s.kv_width, &L.k},
            {"attn_v", s.width, s.kv_width, &L.v},  {"attn_output", s.width, s.width, &L.o},
            {"ffn_gate", s.width, s.ffn, &L.gate},  {"ffn_up", s.width, s.ffn, &L.up},
            {"ffn_down", s.ffn, s.width, &L.down},
        };
        for (const auto& p : projections)
            p.dst->upload(*this, read_sign_weights(f, layer_key(l, p.name), p.in, p.out));
    }
    info.n_vocab = s.vocab;
    info.n_ctx_train = s.trained_ctx;
}

// ---------------------------------------------------------------------------- context

class Qwen3Context final : public bnne_context {
public:
    Qwen3Context(Qwen3Model& m, const BNNE_ContextParams& p);
    ~Qwen3Context() override { resident_free(device_); }
    void decode(const int32_t* tokens, uint32_t n, float* logits) override;
    void decode_greedy(int32_t token, uint32_t n, int32_t* out) override;

    // 0 host step, 1 device path with fused batches, 2 device path with prepared batches
    int path() const override { return device_ ? (resident_fused(device_) ? 1 : 2) : 0; }
    void select_path(int path) override;

private:
    BNNE_Status open_device_path(bool fused, Resident** out);
    void step(uint32_t token, uint32_t pos, float* logits);
    void attend(uint32_t layer, uint32_t pos);
    void host_cache();

    Qwen3Model& m_;
    const Shape& s_;
    // host step: the activation rows, attention scratch and the KV cache
    std::vector<float> x_, norm_, q_, k_, v_, y_, o_, gate_, up_, ex_, scores_, probs_;
    // host step only, per layer and key/value head: keys [n_ctx / 8][head_dim][8] (blocks
    // of eight positions), values [n_ctx][head_dim]
    std::vector<float> keys_, values_;
    uint32_t ctx_blocks_ = 0;  // ceil(n_ctx / 8)
    std::vector<float> cos_, sin_;      // RoPE rotation of pair j at position p: [p][head_dim / 2]
    Resident* device_ = nullptr;
};

Qwen3Context::Qwen3Context(Qwen3Model& m, const BNNE_ContextParams& p)
    : bnne_context(m, p), m_(m), s_(m.shape), x_(s_.width), norm_(s_.width), q_(s_.width), k_(s_.kv_width),
      v_(s_.kv_width), y_(s_.width), o_(s_.width), gate_(s_.ffn), up_(s_.ffn), ex_(s_.ffn), scores_(p.n_ctx), probs_(p.n_ctx) {
    // rotation tables (qwen3.c:276-299): theta = pos * base^(-2j / head_dim), scaled
    const uint32_t half = s_.head_dim / 2;
    cos_.resize((size_t)p.n_ctx * half);
    sin_.resize((size_t)p.n_ctx * half);
    const float span = (float)(s_.ramp_hi - s_.ramp_lo);
    const float ramp_width = span > 0.001f ? span : 0.001f;
    for (uint32_t pos = 0; pos < p.n_ctx; ++pos)
        for (uint32_t j = 0; j < half; ++j) {
            const float unscaled = (float)pos * powf(s_.rope_base, -2.0f * (float)j / (float)s_.head_dim);
            float theta = s_.freq_scale * unscaled;
            if (s_.yarn) {
                const float t = ((float)j - (float)s_.ramp_lo) / ramp_width;
                const float keep = 1.0f - fminf(1.0f, fmaxf(0.0f, t));  // share of the unscaled frequency
                theta = (s_.freq_scale * unscaled) * (1.0f - keep) + unscaled * keep;
            }
            cos_[(size_t)pos * half + j] = cosf(theta) * s_.mscale;
            sin_[(size_t)pos * half + j] = sinf(theta) * s_.mscale;
        }
    // the device path where the backend and the shapes allow it, else the host step
    const BNNE_Status st = open_device_path(true, &device_);
    if (st == BNNE_ENOTSUP) {
        forget_message();
        host_cache();
    } else if (st != BNNE_OK) {
        throw Failure{st};
    }
}

void Qwen3Context::host_cache() {
    ctx_blocks_ = (params.n_ctx + 7u) / 8u;
    keys_.assign((size_t)s_.layers * s_.kv_width * ctx_blocks_ * 8u, 0.0f);
    values_.assign((size_t)s_.layers * s_.kv_width * params.n_ctx, 0.0f);
    scores_.assign((size_t)ctx_blocks_ * 8u, 0.0f);  // the key blocks' lanes past the position too
}

BNNE_Status Qwen3Context::open_device_path(bool fused, Resident** out) {
    std::vector<const float*> norms[4];
    std::vector<const SignLinear*> lin[7];
    for (const auto& l : m_.layers) {
        norms[0].push_back(l->attn_norm.data());
        norms[1].push_back(l->ffn_norm.data());
        norms[2].push_back(l->q_norm.data());
        norms[3].push_back(l->k_norm.data());
        const SignLinear* proj[7] = {&l->q, &l->k, &l->v, &l->o, &l->gate, &l->up, &l->down};
        for (int i = 0; i < 7; ++i)
            lin[i].push_back(proj[i]);
    }
    ResidentModel rm{};
    rm.C = s_.width, rm.H = s_.heads, rm.Hk = s_.kv_heads, rm.HD = s_.head_dim, rm.FF = s_.ffn;
    rm.L = s_.layers, rm.V = s_.vocab, rm.kv_dim = s_.kv_width, rm.n_ctx = params.n_ctx, rm.eps = s_.eps;
    rm.attn_norm = norms[0].data(), rm.ffn_norm = norms[1].data();
    rm.q_norm = norms[2].data(), rm.k_norm = norms[3].data(), rm.final_norm = m_.final_norm.data();
    rm.emb_bits = m_.embedding.bits.data(), rm.emb_scales = m_.embedding.scales.data();
    rm.rope_cos = cos_.data(), rm.rope_sin = sin_.data();
    rm.wq = lin[0].data(), rm.wk = lin[1].data(), rm.wv = lin[2].data(), rm.wo = lin[3].data();
    rm.gate = lin[4].data(), rm.up = lin[5].data(), rm.down = lin[6].data(), rm.lm_head = &m_.lm_head;
    return resident_create(this, rm, fused, out);
}

void Qwen3Context::select_path(int path) {
    if (path < 0 || path > 2)
        raise(BNNE_EINVAL, "decode path %d (0 host, 1 device with fused batches, 2 device)", path);
    if (path == this->path())
        return;
    if (pos != 0)
        raise(BNNE_EINVAL, "the decode path is chosen before the first token");
    if (path == 0) {
        host_cache();
        resident_free(device_);
        device_ = nullptr;
        return;
    }
    Resident* fresh = nullptr;
    const BNNE_Status st = open_device_path(path == 1, &fresh);
    if (st != BNNE_OK)
        throw Failure{st};
    resident_free(device_);
    device_ = fresh;
    std::vector<float>().swap(keys_);
    std::vector<float>().swap(values_);
}

// out = x / rms * gain with rms = sqrt(sum of x_i^2 in index order / n + eps) (qwen3.c:342-353);
// out may be x.
void scale_rows(const float* x, float rms, const float* gain, float* out, uint32_t n);

void rmsnorm(const float* x, uint32_t n, float eps, const float* gain, float* out) {
    float squares = 0.0f;
    for (uint32_t i = 0; i < n; ++i)
        squares += x[i] * x[i];
    const float rms = sqrtf(squares / (float)n + eps);
    if (!std::isfinite(rms) || rms == 0.0f)
        raise(BNNE_ECOMPUTE, "RMSNorm divisor is zero or not finite");
    scale_rows(x, rms, gain, out, n);
}

// Rotates the pairs (j, j + half) of one head (qwen3.c:368-376).
void rotate(float* head, const float* c, const float* s, uint32_t half) {
    for (uint32_t j = 0; j < half; ++j) {
        const float a = head[j], b = head[j + half];
        head[j] = a * c[j] - b * s[j];
        head[j + half] = a * s[j] + b * c[j];
    }
}

// Eight binary32 lanes (GCC vector extension).  The target clones below compile them to
// AVX2 on processors that have it and to pairs of SSE2 operations elsewhere; neither
// enables FMA.  Only lane-wise multiplies and adds are used, each rounded once, and each
// lane carries one sum of the scalar loop in the scalar loop's order, so the results are
// those of the scalar loops bit for bit.
typedef float f32x8 __attribute__((vector_size(32)));
// the same, for loads and stores at any float address
typedef float f32x8_at __attribute__((vector_size(32), aligned(4), may_alias));
#define LOAD8(p) (*(const f32x8_at*)(p))
#define STORE8(p, v) (*(f32x8_at*)(p) = (v))

// scores[t] = (q . key_t) * scale for t < 8 * ceil(n / 8) (qwen3.c:441-452), each dot in
// index order.  The keys of a head come in blocks of eight positions, kb[(t / 8) * dim * 8
// + i * 8 + t % 8] = key_t[i], so that eight positions' sums advance as the lanes of one
// vector over contiguous memory; the lanes past n compute values that are not used.
__attribute__((target_clones("avx2", "default"))) void
key_scores(const float* q, const float* kb, uint32_t dim, uint32_t n, float scale, float* scores) {
    const uint32_t blocks = (n + 7u) / 8u;
    const size_t stride = (size_t)dim * 8u;
    const float sc = scale;
    uint32_t b = 0;
    for (; b + 4u <= blocks; b += 4u) {
        const float* k = kb + b * stride;
        f32x8 d0 = {}, d1 = {}, d2 = {}, d3 = {};
        for (uint32_t i = 0; i < dim; ++i) {
            const float qi = q[i];
            d0 += qi * LOAD8(k + i * 8u);
            d1 += qi * LOAD8(k + stride + i * 8u);
            d2 += qi * LOAD8(k + 2u * stride + i * 8u);
            d3 += qi * LOAD8(k + 3u * stride + i * 8u);
        }
        STORE8(scores + 8u * b, d0 * sc);
        STORE8(scores + 8u * b + 8u, d1 * sc);
        STORE8(scores + 8u * b + 16u, d2 * sc);
        STORE8(scores + 8u * b + 24u, d3 * sc);
    }
    for (; b < blocks; ++b) {
        const float* k = kb + b * stride;
        f32x8 d = {};
        for (uint32_t i = 0; i < dim; ++i)
            d += q[i] * LOAD8(k + i * 8u);
        STORE8(scores + 8u * b, d * sc);
    }
}

// out[i] = sum over t < n in position order of p[t] * v[t * dim + i], i < dim
// (qwen3.c:466-478): the lanes are eight of the outputs.
__attribute__((target_clones("avx2", "default"))) void
weighted_rows(const float* p, const float* v, uint32_t n, uint32_t dim, float* out) {
    uint32_t i = 0;
    for (; i + 64u <= dim; i += 64u) {
        f32x8 a0 = {}, a1 = {}, a2 = {}, a3 = {}, a4 = {}, a5 = {}, a6 = {}, a7 = {};
        for (uint32_t t = 0; t < n; ++t) {
            const float* r = v + (size_t)t * dim + i;
            const float pt = p[t];
            a0 += pt * LOAD8(r);
            a1 += pt * LOAD8(r + 8);
            a2 += pt * LOAD8(r + 16);
            a3 += pt * LOAD8(r + 24);
            a4 += pt * LOAD8(r + 32);
            a5 += pt * LOAD8(r + 40);
            a6 += pt * LOAD8(r + 48);
            a7 += pt * LOAD8(r + 56);
        }
        STORE8(out + i, a0);
        STORE8(out + i + 8, a1);
        STORE8(out + i + 16, a2);
        STORE8(out + i + 24, a3);
        STORE8(out + i + 32, a4);
        STORE8(out + i + 40, a5);
        STORE8(out + i + 48, a6);
        STORE8(out + i + 56, a7);
    }
    for (; i + 8u <= dim; i += 8u) {
        f32x8 a = {};
        for (uint32_t t = 0; t < n; ++t)
            a += p[t] * LOAD8(v + (size_t)t * dim + i);
        STORE8(out + i, a);
    }
    for (; i < dim; ++i) {
        float a = 0.0f;
        for (uint32_t t = 0; t < n; ++t)
            a += p[t] * v[(size_t)t * dim + i];
        out[i] = a;
    }
}

// out[i] = expf(in[i]) for i < n, bit for bit the host C library's expf (host_expf.h).
void expf_rows(const float* in, float* out, uint32_t n) {
    static const bool lanes = bnne_expf_lanes_usable();
    if (lanes) {
        bnne_expf_lanes(in, out, n);
        return;
    }
    for (uint32_t i = 0; i < n; ++i)
        out[i] = expf(in[i]);
}

// out[i] = x[i] / rms * gain[i], each operation rounded once, eight lanes at a time
// (out may be x).
__attribute__((target_clones("avx2", "default"))) void
scale_rows(const float* x, float rms, const float* gain, float* out, uint32_t n) {
    uint32_t i = 0;
    for (; i + 8u <= n; i += 8u)
        STORE8(out + i, LOAD8(x + i) / rms * LOAD8(gain + i));
    for (; i < n; ++i)
        out[i] = x[i] / rms * gain[i];
}

// x[i] += o[i], eight lanes at a time.
__attribute__((target_clones("avx2", "default"))) void add_rows(float* x, const float* o, uint32_t n) {
    uint32_t i = 0;
    for (; i + 8u <= n; i += 8u)
        STORE8(x + i, LOAD8(x + i) + LOAD8(o + i));
    for (; i < n; ++i)
        x[i] += o[i];
}

// gate[i] = gate[i] / (1 + e[i]) * up[i] (SiLU(gate) * up with e = expf(-gate),
// qwen3.c:491-495), each operation rounded once, eight lanes at a time.
__attribute__((target_clones("avx2", "default"))) void
silu_mul(float* gate, const float* e, const float* up, uint32_t n) {
    uint32_t i = 0;
    for (; i + 8u <= n; i += 8u) {
        const f32x8 one = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
        STORE8(gate + i, LOAD8(gate + i) / (one + LOAD8(e + i)) * LOAD8(up + i));
    }
    for (; i < n; ++i)
        gate[i] = gate[i] / (1.0f + e[i]) * up[i];
}

// Every query head against cache rows 0..pos of its key/value head (qwen3.c:441-478):
// scores q.k * (1 / sqrt(head_dim)), softmax, probability-weighted sum of the values.
void Qwen3Context::attend(uint32_t layer, uint32_t pos) {
    const uint32_t HD = s_.head_dim, group = s_.heads / s_.kv_heads;
    const float scale = 1.0f / sqrtf((float)HD);
    for (uint32_t h = 0; h < s_.heads; ++h) {
        const float* q = q_.data() + (size_t)h * HD;
        const size_t kv = (size_t)layer * s_.kv_heads + h / group;
        key_scores(q, keys_.data() + kv * HD * ctx_blocks_ * 8u, HD, pos + 1u, scale, scores_.data());
        float top = -INFINITY;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float score = scores_[t];
            if (!std::isfinite(score))
                raise(BNNE_ECOMPUTE, "non-finite attention score");
            if (score > top)
                top = score;
        }
        for (uint32_t t = 0; t <= pos; ++t)
            probs_[t] = scores_[t] - top;
        expf_rows(probs_.data(), probs_.data(), pos + 1u);
        float total = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t)
            total += probs_[t];
        if (!(total > 0.0f) || !std::isfinite(total))
            raise(BNNE_ECOMPUTE, "softmax normaliser is zero or not finite");
        for (uint32_t t = 0; t <= pos; ++t)
            probs_[t] /= total;
        weighted_rows(probs_.data(), values_.data() + kv * params.n_ctx * HD, pos + 1u, HD, y_.data() + (size_t)h * HD);
    }
}

void Qwen3Context::step(uint32_t token, uint32_t pos, float* logits) {
    const uint32_t C = s_.width, HD = s_.head_dim, half = HD / 2;
    // embedding row: +scale / -scale by sign bit (qwen3.c:355-366)
    const uint8_t* bits = m_.embedding.bits.data() + (size_t)token * (C / 8u);
    const uint16_t* scales = m_.embedding.scales.data() + (size_t)token * (C / kGroup);
    for (uint32_t i = 0; i < C; ++i) {
        const float scale = half_to_float(scales[i / kGroup]);
        x_[i] = (bits[i / 8u] >> (i % 8u)) & 1u ? scale : -scale;
    }
    for (uint32_t l = 0; l < s_.layers; ++l) {
        const Layer& L = *m_.layers[l];
        rmsnorm(x_.data(), C, s_.eps, L.attn_norm.data(), norm_.data());
        L.q.apply(*this, norm_.data(), q_.data());
        L.k.apply(*this, norm_.data(), k_.data());
        L.v.apply(*this, norm_.data(), v_.data());
        for (uint32_t h = 0; h < s_.heads; ++h)
            rmsnorm(q_.data() + (size_t)h * HD, HD, s_.eps, L.q_norm.data(), q_.data() + (size_t)h * HD);
        for (uint32_t h = 0; h < s_.kv_heads; ++h)
            rmsnorm(k_.data() + (size_t)h * HD, HD, s_.eps, L.k_norm.data(), k_.data() + (size_t)h * HD);
        const float* c = cos_.data() + (size_t)pos * half;
        const float* sn = sin_.data() + (size_t)pos * half;
        for (uint32_t h = 0; h < s_.heads; ++h)
            rotate(q_.data() + (size_t)h * HD, c, sn, half);
        for (uint32_t h = 0; h < s_.kv_heads; ++h)
            rotate(k_.data() + (size_t)h * HD, c, sn, half);
        // per key/value head: the keys in blocks of eight positions, [pos / 8][HD][pos % 8],
        // the values by position, [pos][HD]
        for (uint32_t kh = 0; kh < s_.kv_heads; ++kh) {
            const size_t kv = (size_t)l * s_.kv_heads + kh;
            float* key_lane = keys_.data() + (kv * ctx_blocks_ + pos / 8u) * HD * 8u + pos % 8u;
            for (uint32_t i = 0; i < HD; ++i)
                key_lane[i * 8u] = k_[(size_t)kh * HD + i];
            std::memcpy(values_.data() + (kv * params.n_ctx + pos) * HD, v_.data() + (size_t)kh * HD, HD * sizeof(float));
        }
        attend(l, pos);
        L.o.apply(*this, y_.data(), o_.data());
        add_rows(x_.data(), o_.data(), C);
        rmsnorm(x_.data(), C, s_.eps, L.ffn_norm.data(), norm_.data());
        L.gate.apply(*this, norm_.data(), gate_.data());
        L.up.apply(*this, norm_.data(), up_.data());
        for (uint32_t i = 0; i < s_.ffn; ++i)
            ex_[i] = -gate_[i];
        expf_rows(ex_.data(), ex_.data(), s_.ffn);
        silu_mul(gate_.data(), ex_.data(), up_.data(), s_.ffn);
        L.down.apply(*this, gate_.data(), o_.data());
        add_rows(x_.data(), o_.data(), C);
    }
    if (logits) {
        rmsnorm(x_.data(), C, s_.eps, m_.final_norm.data(), norm_.data());
        m_.lm_head.apply(*this, norm_.data(), logits);
    }
}

void Qwen3Context::decode(const int32_t* tokens, uint32_t n, float* logits) {
    if (device_) {
        const BNNE_Status st = resident_step(this, device_, tokens, n, pos, logits);
        if (st != BNNE_OK)
            throw Failure{st};
        return;
    }
    for (uint32_t i = 0; i < n; ++i)
        step((uint32_t)tokens[i], pos + i, i + 1 == n ? logits : nullptr);
}

void Qwen3Context::decode_greedy(int32_t token, uint32_t n, int32_t* out) {
    if (!device_) {
        bnne_context::decode_greedy(token, n, out);
        return;
    }
    const BNNE_Status st = resident_greedy(this, device_, token, n, pos, out);
    if (st != BNNE_OK)
        throw Failure{st};
}

bnne_context* Qwen3Model::new_context(const BNNE_ContextParams& p) { return new Qwen3Context(*this, p); }

}  // namespace

bnne_model* make_qwen3() { return new Qwen3Model; }

}  // namespace bnne
