// Qwen3 decoder (architecture "qwen3"): loading from GGUF and the per-token step.
//
// Every linear layer goes through linear_forward (BNN_Execute GEMV_F32); the rest of
// the step runs on the host.  The host arithmetic follows the reference's
// qwen3_step (bnn-sw-v2/qwen3/qwen3.c:396-512) operation for operation -- the same
// sequential sums, the same division-then-multiply in RMSNorm, the same libm calls
// (sqrtf, expf, powf, cosf, sinf, logf) -- and is compiled without FP contraction,
// so that with bit-exact linear results the logits are bit-identical.
//
// Model layout (qwen3.c:144-274): token_embd.weight is Q1_0 [C, V] and doubles as the
// lm_head (tied embeddings); per layer attn_norm, ffn_norm (C), attn_q_norm,
// attn_k_norm (head_dim) in F32/F16, and Q1_0 attn_q/k/v/output, ffn_gate/up/down.
#include "engine_internal.h"
#include "resident.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <math.h>

namespace bnne {
namespace {

constexpr uint32_t kMaxLayers = 128, kMaxHeads = 256, kMaxVocab = 1u << 20;
constexpr double kPi = 3.14159265358979323846;

struct Block {
    float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    Linear wq, wk, wv, wo, gate, up, down;
};

struct Model {
    uint32_t C, H, Hk, HD, FF, L, V, kv_dim;
    float eps, rope_base, rope_freq_scale, rope_mscale;
    int32_t rope_corr0, rope_corr1;
    bool rope_yarn;
    uint8_t* emb_bits;
    uint16_t* emb_scales;
    Linear lm_head;
    float* final_norm;
    Block* blocks;
};

struct State {
    uint32_t n_ctx;
    float *x, *norm, *q, *k, *v, *y, *o, *gate, *up, *scores, *probs;
    float *k_cache, *v_cache, *rope_cos, *rope_sin;  // host KV cache: host step only
    Resident* resident;  // device-resident step when non-null
};

float* alloc_f32(size_t count) {
    if (!count || count > SIZE_MAX / sizeof(float))
        return nullptr;
    return static_cast<float*>(std::malloc(count * sizeof(float)));
}

void unload(void* impl) {
    Model* m = static_cast<Model*>(impl);
    if (!m)
        return;
    if (m->blocks) {
        for (uint32_t l = 0; l < m->L; ++l) {
            Block& b = m->blocks[l];
            std::free(b.attn_norm);
            std::free(b.q_norm);
            std::free(b.k_norm);
            std::free(b.ffn_norm);
            for (Linear* lin : {&b.wq, &b.wk, &b.wv, &b.wo, &b.gate, &b.up, &b.down})
                linear_free(lin);
        }
    }
    std::free(m->blocks);
    linear_free(&m->lm_head);
    std::free(m->final_norm);
    std::free(m->emb_bits);
    std::free(m->emb_scales);
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

BNNE_Status load_linear(bnne_model* mm, const Gguf* g, const char* name, uint32_t in, uint32_t out, Linear* l) {
    const BNNE_Status st = linear_load(mm, g, name, l);
    if (st != BNNE_OK)
        return st;
    if (l->in != in || l->out != out) {
        const uint32_t ai = l->in, ao = l->out;
        linear_free(l);
        return error(BNNE_EFORMAT, "tensor '%s' has shape %u->%u, expected %u->%u", name, ai, ao, in, out);
    }
    return BNNE_OK;
}

int32_t clamp_dim(double v, int32_t lo, int32_t hi) {
    if (v <= (double)lo)
        return lo;
    if (v >= (double)hi)
        return hi;
    return (int32_t)v;
}

// RoPE scaling parameters (qwen3.c:125-142): plain scaling by 1/factor, or YaRN with
// the correction range from the original context length.
BNNE_Status init_rope(Model* m, const Gguf* g) {
    const float freq_scale = 1.0f / g->rope_factor;
    const bool yarn = std::strcmp(g->rope_scaling_type, "yarn") == 0;
    int32_t corr0 = 0, corr1 = (int32_t)(m->HD - 1);
    float mscale = 1.0f;
    if (yarn && g->rope_original_context) {
        const double base = m->rope_base, orig = (double)g->rope_original_context;
        const double lo = std::floor((double)m->HD * std::log(orig / (32.0 * 2.0 * kPi)) / (2.0 * std::log(base)));
        const double hi = std::ceil((double)m->HD * std::log(orig / (2.0 * kPi)) / (2.0 * std::log(base)));
        corr0 = clamp_dim(lo, 0, (int32_t)m->HD - 1);
        corr1 = clamp_dim(hi, 0, (int32_t)m->HD - 1);
        mscale = 1.0f + 0.1f * logf(1.0f / freq_scale);
    }
    if (!(freq_scale > 0.0f) || !std::isfinite(mscale))
        return error(BNNE_EFORMAT, "invalid Qwen3 rope scaling");
    m->rope_freq_scale = freq_scale;
    m->rope_mscale = mscale;
    m->rope_corr0 = corr0;
    m->rope_corr1 = corr1;
    m->rope_yarn = yarn;
    return BNNE_OK;
}

BNNE_Status load(bnne_model* mm, const Gguf* g, void** out_impl) {
    *out_impl = nullptr;
    Model* m = static_cast<Model*>(std::calloc(1, sizeof(Model)));
    if (!m)
        return error(BNNE_ENOMEM, "out of memory");
    const GgufTensor* emb = gguf_find(g, "token_embd.weight");
    if (!emb || emb->type != kTypeQ1_0 || emb->rank != 2) {
        unload(m);
        return error(BNNE_EFORMAT, "missing token_embd.weight");
    }
    if (g->block_count == 0 || g->block_count > kMaxLayers || g->embedding_length == 0 ||
        g->embedding_length > UINT32_MAX || g->feed_forward_length == 0 || g->feed_forward_length > UINT32_MAX ||
        g->head_count == 0 || g->head_count > kMaxHeads || g->head_count_kv == 0 || g->head_count_kv > kMaxHeads ||
        g->key_length == 0 || g->key_length > UINT32_MAX || g->key_length != g->value_length ||
        g->context_length == 0 || g->context_length > UINT32_MAX || g->rms_epsilon <= 0.0f ||
        g->rope_freq_base <= 0.0f || emb->dims[0] != g->embedding_length || emb->dims[1] == 0 ||
        emb->dims[1] > kMaxVocab) {
        unload(m);
        return error(BNNE_EFORMAT, "unsupported Qwen3 dimensions");
    }
    m->L = (uint32_t)g->block_count;
    m->C = (uint32_t)g->embedding_length;
    m->FF = (uint32_t)g->feed_forward_length;
    m->H = (uint32_t)g->head_count;
    m->Hk = (uint32_t)g->head_count_kv;
    m->HD = (uint32_t)g->key_length;
    m->V = (uint32_t)emb->dims[1];
    m->eps = g->rms_epsilon;
    m->rope_base = g->rope_freq_base;
    if (m->HD > m->C || (uint64_t)m->H * m->HD != m->C || m->H % m->Hk != 0 || m->C % kGroup != 0 ||
        m->FF % kGroup != 0 || m->HD % 2 != 0) {
        unload(m);
        return error(BNNE_EFORMAT, "inconsistent Qwen3 dimensions");
    }
    m->kv_dim = m->Hk * m->HD;
    if (m->kv_dim % kGroup != 0) {
        unload(m);
        return error(BNNE_EFORMAT, "Qwen3 KV width is not group aligned");
    }
    if (mm->caps.group_size != kGroup || !(mm->caps.supported_ops & BNN_CAP_GEMV_F32)) {
        unload(m);
        return error(BNNE_ENOTSUP, "Qwen3 requires group 128 with F32 GEMV support");
    }
    m->blocks = static_cast<Block*>(std::calloc(m->L, sizeof(Block)));
    if (!m->blocks) {
        unload(m);
        return error(BNNE_ENOMEM, "out of memory");
    }
    BNNE_Status st = init_rope(m, g);
    if (st == BNNE_OK)
        st = read_vector(g, "output_norm.weight", m->C, &m->final_norm);
    char name[64];
    for (uint32_t l = 0; st == BNNE_OK && l < m->L; ++l) {
        Block& b = m->blocks[l];
        std::snprintf(name, sizeof name, "blk.%u.attn_norm.weight", l);
        st = read_vector(g, name, m->C, &b.attn_norm);
        if (st != BNNE_OK)
            break;
        std::snprintf(name, sizeof name, "blk.%u.ffn_norm.weight", l);
        st = read_vector(g, name, m->C, &b.ffn_norm);
        if (st != BNNE_OK)
            break;
        std::snprintf(name, sizeof name, "blk.%u.attn_q_norm.weight", l);
        st = read_vector(g, name, m->HD, &b.q_norm);
        if (st != BNNE_OK)
            break;
        std::snprintf(name, sizeof name, "blk.%u.attn_k_norm.weight", l);
        st = read_vector(g, name, m->HD, &b.k_norm);
    }
    if (st == BNNE_OK)
        st = q1_0_read(g, "token_embd.weight", m->C, m->V, &m->emb_bits, &m->emb_scales);
    if (st == BNNE_OK)
        st = linear_init(mm, m->C, m->V, m->emb_bits, m->emb_scales, &m->lm_head);
    for (uint32_t l = 0; st == BNNE_OK && l < m->L; ++l) {
        Block& b = m->blocks[l];
        struct {
            const char* suffix;
            uint32_t in, out;
            Linear* lin;
        } const parts[] = {
            {"attn_q", m->C, m->C, &b.wq},       {"attn_k", m->C, m->kv_dim, &b.wk},
            {"attn_v", m->C, m->kv_dim, &b.wv},  {"attn_output", m->C, m->C, &b.wo},
            {"ffn_gate", m->C, m->FF, &b.gate},  {"ffn_up", m->C, m->FF, &b.up},
            {"ffn_down", m->FF, m->C, &b.down},
        };
        for (const auto& p : parts) {
            std::snprintf(name, sizeof name, "blk.%u.%s.weight", l, p.suffix);
            st = load_linear(mm, g, name, p.in, p.out, p.lin);
            if (st != BNNE_OK)
                break;
        }
    }
    if (st != BNNE_OK) {
        unload(m);
        return st;
    }
    mm->info.n_vocab = m->V;
    mm->info.n_ctx_train = (uint32_t)g->context_length;
    *out_impl = m;
    return BNNE_OK;
}

void ctx_free(void* state) {
    State* s = static_cast<State*>(state);
    if (!s)
        return;
    resident_free(s->resident);
    for (float* p : {s->x, s->norm, s->q, s->k, s->v, s->y, s->o, s->gate, s->up, s->scores, s->probs, s->k_cache,
                     s->v_cache, s->rope_cos, s->rope_sin})
        std::free(p);
    std::free(s);
}

// cos/sin tables per (position, pair) (qwen3.c:276-299).
void init_rope_tables(const Model* m, State* s) {
    const uint32_t half = m->HD / 2;
    for (uint32_t pos = 0; pos < s->n_ctx; ++pos) {
        for (uint32_t j = 0; j < half; ++j) {
            const float theta_extrap = (float)pos * powf(m->rope_base, -2.0f * (float)j / (float)m->HD);
            float theta = m->rope_freq_scale * theta_extrap;
            if (m->rope_yarn) {
                const float span = (float)(m->rope_corr1 - m->rope_corr0);
                const float denom = span > 0.001f ? span : 0.001f;
                const float y = ((float)j - (float)m->rope_corr0) / denom;
                const float ramp = 1.0f - fminf(1.0f, fmaxf(0.0f, y));
                theta = (m->rope_freq_scale * theta_extrap) * (1.0f - ramp) + theta_extrap * ramp;
            }
            s->rope_cos[(size_t)pos * half + j] = cosf(theta) * m->rope_mscale;
            s->rope_sin[(size_t)pos * half + j] = sinf(theta) * m->rope_mscale;
        }
    }
}

BNNE_Status alloc_host_cache(const Model* m, State* s) {
    const size_t cache = (size_t)m->L * s->n_ctx * m->kv_dim;
    s->k_cache = alloc_f32(cache);
    s->v_cache = alloc_f32(cache);
    if (!s->k_cache || !s->v_cache) {
        std::free(s->k_cache);
        std::free(s->v_cache);
        s->k_cache = s->v_cache = nullptr;
        return error(BNNE_ENOMEM, "out of memory");
    }
    return BNNE_OK;
}

BNNE_Status make_resident(bnne_context* c, const Model* m, State* s, bool fused) {
    const float* attn[kMaxLayers];
    const float* ffn[kMaxLayers];
    const float* qn[kMaxLayers];
    const float* kn[kMaxLayers];
    const Linear* lin[7][kMaxLayers];
    for (uint32_t l = 0; l < m->L; ++l) {
        const Block& b = m->blocks[l];
        attn[l] = b.attn_norm, ffn[l] = b.ffn_norm, qn[l] = b.q_norm, kn[l] = b.k_norm;
        lin[0][l] = &b.wq, lin[1][l] = &b.wk, lin[2][l] = &b.wv, lin[3][l] = &b.wo;
        lin[4][l] = &b.gate, lin[5][l] = &b.up, lin[6][l] = &b.down;
    }
    ResidentModel rm = {};
    rm.C = m->C, rm.H = m->H, rm.Hk = m->Hk, rm.HD = m->HD, rm.FF = m->FF, rm.L = m->L, rm.V = m->V;
    rm.kv_dim = m->kv_dim, rm.n_ctx = s->n_ctx, rm.eps = m->eps;
    rm.attn_norm = attn, rm.ffn_norm = ffn, rm.q_norm = qn, rm.k_norm = kn, rm.final_norm = m->final_norm;
    rm.emb_bits = m->emb_bits, rm.emb_scales = m->emb_scales, rm.rope_cos = s->rope_cos, rm.rope_sin = s->rope_sin;
    rm.wq = lin[0], rm.wk = lin[1], rm.wv = lin[2], rm.wo = lin[3], rm.gate = lin[4], rm.up = lin[5];
    rm.down = lin[6], rm.lm_head = &m->lm_head;
    return resident_create(c, rm, fused, &s->resident);
}

// Every context starts on the device-resident step; one whose shapes that step
// does not support (resident_create: ENOTSUP) runs the host step.
BNNE_Status ctx_init(bnne_context* c, void** out_state) {
    *out_state = nullptr;
    const Model* m = static_cast<const Model*>(c->model->impl);
    State* s = static_cast<State*>(std::calloc(1, sizeof(State)));
    if (!s)
        return error(BNNE_ENOMEM, "out of memory");
    s->n_ctx = c->params.n_ctx;
    const size_t half = m->HD / 2;
    s->x = alloc_f32(m->C);
    s->norm = alloc_f32(m->C);
    s->q = alloc_f32(m->C);
    s->y = alloc_f32(m->C);
    s->o = alloc_f32(m->C);
    s->k = alloc_f32(m->kv_dim);
    s->v = alloc_f32(m->kv_dim);
    s->gate = alloc_f32(m->FF);
    s->up = alloc_f32(m->FF);
    s->scores = alloc_f32(s->n_ctx);
    s->probs = alloc_f32(s->n_ctx);
    s->rope_cos = alloc_f32((size_t)s->n_ctx * half);
    s->rope_sin = alloc_f32((size_t)s->n_ctx * half);
    if (!s->x || !s->norm || !s->q || !s->y || !s->o || !s->k || !s->v || !s->gate || !s->up || !s->scores ||
        !s->probs || !s->rope_cos || !s->rope_sin) {
        ctx_free(s);
        return error(BNNE_ENOMEM, "out of memory");
    }
    init_rope_tables(m, s);
    BNNE_Status st = make_resident(c, m, s, true);
    if (st == BNNE_ENOTSUP) {
        error_clear();
        st = alloc_host_cache(m, s);
    }
    if (st != BNNE_OK) {
        ctx_free(s);
        return st;
    }
    *out_state = s;
    return BNNE_OK;
}

// out = x / rms * gain, rms = sqrt(sum x^2 / n + eps), sum in index order (qwen3.c:342-353).
BNNE_Status rmsnorm(const float* x, uint32_t n, float eps, const float* gain, float* out) {
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i)
        sum += x[i] * x[i];
    const float rms = sqrtf(sum / (float)n + eps);
    if (!std::isfinite(rms) || rms == 0.0f)
        return error(BNNE_ECOMPUTE, "Qwen3 RMSNorm produced a non-finite divisor");
    for (uint32_t i = 0; i < n; ++i)
        out[i] = x[i] / rms * gain[i];
    return BNNE_OK;
}

// Embedding row: +scale where the sign bit is 1, -scale where 0 (qwen3.c:355-366).
void embed(const Model* m, uint32_t token, float* out) {
    const uint8_t* bits = m->emb_bits + (size_t)token * (m->C / 8u);
    const uint16_t* scales = m->emb_scales + (size_t)token * (m->C / kGroup);
    for (uint32_t g = 0; g < m->C / kGroup; ++g) {
        const float s = fp16_to_fp32(scales[g]);
        for (uint32_t j = 0; j < kGroup; ++j) {
            const bool bit = (bits[g * 16 + (j >> 3)] >> (j & 7u)) & 1u;
            out[g * kGroup + j] = bit ? s : -s;
        }
    }
}

// Rotation of the pairs (j, j + half) (qwen3.c:368-376).
void rope(float* v, const float* cs, const float* sn, uint32_t half) {
    for (uint32_t j = 0; j < half; ++j) {
        const float a = v[j], b = v[j + half];
        v[j] = a * cs[j] - b * sn[j];
        v[j + half] = a * sn[j] + b * cs[j];
    }
}

// Causal attention of all heads against cache rows 0..pos (qwen3.c:441-478).
BNNE_Status attention(const Model* m, State* s, uint32_t layer, uint32_t pos) {
    const uint32_t kv_mul = m->H / m->Hk;
    const float scale = 1.0f / sqrtf((float)m->HD);
    const float* kc = s->k_cache + (size_t)layer * s->n_ctx * m->kv_dim;
    const float* vc = s->v_cache + (size_t)layer * s->n_ctx * m->kv_dim;
    for (uint32_t h = 0; h < m->H; ++h) {
        const size_t head_off = (size_t)(h / kv_mul) * m->HD;
        const float* q = s->q + (size_t)h * m->HD;
        float maximum = -INFINITY;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float* key = kc + (size_t)t * m->kv_dim + head_off;
            float dot = 0.0f;
            for (uint32_t i = 0; i < m->HD; ++i)
                dot += q[i] * key[i];
            const float score = dot * scale;
            if (!std::isfinite(score))
                return error(BNNE_ECOMPUTE, "Qwen3 attention score is not finite");
            s->scores[t] = score;
            if (score > maximum)
                maximum = score;
        }
        float sum = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float p = expf(s->scores[t] - maximum);
            s->probs[t] = p;
            sum += p;
        }
        if (!(sum > 0.0f) || !std::isfinite(sum))
            return error(BNNE_ECOMPUTE, "Qwen3 attention softmax failed");
        for (uint32_t t = 0; t <= pos; ++t)
            s->probs[t] /= sum;
        for (uint32_t i = 0; i < m->HD; ++i) {
            float acc = 0.0f;
            for (uint32_t t = 0; t <= pos; ++t)
                acc += s->probs[t] * vc[(size_t)t * m->kv_dim + head_off + i];
            s->y[(size_t)h * m->HD + i] = acc;
        }
    }
    return BNNE_OK;
}

#define TRY(expr)                          \
    do {                                   \
        const BNNE_Status st_ = (expr);    \
        if (st_ != BNNE_OK)                \
            return st_;                    \
    } while (0)

BNNE_Status step(bnne_context* c, uint32_t token, uint32_t pos, float* logits) {
    const Model* m = static_cast<const Model*>(c->model->impl);
    State* s = static_cast<State*>(c->state);
    const uint32_t half = m->HD / 2;
    embed(m, token, s->x);
    for (uint32_t l = 0; l < m->L; ++l) {
        const Block& b = m->blocks[l];
        TRY(rmsnorm(s->x, m->C, m->eps, b.attn_norm, s->norm));
        TRY(linear_forward(c, &b.wq, s->norm, s->q));
        TRY(linear_forward(c, &b.wk, s->norm, s->k));
        TRY(linear_forward(c, &b.wv, s->norm, s->v));
        for (uint32_t h = 0; h < m->H; ++h)
            TRY(rmsnorm(s->q + (size_t)h * m->HD, m->HD, m->eps, b.q_norm, s->q + (size_t)h * m->HD));
        for (uint32_t h = 0; h < m->Hk; ++h)
            TRY(rmsnorm(s->k + (size_t)h * m->HD, m->HD, m->eps, b.k_norm, s->k + (size_t)h * m->HD));
        const float* cs = s->rope_cos + (size_t)pos * half;
        const float* sn = s->rope_sin + (size_t)pos * half;
        for (uint32_t h = 0; h < m->H; ++h)
            rope(s->q + (size_t)h * m->HD, cs, sn, half);
        for (uint32_t h = 0; h < m->Hk; ++h)
            rope(s->k + (size_t)h * m->HD, cs, sn, half);
        const size_t at = ((size_t)l * s->n_ctx + pos) * m->kv_dim;
        std::memcpy(s->k_cache + at, s->k, (size_t)m->kv_dim * sizeof(float));
        std::memcpy(s->v_cache + at, s->v, (size_t)m->kv_dim * sizeof(float));
        TRY(attention(m, s, l, pos));
        TRY(linear_forward(c, &b.wo, s->y, s->o));
        for (uint32_t i = 0; i < m->C; ++i)
            s->x[i] += s->o[i];
        TRY(rmsnorm(s->x, m->C, m->eps, b.ffn_norm, s->norm));
        TRY(linear_forward(c, &b.gate, s->norm, s->gate));
        TRY(linear_forward(c, &b.up, s->norm, s->up));
        for (uint32_t i = 0; i < m->FF; ++i) {
            const float g = s->gate[i];
            const float silu = g / (1.0f + expf(-g));
            s->gate[i] = silu * s->up[i];
        }
        TRY(linear_forward(c, &b.down, s->gate, s->o));
        for (uint32_t i = 0; i < m->C; ++i)
            s->x[i] += s->o[i];
    }
    if (logits) {
        TRY(rmsnorm(s->x, m->C, m->eps, m->final_norm, s->norm));
        TRY(linear_forward(c, &m->lm_head, s->norm, logits));
    }
    return BNNE_OK;
}

BNNE_Status decode(bnne_context* c, const int32_t* tokens, uint32_t n, float* logits) {
    State* s = static_cast<State*>(c->state);
    if (s->resident)
        return resident_step(c, s->resident, tokens, n, c->pos, logits);
    for (uint32_t i = 0; i < n; ++i)
        TRY(step(c, (uint32_t)tokens[i], c->pos + i, i + 1 == n ? logits : nullptr));
    return BNNE_OK;
}

// Positions beyond 'pos' are simply overwritten by later steps.
BNNE_Status truncate(bnne_context*, uint32_t) { return BNNE_OK; }

}  // namespace

const Arch kArchQwen3 = {"qwen3", BNNE_TASK_LLM, load, unload, ctx_init, ctx_free, nullptr, decode, truncate};

BNNE_Status qwen3_set_resident(bnne_context* c, int mode) {
    if (c->model->arch != &kArchQwen3)
        return error(BNNE_ENOTSUP, "only qwen3 contexts have a device-resident step");
    if (mode < 0 || mode > 2)
        return error(BNNE_EINVAL, "unknown decode path %d", mode);
    State* s = static_cast<State*>(c->state);
    if (mode == qwen3_resident_mode(c))
        return BNNE_OK;
    if (c->pos != 0)
        return error(BNNE_EINVAL, "the decode path can only change before the first token");
    const Model* m = static_cast<const Model*>(c->model->impl);
    if (mode != 0) {
        Resident* old = s->resident;
        s->resident = nullptr;
        const BNNE_Status st = make_resident(c, m, s, mode == 1);
        if (st != BNNE_OK) {
            s->resident = old;
            return st;
        }
        resident_free(old);
        std::free(s->k_cache);
        std::free(s->v_cache);
        s->k_cache = s->v_cache = nullptr;
        return BNNE_OK;
    }
    const BNNE_Status st = alloc_host_cache(m, s);
    if (st != BNNE_OK)
        return st;
    resident_free(s->resident);
    s->resident = nullptr;
    return BNNE_OK;
}

int qwen3_resident_mode(const bnne_context* c) {
    if (c->model->arch != &kArchQwen3)
        return 0;
    const Resident* r = static_cast<const State*>(c->state)->resident;
    return r == nullptr ? 0 : resident_fused(r) ? 1 : 2;
}

}  // namespace bnne
