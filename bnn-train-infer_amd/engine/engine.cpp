// Public engine API: model load/free, contexts, Decode/Classify dispatch, statistics,
// errors.  Behaviour (argument checks, status codes, statistics taxonomy) follows the
// reference engine (bnn-sw-v2/engine.c:16-338, common.c:1-88).
#include "engine_internal.h"

#include <cfloat>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>

#define BNNE_EXPORT extern "C" __attribute__((visibility("default")))

namespace bnne {

namespace {
thread_local char g_error[192];
}

void error_clear() { g_error[0] = '\0'; }

BNNE_Status error(BNNE_Status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(g_error, sizeof g_error, format, args);
    va_end(args);
    return status;
}

// Accelerator status -> engine status (common.c:27-40).
BNNE_Status accel_error(BNN_Status status, const char* operation) {
    if (status == BNN_OK)
        return BNNE_OK;
    BNNE_Status mapped;
    switch (status) {
    case BNN_ENOMEM: mapped = BNNE_ENOMEM; break;
    case BNN_ENOTSUP: mapped = BNNE_ENOTSUP; break;
    case BNN_ERANGE: mapped = BNNE_ERANGE; break;
    case BNN_EIO: case BNN_ETIMEOUT: mapped = BNNE_EIO; break;
    default: mapped = BNNE_ECOMPUTE; break;
    }
    return error(mapped, "%s: %s", operation, BNN_StatusString(status));
}

uint64_t now_ns() {
    timespec ts;
    if (clock_gettime(CLOCK_MONOTONIC, &ts) != 0)
        return 0;
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

// Exact binary16 -> binary32 (every binary16 value is representable).
float fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1fu, f = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (f << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    } else {
        const float mag = std::ldexp((float)f, -24);  // f * 2^-24, exact
        std::memcpy(&bits, &mag, 4);
        bits |= sign;
    }
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}

const Arch* arch_find(const char* name) {
    static const Arch* const archs[] = {&kArchBnnMlp, &kArchQwen3};
    if (!name)
        return nullptr;
    for (const Arch* a : archs)
        if (std::strcmp(a->name, name) == 0)
            return a;
    return nullptr;
}

}  // namespace bnne

using namespace bnne;

BNNE_EXPORT void BNNE_ModelFree(BNNE_Model model);
BNNE_EXPORT void BNNE_ContextFree(BNNE_Context ctx);
BNNE_EXPORT void BNNE_ContextParamsInit(BNNE_ContextParams* params);

BNNE_EXPORT BNNE_Status BNNE_ModelLoad(BNN_Device device, const char* gguf_path, BNNE_Model* out_model) {
    if (out_model)
        *out_model = nullptr;
    error_clear();
    if (!device || !gguf_path || !out_model)
        return BNNE_EINVAL;
    if (!(sizeof(float) == 4 && FLT_RADIX == 2 && FLT_MANT_DIG == 24 && FLT_MAX_EXP == 128))
        return error(BNNE_ENOTSUP, "IEEE-754 binary32 float is required");
    const uint64_t start = now_ns();
    Gguf* g = nullptr;
    BNNE_Status st = gguf_open(gguf_path, &g);
    if (st != BNNE_OK)
        return st;
    const Arch* arch = arch_find(g->architecture);
    if (!arch) {
        error(BNNE_ENOTSUP, "unsupported GGUF architecture '%s'", g->architecture);
        gguf_close(g);
        return BNNE_ENOTSUP;
    }
    auto* m = static_cast<bnne_model*>(std::calloc(1, sizeof(bnne_model)));
    if (!m) {
        gguf_close(g);
        return error(BNNE_ENOMEM, "out of memory");
    }
    m->device = device;
    m->gguf = g;
    m->arch = arch;
    st = accel_error(BNN_DeviceGetCaps(device, &m->caps), "BNN_DeviceGetCaps");
    if (st == BNNE_OK && (m->caps.api_version != BNN_API_VERSION || m->caps.group_size == 0 ||
                          m->caps.max_in_features == 0 || m->caps.max_out_features == 0 || m->caps.max_rows == 0))
        st = error(BNNE_ENOTSUP, "device does not support this engine");
    if (st == BNNE_OK)
        st = arch->load(m, g, &m->impl);
    if (st != BNNE_OK) {
        BNNE_ModelFree(m);
        return st;
    }
    if (arch->task == BNNE_TASK_LLM) {
        st = vocab_build(g, &m->vocab);
        if (st != BNNE_OK) {
            BNNE_ModelFree(m);
            return st;
        }
        m->info.bos_token = g->has_bos ? (int32_t)g->bos_token_id : -1;
        m->info.eos_token = g->has_eos ? (int32_t)g->eos_token_id : -1;
    }
    m->info.task = arch->task;
    m->info.arch = arch->name;
    m->info.load_ns = now_ns() - start;
    *out_model = m;
    return BNNE_OK;
}

BNNE_EXPORT void BNNE_ModelFree(BNNE_Model m) {
    if (!m)
        return;
    if (m->arch && m->arch->unload && m->impl)
        m->arch->unload(m->impl);
    vocab_free(m->vocab);
    gguf_close(m->gguf);
    std::free(m);
}

BNNE_EXPORT BNNE_Status BNNE_ModelGetInfo(BNNE_Model m, BNNE_ModelInfo* out) {
    if (!m || !out)
        return BNNE_EINVAL;
    *out = m->info;
    return BNNE_OK;
}

// Text encoding is not part of this build: callers pass token IDs.
BNNE_EXPORT BNNE_Status BNNE_Tokenize(BNNE_Model m, const char* text, int, int32_t* ids, uint32_t capacity,
                                      uint32_t* out_count) {
    if (out_count)
        *out_count = 0;
    error_clear();
    if (!m || !text || !ids || !out_count || capacity == 0)
        return BNNE_EINVAL;
    return error(BNNE_ENOTSUP, m->vocab ? "text encoding is not part of this engine build; pass token IDs"
                                        : "model has no text tokenizer");
}

BNNE_EXPORT BNNE_Status BNNE_TokenPiece(BNNE_Model m, int32_t id, const char** out_bytes, size_t* out_len) {
    if (out_bytes)
        *out_bytes = nullptr;
    if (out_len)
        *out_len = 0;
    error_clear();
    if (!m || !out_bytes || !out_len)
        return BNNE_EINVAL;
    if (!m->vocab)
        return error(BNNE_ENOTSUP, "model has no text tokenizer");
    if (id < 0 || (uint64_t)id >= m->vocab->count)
        return BNNE_ERANGE;
    *out_bytes = m->vocab->text + m->vocab->off[id];
    *out_len = m->vocab->len[id];
    return BNNE_OK;
}

BNNE_EXPORT int BNNE_TokenIsEog(BNNE_Model m, int32_t id) {
    if (!m || !m->vocab || id < 0 || (uint32_t)id >= m->info.n_vocab || (uint64_t)id >= m->vocab->count)
        return 0;
    for (uint32_t k = 0; k < m->vocab->n_eog; ++k)
        if (m->vocab->eog[k] == (uint32_t)id)
            return 1;
    return 0;
}

BNNE_EXPORT void BNNE_ContextParamsInit(BNNE_ContextParams* p) {
    if (p) {
        p->n_ctx = 0;
        p->n_batch = 0;
        p->enable_stats = 1;
    }
}

BNNE_EXPORT BNNE_Status BNNE_ContextCreate(BNNE_Model m, const BNNE_ContextParams* params, BNNE_Context* out) {
    if (out)
        *out = nullptr;
    error_clear();
    if (!m || !out)
        return BNNE_EINVAL;
    auto* c = static_cast<bnne_context*>(std::calloc(1, sizeof(bnne_context)));
    if (!c)
        return error(BNNE_ENOMEM, "out of memory");
    c->model = m;
    BNNE_ContextParamsInit(&c->params);
    if (params)
        c->params = *params;
    if (m->info.task == BNNE_TASK_LLM) {
        if (c->params.n_ctx == 0)
            c->params.n_ctx = m->info.n_ctx_train;
        if (c->params.n_ctx == 0 || c->params.n_ctx > m->info.n_ctx_train) {
            const uint32_t n = c->params.n_ctx;
            BNNE_ContextFree(c);
            return error(BNNE_ERANGE, "context length %u exceeds model capacity %u", n, m->info.n_ctx_train);
        }
        if (c->params.n_batch == 0 || c->params.n_batch > c->params.n_ctx)
            c->params.n_batch = c->params.n_ctx;
    } else if (c->params.n_batch == 0) {
        c->params.n_batch = 1;
    }
    if (m->arch->ctx_init) {
        const BNNE_Status st = m->arch->ctx_init(c, &c->state);
        if (st != BNNE_OK) {
            BNNE_ContextFree(c);
            return st;
        }
    }
    c->max_in = m->max_in ? m->max_in : 1;
    c->max_out = m->max_out ? m->max_out : 1;
    BNNE_Status st = accel_error(BNN_BufferAlloc(m->device, (size_t)c->max_in * sizeof(float), &c->in_buf),
                                 "BNN_BufferAlloc(input)");
    if (st == BNNE_OK)
        st = accel_error(BNN_BufferAlloc(m->device, (size_t)c->max_out * sizeof(float), &c->out_buf),
                         "BNN_BufferAlloc(output)");
    if (st != BNNE_OK) {
        BNNE_ContextFree(c);
        return st;
    }
    c->pos = 0;
    *out = c;
    return BNNE_OK;
}

BNNE_EXPORT void BNNE_ContextFree(BNNE_Context c) {
    if (!c)
        return;
    if (c->model && c->model->arch && c->model->arch->ctx_free && c->state)
        c->model->arch->ctx_free(c->state);
    BNN_BufferFree(c->in_buf);
    BNN_BufferFree(c->out_buf);
    std::free(c);
}

namespace {
struct StatsMark {
    BNNE_Stats before;
    uint64_t start;
};

void stats_begin(bnne_context* c, StatsMark* mark) {
    if (!c->params.enable_stats)
        return;
    mark->before = c->stats;
    mark->start = now_ns();
}

// total = quantize + transfer + execute + host: the host share is what the stages
// accumulated during the call did not account for (engine.c:225-239).
void stats_end(bnne_context* c, const StatsMark* mark, uint64_t items) {
    if (!c->params.enable_stats)
        return;
    const uint64_t end = now_ns();
    const uint64_t total = end > mark->start ? end - mark->start : 0;
    const uint64_t stages = (c->stats.quantize_ns - mark->before.quantize_ns) +
                            (c->stats.transfer_ns - mark->before.transfer_ns) +
                            (c->stats.execute_ns - mark->before.execute_ns);
    c->stats.total_ns += total;
    c->stats.host_ns += total > stages ? total - stages : 0;
    c->stats.calls++;
    c->stats.items += items;
}
}  // namespace

BNNE_EXPORT BNNE_Status BNNE_Decode(BNNE_Context c, const int32_t* tokens, uint32_t n, float* logits) {
    error_clear();
    if (!c || !tokens || n == 0)
        return BNNE_EINVAL;
    if (c->model->info.task != BNNE_TASK_LLM || !c->model->arch->decode)
        return error(BNNE_ENOTSUP, "model is not a language model");
    if (n > c->params.n_batch)
        return error(BNNE_ERANGE, "token count exceeds context batch size");
    if (c->pos > c->params.n_ctx || n > c->params.n_ctx - c->pos)
        return error(BNNE_ERANGE, "decode exceeds context length");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= c->model->info.n_vocab)
            return error(BNNE_ERANGE, "token ID is outside vocabulary");
    StatsMark mark = {};
    stats_begin(c, &mark);
    const BNNE_Status st = c->model->arch->decode(c, tokens, n, logits);
    if (st != BNNE_OK)
        return st;
    if (logits)
        for (uint32_t i = 0; i < c->model->info.n_vocab; ++i)
            if (!std::isfinite(logits[i]))
                return error(BNNE_ECOMPUTE, "model produced NaN or Inf logits");
    c->pos += n;
    stats_end(c, &mark, n);
    return BNNE_OK;
}

BNNE_EXPORT BNNE_Status BNNE_Classify(BNNE_Context c, const float* input, uint32_t n, float* logits) {
    error_clear();
    if (!c || !input || !logits || n == 0)
        return BNNE_EINVAL;
    if (c->model->info.task != BNNE_TASK_CLASSIFY || !c->model->arch->classify)
        return error(BNNE_ENOTSUP, "model is not a classifier");
    if (n > c->params.n_batch)
        return error(BNNE_ERANGE, "sample count exceeds context batch size");
    const uint64_t inputs = (uint64_t)n * c->model->info.input_size;
    for (uint64_t i = 0; i < inputs; ++i)
        if (!std::isfinite(input[i]))
            return error(BNNE_EINVAL, "input contains NaN or Inf");
    StatsMark mark = {};
    stats_begin(c, &mark);
    const BNNE_Status st = c->model->arch->classify(c, input, n, logits);
    if (st != BNNE_OK)
        return st;
    const uint64_t outputs = (uint64_t)n * c->model->info.n_classes;
    for (uint64_t i = 0; i < outputs; ++i)
        if (!std::isfinite(logits[i]))
            return error(BNNE_ECOMPUTE, "model produced NaN or Inf logits");
    stats_end(c, &mark, n);
    return BNNE_OK;
}

BNNE_EXPORT uint32_t BNNE_ContextPos(BNNE_Context c) { return c ? c->pos : 0; }

BNNE_EXPORT BNNE_Status BNNE_ContextTruncate(BNNE_Context c, uint32_t pos) {
    error_clear();
    if (!c)
        return BNNE_EINVAL;
    if (pos > c->pos)
        return error(BNNE_EINVAL, "truncate position is beyond current position");
    if (c->model->info.task == BNNE_TASK_LLM && c->model->arch->truncate) {
        const BNNE_Status st = c->model->arch->truncate(c, pos);
        if (st != BNNE_OK)
            return st;
    }
    c->pos = pos;
    return BNNE_OK;
}

BNNE_EXPORT BNNE_Status BNNE_ContextGetStats(BNNE_Context c, BNNE_Stats* out) {
    if (!c || !out)
        return BNNE_EINVAL;
    *out = c->stats;
    return BNNE_OK;
}

BNNE_EXPORT BNNE_Status BNNE_ContextResetStats(BNNE_Context c) {
    if (!c)
        return BNNE_EINVAL;
    std::memset(&c->stats, 0, sizeof c->stats);
    return BNNE_OK;
}

BNNE_EXPORT const char* BNNE_StatusString(BNNE_Status s) {
    switch (s) {
    case BNNE_OK: return "success";
    case BNNE_EINVAL: return "invalid argument";
    case BNNE_ENOMEM: return "out of memory";
    case BNNE_ENOTSUP: return "unsupported model or device capability";
    case BNNE_ERANGE: return "size or capacity out of range";
    case BNNE_EIO: return "I/O error";
    case BNNE_EFORMAT: return "invalid or truncated model";
    case BNNE_ECOMPUTE: return "computation failed or produced non-finite values";
    default: return "unknown status";
    }
}

BNNE_EXPORT const char* BNNE_LastError(void) { return g_error; }

// ---- extensions (include/bnn-engine-hip.h) ----

BNNE_EXPORT BNNE_Status BNNEX_ContextSetResident(BNNE_Context c, int enable) {
    error_clear();
    if (!c)
        return BNNE_EINVAL;
    return qwen3_set_resident(c, enable);
}

BNNE_EXPORT int BNNEX_ContextIsResident(BNNE_Context c) { return c ? qwen3_resident_mode(c) : 0; }
