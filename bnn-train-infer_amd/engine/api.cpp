// The exported engine API (include/bnn-engine.h, include/bnn-engine-hip.h).
//
// Each entry point checks its arguments, then runs the work under guarded(), which
// turns a thrown Failure back into the status code.  What callers see -- the checks,
// the statuses, the rule that failed create calls leave *out NULL, the statistics
// taxonomy (total = quantize + transfer + execute + host, counted for successful
// Classify/Decode calls) -- is the contract of the reference engine
// (bnn-sw-v2/engine.c:16-338), on which the reference CLI relies.
#include "engine.hpp"

#include <cfloat>
#include <cmath>
#include <cstring>

#define BNNE_EXPORT extern "C" __attribute__((visibility("default")))

namespace bnne {

namespace {

bool binary32_floats() { return sizeof(float) == 4 && FLT_RADIX == 2 && FLT_MANT_DIG == 24 && FLT_MAX_EXP == 128; }

// Counts one successful Classify/Decode call: its wall time, and as host time the part
// the stage counters (quantize, transfer, execute) did not take during the call.
class CallStats {
public:
    explicit CallStats(bnne_context& ctx) : ctx_(ctx), on_(ctx.params.enable_stats != 0) {
        if (on_) {
            start_ = clock_ns();
            staged_ = staged();
        }
    }
    void done(uint64_t items) {
        if (!on_)
            return;
        const uint64_t now = clock_ns();
        const uint64_t total = now > start_ ? now - start_ : 0;
        const uint64_t stages = staged() - staged_;
        ctx_.stats.total_ns += total;
        ctx_.stats.host_ns += total > stages ? total - stages : 0;
        ctx_.stats.calls += 1;
        ctx_.stats.items += items;
    }

private:
    uint64_t staged() const { return ctx_.stats.quantize_ns + ctx_.stats.transfer_ns + ctx_.stats.execute_ns; }
    bnne_context& ctx_;
    bool on_;
    uint64_t start_ = 0, staged_ = 0;
};

// Branch-free over the bit patterns (an exponent of all ones is an infinity or a NaN) and
// vectorised (this build's -O2 leaves loops scalar): a classify call's input rows, tens of
// thousands of values, are checked on every call.
__attribute__((optimize("tree-vectorize"))) bool all_finite(const float* v, uint64_t n) {
    uint32_t bad = 0;
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t u;
        std::memcpy(&u, v + i, sizeof u);
        bad |= (uint32_t)((u & 0x7F800000u) == 0x7F800000u);
    }
    return bad == 0;
}

}  // namespace
}  // namespace bnne

using namespace bnne;

BNNE_EXPORT BNNE_Status BNNE_ModelLoad(BNN_Device device, const char* gguf_path, BNNE_Model* out_model) {
    if (out_model)
        *out_model = nullptr;
    forget_message();
    if (!device || !gguf_path || !out_model)
        return BNNE_EINVAL;
    return guarded([&] {
        if (!binary32_floats())
            raise(BNNE_ENOTSUP, "the engine needs IEEE-754 binary32 floats");
        const uint64_t start = clock_ns();
        std::unique_ptr<GgufFile> file = GgufFile::open(gguf_path);
        const Architecture* arch = find_architecture(file->architecture());
        if (!arch)
            raise(BNNE_ENOTSUP, "%s: no engine for architecture '%s'", gguf_path, file->architecture().c_str());
        std::unique_ptr<bnne_model> model(arch->make());
        model->device = device;
        model->arch = arch;
        model->file = std::move(file);
        require(BNN_DeviceGetCaps(device, &model->caps), "BNN_DeviceGetCaps");
        const BNN_Caps& caps = model->caps;
        if (caps.api_version != BNN_API_VERSION || caps.group_size == 0 || caps.max_in_features == 0 ||
            caps.max_out_features == 0 || caps.max_rows == 0)
            raise(BNNE_ENOTSUP, "the accelerator's capabilities do not fit this engine");
        model->load();
        if (arch->task == BNNE_TASK_LLM) {  // special tokens: -1 where the file names none
            model->vocab.reset(new Vocab(*model->file));
            const std::optional<uint64_t> bos = model->file->integer("tokenizer.ggml.bos_token_id");
            const std::optional<uint64_t> eos = model->file->integer("tokenizer.ggml.eos_token_id");
            model->info.bos_token = bos ? (int32_t)(uint32_t)*bos : -1;
            model->info.eos_token = eos ? (int32_t)(uint32_t)*eos : -1;
        }
        model->info.task = arch->task;
        model->info.arch = arch->name;
        model->info.load_ns = clock_ns() - start;
        *out_model = model.release();
    });
}

BNNE_EXPORT void BNNE_ModelFree(BNNE_Model model) { delete model; }

BNNE_EXPORT BNNE_Status BNNE_ModelGetInfo(BNNE_Model model, BNNE_ModelInfo* out_info) {
    if (!model || !out_info)
        return BNNE_EINVAL;
    *out_info = model->info;
    return BNNE_OK;
}

// Text is not encoded by this build (callers pass token IDs).
BNNE_EXPORT BNNE_Status BNNE_Tokenize(BNNE_Model model, const char* text, int, int32_t* ids, uint32_t capacity,
                                      uint32_t* out_count) {
    if (out_count)
        *out_count = 0;
    forget_message();
    if (!model || !text || !ids || !out_count || capacity == 0)
        return BNNE_EINVAL;
    return complain(BNNE_ENOTSUP, model->vocab ? "this engine takes token IDs; it does not encode text"
                                               : "the model has no vocabulary");
}

BNNE_EXPORT BNNE_Status BNNE_TokenPiece(BNNE_Model model, int32_t id, const char** out_bytes, size_t* out_len) {
    if (out_bytes)
        *out_bytes = nullptr;
    if (out_len)
        *out_len = 0;
    forget_message();
    if (!model || !out_bytes || !out_len)
        return BNNE_EINVAL;
    if (!model->vocab)
        return complain(BNNE_ENOTSUP, "the model has no vocabulary");
    if (id < 0 || (uint32_t)id >= model->vocab->size())
        return BNNE_ERANGE;
    const std::string_view piece = model->vocab->piece((uint32_t)id);
    *out_bytes = piece.data();
    *out_len = piece.size();
    return BNNE_OK;
}

BNNE_EXPORT int BNNE_TokenIsEog(BNNE_Model model, int32_t id) {
    if (!model || !model->vocab || id < 0 || (uint32_t)id >= model->info.n_vocab ||
        (uint32_t)id >= model->vocab->size())
        return 0;
    return model->vocab->ends_generation((uint32_t)id) ? 1 : 0;
}

BNNE_EXPORT void BNNE_ContextParamsInit(BNNE_ContextParams* params) {
    if (params)
        *params = BNNE_ContextParams{0, 0, 1};
}

BNNE_EXPORT BNNE_Status BNNE_ContextCreate(BNNE_Model model, const BNNE_ContextParams* params, BNNE_Context* out_ctx) {
    if (out_ctx)
        *out_ctx = nullptr;
    forget_message();
    if (!model || !out_ctx)
        return BNNE_EINVAL;
    return guarded([&] {
        BNNE_ContextParams p;
        BNNE_ContextParamsInit(&p);
        if (params)
            p = *params;
        if (model->info.task == BNNE_TASK_LLM) {
            const uint32_t trained = model->info.n_ctx_train;
            if (p.n_ctx == 0)
                p.n_ctx = trained;
            if (p.n_ctx == 0 || p.n_ctx > trained)
                raise(BNNE_ERANGE, "a context of %u tokens is more than the model's %u", p.n_ctx, trained);
            if (p.n_batch == 0 || p.n_batch > p.n_ctx)
                p.n_batch = p.n_ctx;
        } else if (p.n_batch == 0) {
            p.n_batch = 1;
        }
        std::unique_ptr<bnne_context> ctx(model->new_context(p));
        ctx->allocate_staging();
        *out_ctx = ctx.release();
    });
}

BNNE_EXPORT void BNNE_ContextFree(BNNE_Context ctx) { delete ctx; }

BNNE_EXPORT BNNE_Status BNNE_Decode(BNNE_Context ctx, const int32_t* tokens, uint32_t n_tokens, float* logits) {
    forget_message();
    if (!ctx || !tokens || n_tokens == 0)
        return BNNE_EINVAL;
    const BNNE_ModelInfo& info = ctx->model->info;
    if (info.task != BNNE_TASK_LLM)
        return complain(BNNE_ENOTSUP, "the model is not a language model");
    if (n_tokens > ctx->params.n_batch)
        return complain(BNNE_ERANGE, "%u tokens in one call; the context takes %u", n_tokens, ctx->params.n_batch);
    if (ctx->pos > ctx->params.n_ctx || n_tokens > ctx->params.n_ctx - ctx->pos)
        return complain(BNNE_ERANGE, "the tokens do not fit the remaining context");
    for (uint32_t i = 0; i < n_tokens; ++i)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= info.n_vocab)
            return complain(BNNE_ERANGE, "token %d is not in the vocabulary", tokens[i]);
    CallStats call(*ctx);
    ctx->logits_checked = false;
    const BNNE_Status st = guarded([&] { ctx->decode(tokens, n_tokens, logits); });
    if (st != BNNE_OK)
        return st;
    if (logits && !ctx->logits_checked && !all_finite(logits, info.n_vocab))
        return complain(BNNE_ECOMPUTE, "the logits hold a NaN or infinity");
    ctx->pos += n_tokens;
    call.done(n_tokens);
    return BNNE_OK;
}

BNNE_EXPORT BNNE_Status BNNE_Classify(BNNE_Context ctx, const float* input, uint32_t n_samples, float* logits) {
    forget_message();
    if (!ctx || !input || !logits || n_samples == 0)
        return BNNE_EINVAL;
    const BNNE_ModelInfo& info = ctx->model->info;
    if (info.task != BNNE_TASK_CLASSIFY)
        return complain(BNNE_ENOTSUP, "the model is not a classifier");
    if (n_samples > ctx->params.n_batch)
        return complain(BNNE_ERANGE, "%u samples in one call; the context takes %u", n_samples, ctx->params.n_batch);
    if (!all_finite(input, (uint64_t)n_samples * info.input_size))
        return complain(BNNE_EINVAL, "the input holds a NaN or infinity");
    CallStats call(*ctx);
    const BNNE_Status st = guarded([&] { ctx->classify(input, n_samples, logits); });
    if (st != BNNE_OK)
        return st;
    if (!all_finite(logits, (uint64_t)n_samples * info.n_classes))
        return complain(BNNE_ECOMPUTE, "the logits hold a NaN or infinity");
    call.done(n_samples);
    return BNNE_OK;
}

BNNE_EXPORT uint32_t BNNE_ContextPos(BNNE_Context ctx) { return ctx ? ctx->pos : 0; }

BNNE_EXPORT BNNE_Status BNNE_ContextTruncate(BNNE_Context ctx, uint32_t pos) {
    forget_message();
    if (!ctx)
        return BNNE_EINVAL;
    if (pos > ctx->pos)
        return complain(BNNE_EINVAL, "cannot truncate forward, to %u of %u tokens", pos, ctx->pos);
    const BNNE_Status st = guarded([&] { ctx->rewind(pos); });
    if (st == BNNE_OK)
        ctx->pos = pos;
    return st;
}

BNNE_EXPORT BNNE_Status BNNE_ContextGetStats(BNNE_Context ctx, BNNE_Stats* out_stats) {
    if (!ctx || !out_stats)
        return BNNE_EINVAL;
    *out_stats = ctx->stats;
    return BNNE_OK;
}

BNNE_EXPORT BNNE_Status BNNE_ContextResetStats(BNNE_Context ctx) {
    if (!ctx)
        return BNNE_EINVAL;
    ctx->stats = BNNE_Stats{};
    return BNNE_OK;
}

// The status texts are the reference engine's (bnn-sw-v2/common.c), so that logs of
// the two engines read alike.
BNNE_EXPORT const char* BNNE_StatusString(BNNE_Status status) {
    switch (status) {
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

BNNE_EXPORT const char* BNNE_LastError(void) { return last_message(); }

BNNE_EXPORT BNNE_Status BNNEX_ContextSetResident(BNNE_Context ctx, int path) {
    forget_message();
    if (!ctx)
        return BNNE_EINVAL;
    return guarded([&] { ctx->select_path(path); });
}

BNNE_EXPORT int BNNEX_ContextIsResident(BNNE_Context ctx) { return ctx ? ctx->path() : 0; }

BNNE_EXPORT BNNE_Status BNNEX_DecodeGreedy(BNNE_Context ctx, int32_t token, uint32_t n_steps, int32_t* out_tokens) {
    forget_message();
    if (!ctx || !out_tokens || n_steps == 0)
        return BNNE_EINVAL;
    const BNNE_ModelInfo& info = ctx->model->info;
    if (info.task != BNNE_TASK_LLM)
        return complain(BNNE_ENOTSUP, "the model is not a language model");
    if (ctx->pos > ctx->params.n_ctx || n_steps > ctx->params.n_ctx - ctx->pos)
        return complain(BNNE_ERANGE, "%u steps do not fit the remaining context", n_steps);
    if (token < 0 || (uint32_t)token >= info.n_vocab)
        return complain(BNNE_ERANGE, "token %d is not in the vocabulary", token);
    CallStats call(*ctx);
    const uint32_t pos0 = ctx->pos;
    const BNNE_Status st = guarded([&] { ctx->decode_greedy(token, n_steps, out_tokens); });
    if (st != BNNE_OK)
        return st;
    ctx->pos = pos0 + n_steps;
    call.done(n_steps);
    return BNNE_OK;
}
