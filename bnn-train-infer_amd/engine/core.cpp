// Shared pieces of the engine: failure reporting, clocks, binary16, the architecture
// table and the parts of a context every architecture shares.
#include "engine.hpp"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <ctime>

namespace bnne {
namespace {

thread_local char t_message[256];

void record(const char* format, va_list args) { std::vsnprintf(t_message, sizeof t_message, format, args); }

}  // namespace

void raise(BNNE_Status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    record(format, args);
    va_end(args);
    throw Failure{status};
}

BNNE_Status complain(BNNE_Status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    record(format, args);
    va_end(args);
    return status;
}

void forget_message() { t_message[0] = '\0'; }

const char* last_message() { return t_message; }

// The accelerator statuses a caller of the engine sees as engine statuses
// (bnn-accelerator.h:18-27 -> bnn-engine.h).
BNNE_Status engine_status(BNN_Status status) {
    switch (status) {
    case BNN_OK: return BNNE_OK;
    case BNN_ENOMEM: return BNNE_ENOMEM;
    case BNN_ENOTSUP: return BNNE_ENOTSUP;
    case BNN_ERANGE: return BNNE_ERANGE;
    case BNN_EIO:
    case BNN_ETIMEOUT: return BNNE_EIO;
    default: return BNNE_ECOMPUTE;
    }
}

BNNE_Status accel_status(BNN_Status status, const char* call) {
    if (status == BNN_OK)
        return BNNE_OK;
    return complain(engine_status(status), "%s failed: %s", call, BNN_StatusString(status));
}

void require(BNN_Status status, const char* call) {
    if (status != BNN_OK)
        throw Failure{accel_status(status, call)};
}

uint64_t clock_ns() {
    timespec ts;
    if (clock_gettime(CLOCK_MONOTONIC, &ts) != 0)
        return 0;
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

// binary16 -> binary32 is exact: normal numbers and the specials move their fields,
// subnormals m * 2^-24 are products of a small integer and a power of two.
float half_to_float(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1fu, mantissa = bits & 0x3ffu;
    float magnitude;
    if (exponent == 0) {
        magnitude = (float)mantissa * 0x1p-24f;
    } else {
        const uint32_t b = (exponent == 0x1f ? 0xffu : exponent + 112u) << 23 | mantissa << 13;
        std::memcpy(&magnitude, &b, 4);
    }
    uint32_t out;
    std::memcpy(&out, &magnitude, 4);
    out |= sign;
    float v;
    std::memcpy(&v, &out, 4);
    return v;
}

bnne_model* make_qwen3();
bnne_model* make_bnn_mlp();

const Architecture* find_architecture(std::string_view name) {
    static const Architecture table[] = {
        {"qwen3", BNNE_TASK_LLM, make_qwen3},
        {"bnn-mlp", BNNE_TASK_CLASSIFY, make_bnn_mlp},
    };
    for (const Architecture& a : table)
        if (name == a.name)
            return &a;
    return nullptr;
}

}  // namespace bnne

bnne_context::~bnne_context() {
    BNN_BufferFree(stage_in);
    BNN_BufferFree(stage_out);
}

void bnne_context::allocate_staging() {
    const size_t in_bytes = (size_t)stage_rows * (model->widest_in ? model->widest_in : 1u) * sizeof(float);
    const size_t out_bytes = (size_t)stage_rows * (model->widest_shard ? model->widest_shard : 1u) * sizeof(float);
    bnne::require(BNN_BufferAlloc(model->device, in_bytes, &stage_in), "BNN_BufferAlloc (layer input)");
    bnne::require(BNN_BufferAlloc(model->device, out_bytes, &stage_out), "BNN_BufferAlloc (layer output)");
}

void bnne_context::select_path(int path) {
    if (path < 0 || path > 2)
        bnne::raise(BNNE_EINVAL, "path %d (0 host, 1 device with fused batches, 2 device)", path);
    if (path != 0)
        bnne::raise(BNNE_ENOTSUP, "only qwen3 and bnn-mlp contexts have a device path");
}

void bnne_context::classify(const float*, uint32_t, float*) {
    bnne::raise(BNNE_ENOTSUP, "this model does not classify");
}

void bnne_context::decode(const int32_t*, uint32_t, float*) {
    bnne::raise(BNNE_ENOTSUP, "this model does not decode tokens");
}

void bnne_context::decode_greedy(int32_t token, uint32_t n, int32_t* out) {
    std::vector<float> logits(model->info.n_vocab);
    const uint32_t pos0 = pos;
    struct Restore {
        bnne_context& c;
        uint32_t pos0;
        ~Restore() { c.pos = pos0; }
    } restore{*this, pos0};
    for (uint32_t i = 0; i < n; ++i) {
        logits_checked = false;
        decode(&token, 1, logits.data());
        uint32_t best = 0;
        for (uint32_t v = 0; v < (uint32_t)logits.size(); ++v) {
            if (!std::isfinite(logits[v]))
                bnne::raise(BNNE_ECOMPUTE, "the logits hold a NaN or infinity");
            if (logits[v] > logits[best])
                best = v;
        }
        token = (int32_t)best;
        out[i] = token;
        ++pos;
    }
}

void bnne_context::rewind(uint32_t) {}
