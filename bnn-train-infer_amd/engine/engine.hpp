// Internal interfaces of the model engine behind include/bnn-engine.h.
//
// Structure: a GGUF file is indexed once (GgufFile) and each architecture reads its
// own metadata keys and tensors from it; Q1_0 tensors become SignLinear layers,
// which own their accelerator matrices (one per shard of at most max_out_features
// outputs) and run the accelerator's call pattern; bnne_model / bnne_context (the
// opaque handles of the C API) are base classes that each architecture extends.
// Internal code reports a failure by throwing `Failure` after recording a message;
// every exported function converts it back to a status code at the C boundary.
//
// Host arithmetic is compiled with -fno-fast-math -ffp-contract=off: every float
// operation rounds on its own, so host steps that keep the reference's operation
// order give bit-identical results.
#pragma once

#include "bnn-engine.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <new>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace bnne {

constexpr uint32_t kGroup = 128;  // weights per Q1_0 block (and per accelerator scale group)

// ------------------------------------------------------------------------ failures

struct Failure {
    BNNE_Status status;
};

// Records the message (BNNE_LastError) and throws Failure{status}.
[[noreturn]] void raise(BNNE_Status status, const char* format, ...) __attribute__((format(printf, 2, 3)));
void forget_message();
const char* last_message();
// The engine status a caller sees for an accelerator status.
BNNE_Status engine_status(BNN_Status status);
// Throws unless status is BNN_OK; `call` names the accelerator call in the message.
void require(BNN_Status status, const char* call);
// The same two for code that returns statuses (the device path): record the message
// and return the status instead of throwing.
BNNE_Status complain(BNNE_Status status, const char* format, ...) __attribute__((format(printf, 2, 3)));
BNNE_Status accel_status(BNN_Status status, const char* call);

// Runs body() and turns what it throws into a status: the C boundary of the engine.
template <class Body>
BNNE_Status guarded(Body&& body) noexcept {
    try {
        body();
        return BNNE_OK;
    } catch (const Failure& f) {
        return f.status;
    } catch (const std::bad_alloc&) {
        try {
            raise(BNNE_ENOMEM, "out of host memory");
        } catch (const Failure& f) {
            return f.status;
        }
    } catch (...) {
        return BNNE_ECOMPUTE;
    }
}

// ------------------------------------------------------------------------ time

uint64_t clock_ns();

// Adds the time from its construction to its destruction to *sink (nothing when the
// sink is null, i.e. statistics are off).
class Span {
public:
    explicit Span(uint64_t* sink) : sink_(sink), start_(sink ? clock_ns() : 0) {}
    ~Span() {
        if (sink_)
            *sink_ += clock_ns() - start_;
    }
    Span(const Span&) = delete;
    Span& operator=(const Span&) = delete;

private:
    uint64_t* sink_;
    uint64_t start_;
};

// ------------------------------------------------------------------------ binary16

float half_to_float(uint16_t bits);  // exact
inline bool half_is_finite(uint16_t bits) { return (bits & 0x7c00u) != 0x7c00u; }

// ------------------------------------------------------------------------ GGUF

enum TensorType : uint32_t { kF32 = 0, kF16 = 1, kQ1_0 = 41 };

struct TensorRef {
    std::string_view name;
    uint32_t type;
    uint32_t rank;
    uint64_t dims[4];
    const uint8_t* data;  // inside the mapping
    uint64_t bytes;
};

// A GGUF v3 file, memory-mapped and indexed.  Metadata values are decoded when asked
// for; the keys this engine knows are checked for a usable type when the file opens.
class GgufFile {
public:
    static std::unique_ptr<GgufFile> open(const char* path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const std::string& architecture() const { return architecture_; }
    const TensorRef* tensor(std::string_view name) const;

    std::optional<uint64_t> integer(std::string_view key) const;  // any integer type, signed ones sign-extended
    std::optional<float> real(std::string_view key) const;        // F32 or F64 (narrowed), finite
    std::optional<std::string_view> text(std::string_view key) const;
    std::vector<std::string_view> texts(std::string_view key) const;  // a string array; empty when absent
    std::vector<uint32_t> words(std::string_view key) const;          // an I32/U32 array; empty when absent
    bool has(std::string_view key) const;

    struct Entry {
        std::string_view key;
        uint32_t type;
        const uint8_t* value;  // first byte of the value in the mapping
        const uint8_t* end;    // one past its last byte
    };

private:
    GgufFile() = default;
    const Entry* entry(std::string_view key) const;

    void* map_ = nullptr;
    size_t map_bytes_ = 0;
    std::vector<Entry> entries_;  // in file order; a later repeat of a key wins
    std::vector<TensorRef> tensors_;
    std::string architecture_;
};

// The values of an F32 or F16 tensor with exactly `count` elements, all finite.
std::vector<float> read_floats(const GgufFile& file, std::string_view name, size_t count);

// ------------------------------------------------------------------------ Q1_0 layers

// A Q1_0 tensor [in, out] split into the accelerator's operands: bits[out][in / 8]
// (bit k % 8 of byte k / 8 is the sign of weight k, 1 = +1) and fp16 scales
// [out][in / 128].
struct SignWeights {
    uint32_t in = 0, out = 0;
    std::vector<uint8_t> bits;
    std::vector<uint16_t> scales;
};
// Any shape; `in` must be a multiple of 128 and every scale finite.
SignWeights read_sign_weights(const GgufFile& file, std::string_view name);
// The same, with the shape the architecture expects.
SignWeights read_sign_weights(const GgufFile& file, std::string_view name, uint32_t in, uint32_t out);

struct Shard {
    uint32_t first, count;  // outputs [first, first + count) of the layer
    BNN_Matrix matrix;
};

}  // namespace bnne

struct bnne_model;
struct bnne_context;

namespace bnne {

// A linear layer y = W x resident on the accelerator as shards of at most the device's
// max_out_features outputs.  apply() is the accelerator's call pattern: the input row
// written once to the context's input buffer, then per shard one synchronous
// BNN_Execute(GEMV_F32, rows = 1) and one BNN_BufferRead of its outputs.  apply_rows()
// takes up to the context's stage_rows rows at once: one write of all of them, then per
// shard one GEMM_F32 job over every row (the API computes each row of a GEMM_F32 exactly
// as a GEMV_F32 of that row) and one read.
class SignLinear {
public:
    SignLinear() = default;
    ~SignLinear();
    SignLinear(const SignLinear&) = delete;
    SignLinear& operator=(const SignLinear&) = delete;

    void upload(bnne_model& model, const SignWeights& w);
    void apply(bnne_context& ctx, const float* x, float* y) const;
    // x: rows x in() floats, y: rows x out() floats, rows <= ctx.stage_rows
    void apply_rows(bnne_context& ctx, const float* x, uint32_t rows, float* y) const;

    uint32_t in() const { return in_; }
    uint32_t out() const { return out_; }
    const std::vector<Shard>& shards() const { return shards_; }

private:
    uint32_t in_ = 0, out_ = 0;
    std::vector<Shard> shards_;
};

// ------------------------------------------------------------------------ vocabulary

// Token pieces (the bytes a token stands for) and end-of-generation ids.
class Vocab {
public:
    explicit Vocab(const GgufFile& file);
    uint32_t size() const { return (uint32_t)offset_.size(); }
    std::string_view piece(uint32_t id) const;  // NUL-terminated in storage
    bool ends_generation(uint32_t id) const;

private:
    std::string text_;
    std::vector<uint32_t> offset_, length_;
    std::vector<uint32_t> eog_;
};

// ------------------------------------------------------------------------ architectures

struct Architecture {
    const char* name;  // general.architecture
    BNNE_Task task;
    bnne_model* (*make)();
};
const Architecture* find_architecture(std::string_view name);

}  // namespace bnne

// The opaque handles of bnn-engine.h.  An architecture derives from both.
struct bnne_model {
    BNN_Device device = nullptr;  // borrowed
    BNN_Caps caps{};
    BNNE_ModelInfo info{};
    const bnne::Architecture* arch = nullptr;
    std::unique_ptr<bnne::GgufFile> file;
    std::unique_ptr<bnne::Vocab> vocab;  // language models
    // widest layer input and widest shard output: the sizes of a context's staging buffers
    uint32_t widest_in = 0, widest_shard = 0;

    virtual ~bnne_model() = default;
    // Reads the architecture's hyperparameters and weights from `file` (already open);
    // fills the task fields of `info`.
    virtual void load() = 0;
    // A context of this model with `params` completed by the caller.
    virtual bnne_context* new_context(const BNNE_ContextParams& params) = 0;
};

struct bnne_context {
    bnne_model* model;
    BNNE_ContextParams params;
    uint32_t pos = 0;
    BNNE_Stats stats{};
    uint32_t stage_rows = 1;         // rows the staging buffers hold (set before allocate_staging)
    BNN_Buffer stage_in = nullptr;   // stage_rows x widest_in floats: the input rows of SignLinear
    BNN_Buffer stage_out = nullptr;  // stage_rows x widest_shard floats: one shard's outputs
    bool logits_checked = false;     // set by a decode that verified its logits are finite

    bnne_context(bnne_model& m, const BNNE_ContextParams& p) : model(&m), params(p) {}
    virtual ~bnne_context();
    // Allocates the staging buffers (after the architecture's own state).
    void allocate_staging();

    virtual void classify(const float* input, uint32_t n, float* logits);
    virtual void decode(const int32_t* tokens, uint32_t n, float* logits);
    // n decode steps from `token` at pos, each next token the previous step's argmax
    // (bnn-infer-v2.c:48-54), out[i] the argmax after step i; leaves pos as it found it
    virtual void decode_greedy(int32_t token, uint32_t n, int32_t* out);
    virtual void rewind(uint32_t pos);
    // The execution path (BNNEX_ContextSetResident): 0 the reference's host call pattern,
    // 1 a device path with fused batches, 2 a device path with prepared batches.  Contexts
    // without a device path stay on 0 and refuse the others (BNNE_ENOTSUP).
    virtual int path() const { return 0; }
    virtual void select_path(int path);

    // The statistics counter `field`, or null when statistics are off.
    uint64_t* counter(uint64_t BNNE_Stats::*field) { return params.enable_stats ? &(stats.*field) : nullptr; }
    void count(uint64_t BNNE_Stats::*field, uint64_t n) {
        if (params.enable_stats)
            stats.*field += n;
    }
};
