// Internal interfaces of the BNN engine (the caller of the accelerator API).
//
// Mirrors the reference engine's internal contract (bnn-sw-v2/bnne-internal.h:1-99):
// an architecture registry, a model and a context, a GGUF reader, and the shared
// linear operator that drives BNN_Execute.  Host arithmetic is compiled with the
// reference's numeric flags (-fno-fast-math -ffp-contract=off) and written in the
// reference's operation order, so that logits are bit-identical for identical
// accelerator results.
#ifndef BNNE_ENGINE_INTERNAL_H
#define BNNE_ENGINE_INTERNAL_H

#include "bnn-engine.h"

#include <cstddef>
#include <cstdint>

namespace bnne {

constexpr uint32_t kGroup = 128;      // Q1_0 group size (linear.c:9)
constexpr uint32_t kMaxDims = 4;      // gguf.h:8
constexpr uint32_t kTypeF32 = 0, kTypeF16 = 1, kTypeQ1_0 = 41;

// ---------------------------------------------------------------- GGUF (v3 only)

struct GgufString {  // points into the mapping, not NUL-terminated
    const uint8_t* data;
    uint32_t length;
};

struct GgufTensor {
    GgufString name;
    uint32_t rank;
    uint64_t dims[kMaxDims];
    uint32_t type;
    uint64_t offset;
    uint64_t bytes;
};

// The metadata the engine reads (gguf.h:29-88); everything else is skipped.
struct Gguf {
    uint8_t* mapping;
    size_t mapping_bytes;
    uint64_t data_offset;
    uint32_t alignment;
    uint64_t tensor_count;
    GgufTensor* tensors;

    char architecture[32];
    uint64_t block_count, embedding_length, feed_forward_length;
    uint64_t head_count, head_count_kv, key_length, value_length, context_length;
    float rms_epsilon, rope_freq_base, rope_factor;
    uint64_t rope_original_context;
    char rope_scaling_type[16];

    uint64_t mlp_block_count, mlp_class_count, mlp_input_features, mlp_input_pixels;
    float mlp_input_mean, mlp_input_std;
    char (*mlp_activations)[16];  // by block index; "" where absent
    uint64_t mlp_activation_count;

    GgufString* tokens;  // tokenizer.ggml.tokens (strings point into the mapping)
    uint64_t token_count;
    uint32_t* token_types;  // tokenizer.ggml.token_type, may be absent
    uint64_t token_type_count;
    int has_eos, has_bos;
    uint32_t eos_token_id, bos_token_id;
};

BNNE_Status gguf_open(const char* path, Gguf** out);
void gguf_close(Gguf* g);
const GgufTensor* gguf_find(const Gguf* g, const char* name);
const uint8_t* gguf_data(const Gguf* g, const GgufTensor* t);

// ---------------------------------------------------------------- vocabulary

// Token pieces (the bytes each token stands for) and the end-of-generation ids.
struct Vocab {
    char* text;  // all pieces, each NUL-terminated
    uint32_t *off, *len;
    uint64_t count;
    uint32_t eog[8];
    uint32_t n_eog;
};

BNNE_Status vocab_build(const Gguf* g, Vocab** out);
void vocab_free(Vocab* v);

// ---------------------------------------------------------------- errors, time

BNNE_Status error(BNNE_Status status, const char* format, ...);
BNNE_Status accel_error(BNN_Status status, const char* operation);
void error_clear();
uint64_t now_ns();
float fp16_to_fp32(uint16_t half);

// ---------------------------------------------------------------- linear operator

struct LinearChunk {  // one BNN_Matrix per slice of at most max_out_features outputs
    uint32_t out_off, out_len;
    BNN_Matrix matrix;
};

struct Linear {
    uint32_t in, out;
    LinearChunk* chunks;
    uint32_t n_chunks;
};

BNNE_Status q1_0_read(const Gguf* g, const char* tensor, uint32_t in, uint32_t out, uint8_t** out_bits,
                      uint16_t** out_scales);
BNNE_Status linear_init(bnne_model* m, uint32_t in, uint32_t out, const uint8_t* bits, const uint16_t* scales,
                        Linear* l);
BNNE_Status linear_load(bnne_model* m, const Gguf* g, const char* tensor, Linear* l);
void linear_free(Linear* l);
BNNE_Status linear_forward(bnne_context* c, const Linear* l, const float* x, float* y);
BNNE_Status tensor_f32(const Gguf* g, const char* tensor, float** out, size_t* out_n);

// ---------------------------------------------------------------- architectures

struct Arch {
    const char* name;  // exact general.architecture
    BNNE_Task task;
    BNNE_Status (*load)(bnne_model* m, const Gguf* g, void** out_impl);
    void (*unload)(void* impl);
    BNNE_Status (*ctx_init)(bnne_context* c, void** out_state);
    void (*ctx_free)(void* state);
    BNNE_Status (*classify)(bnne_context* c, const float* in, uint32_t n, float* logits);
    BNNE_Status (*decode)(bnne_context* c, const int32_t* tokens, uint32_t n, float* logits);
    BNNE_Status (*truncate)(bnne_context* c, uint32_t pos);
};

extern const Arch kArchQwen3;
extern const Arch kArchBnnMlp;
// Decode path of a qwen3 context: 0 host call pattern, 1 device with fused
// batches (where the backend takes them), 2 device with prepared batches.
BNNE_Status qwen3_set_resident(bnne_context* c, int mode);
int qwen3_resident_mode(const bnne_context* c);
const Arch* arch_find(const char* name);

}  // namespace bnne

struct bnne_model {
    BNN_Device device;  // borrowed
    BNN_Caps caps;
    const bnne::Arch* arch;
    void* impl;
    bnne::Gguf* gguf;
    bnne::Vocab* vocab;  // LLM only
    BNNE_ModelInfo info;
    uint32_t max_in, max_out;  // widest linear input / chunk output, sizes the context buffers
};

struct bnne_context {
    bnne_model* model;
    BNNE_ContextParams params;
    void* state;
    BNN_Buffer in_buf;   // max_in F32 elements
    BNN_Buffer out_buf;  // max_out F32 elements
    uint32_t max_in, max_out;
    uint32_t pos;
    BNNE_Stats stats;
};

#endif
