/*
 * bnn-engine.h -- the BNN inference engine API (v3), restated for the MI355X build.
 *
 * ABI-identical to the reference's bnn-sw-v2/bnn-engine.h:1-162 (same types, enumerator
 * values, struct field order and function signatures), so that a caller of the
 * reference engine (the bnn-infer-v2 CLI, bnn-infer-v2.c:163-522) links against
 * libbnn_engine.so unchanged.  The engine is the caller of the accelerator API
 * (bnn-accelerator.h): every linear layer runs through BNN_Execute(GEMV_F32).
 *
 * Handles: BNNE_Model is read-only after load (GGUF metadata, weights resident on
 * the device); BNNE_Context is mutable (device workspace, KV cache, statistics).
 * Lifetime: BNN_DeviceOpen -> BNNE_ModelLoad -> BNNE_ContextCreate -> ...
 *           -> BNNE_ContextFree -> BNNE_ModelFree -> BNN_DeviceClose.
 * Calls that reach one BNN_Device must be serialised by the caller.
 * Failed create calls set *out = NULL; every Free accepts NULL.
 */
#ifndef BNN_ENGINE_H
#define BNN_ENGINE_H

#include "bnn-accelerator.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BNNE_API_VERSION 3u
#define BNNE_MAX_RANK 4u

typedef struct bnne_model* BNNE_Model;
typedef struct bnne_context* BNNE_Context;

typedef enum {
    BNNE_OK = 0,
    BNNE_EINVAL = -1,
    BNNE_ENOMEM = -2,
    BNNE_ENOTSUP = -3,  /* unknown architecture, task mismatch, device too small */
    BNNE_ERANGE = -4,   /* capacity or context length exceeded */
    BNNE_EIO = -5,
    BNNE_EFORMAT = -6,  /* malformed GGUF or missing required field */
    BNNE_ECOMPUTE = -7  /* accelerator failure or non-finite values */
} BNNE_Status;

typedef enum {
    BNNE_TASK_CLASSIFY = 1, /* FP32 tensor -> FP32 logits[n_classes] */
    BNNE_TASK_LLM = 2       /* int32 tokens -> FP32 logits[n_vocab], with KV cache */
} BNNE_Task;

typedef struct {
    BNNE_Task task;
    const char* arch;  /* general.architecture, valid until BNNE_ModelFree */
    uint64_t load_ns;  /* model load time including the weight upload */

    /* TASK_CLASSIFY (0 otherwise) */
    uint32_t input_rank;
    uint32_t input_dims[BNNE_MAX_RANK];
    uint32_t input_size;
    uint32_t n_classes;

    /* TASK_LLM (0 / -1 otherwise) */
    uint32_t n_vocab;
    uint32_t n_ctx_train;
    int32_t bos_token;
    int32_t eos_token;
} BNNE_ModelInfo;

typedef struct {
    uint32_t n_ctx;    /* LLM KV-cache capacity in tokens; 0 = n_ctx_train */
    uint32_t n_batch;  /* most tokens or samples per call; 0 = default */
    int enable_stats;  /* default 1 */
} BNNE_ContextParams;

/* Monotonic wall-clock nanoseconds of successful Classify/Decode calls:
 * total_ns = quantize_ns + transfer_ns + execute_ns + host_ns. */
typedef struct {
    uint64_t calls, items;
    uint64_t total_ns, quantize_ns, transfer_ns, execute_ns, host_ns;
    uint64_t device_calls, bytes_written, bytes_read;
    uint64_t logical_macs, executed_macs;
} BNNE_Stats;

BNNE_Status BNNE_ModelLoad(BNN_Device device, const char* gguf_path, BNNE_Model* out_model);
void BNNE_ModelFree(BNNE_Model model);
BNNE_Status BNNE_ModelGetInfo(BNNE_Model model, BNNE_ModelInfo* out_info);

/* Text tokenizer entry points (TASK_LLM).  This build runs on token IDs; the
 * tokenizer calls return BNNE_ENOTSUP. */
BNNE_Status BNNE_Tokenize(BNNE_Model model, const char* text, int parse_special, int32_t* ids,
                          uint32_t capacity, uint32_t* out_count);
BNNE_Status BNNE_TokenPiece(BNNE_Model model, int32_t id, const char** out_bytes, size_t* out_len);
int BNNE_TokenIsEog(BNNE_Model model, int32_t id);

void BNNE_ContextParamsInit(BNNE_ContextParams* params);
BNNE_Status BNNE_ContextCreate(BNNE_Model model, const BNNE_ContextParams* params, BNNE_Context* out_ctx);
void BNNE_ContextFree(BNNE_Context ctx);

BNNE_Status BNNE_Classify(BNNE_Context ctx, const float* input, uint32_t n_samples, float* logits);
BNNE_Status BNNE_Decode(BNNE_Context ctx, const int32_t* tokens, uint32_t n_tokens, float* logits);
uint32_t BNNE_ContextPos(BNNE_Context ctx);
BNNE_Status BNNE_ContextTruncate(BNNE_Context ctx, uint32_t pos);

BNNE_Status BNNE_ContextGetStats(BNNE_Context ctx, BNNE_Stats* out_stats);
BNNE_Status BNNE_ContextResetStats(BNNE_Context ctx);

const char* BNNE_StatusString(BNNE_Status status);
const char* BNNE_LastError(void);

#ifdef __cplusplus
}
#endif
#endif
