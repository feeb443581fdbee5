/*
 * Extensions of the engine API (bnn-engine.h) in this build; no counterpart in the
 * reference engine.
 *
 * A Qwen3 context runs each decode step on the device by default: activations,
 * the KV cache and every step of the model stay in HBM, the linear layers run as
 * prepared batches of the accelerator (BNNX_BatchCreate), and the host waits once
 * per BNNE_Decode call.  The other path is the reference's call pattern: host
 * arithmetic, one synchronous BNN_Execute per linear layer chunk, the activations
 * copied across for every call.  Both compute the same logits bit for bit.
 * Statistics of the device path: execute_ns is the wait for the device,
 * transfer_ns the logits copy, device_calls the linear jobs run.
 */
#ifndef BNN_ENGINE_HIP_H
#define BNN_ENGINE_HIP_H

#include "bnn-engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Selects the device path (enable != 0) or the host call pattern for a qwen3
 * context.  Only before its first token (BNNE_EINVAL otherwise); BNNE_ENOTSUP for
 * other architectures or shapes the device path does not take. */
BNNE_Status BNNEX_ContextSetResident(BNNE_Context ctx, int enable);

/* 1 when the context runs the device path. */
int BNNEX_ContextIsResident(BNNE_Context ctx);

#ifdef __cplusplus
}
#endif
#endif
