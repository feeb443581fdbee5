/*
 * Extensions of the engine API (bnn-engine.h) in this build; no counterpart in the
 * reference engine.
 *
 * A Qwen3 context runs each decode step on the device by default: activations,
 * the KV cache and every step of the model stay in HBM, the linear layers run as
 * fused batches of the accelerator (BNNX_BatchCreateFused: each layer's input
 * row -- RMSNorm with the residual add, attention output, SiLU(gate)*up -- is
 * produced inside the layer's one launch) or, for layers wider than those take,
 * prepared batches (BNNX_BatchCreate), and the host waits once per BNNE_Decode
 * call.  The other path is the reference's call pattern: host
 * arithmetic, one synchronous BNN_Execute per linear layer chunk, the activations
 * copied across for every call.  Both compute the same logits bit for bit.
 * Statistics of the device path: execute_ns is the wait for the device,
 * transfer_ns the logits copy, device_calls the linear jobs run.
 *
 * A bnn-mlp context classifies on the device by default as well: a call's rows
 * are copied to the device once per chunk, every block runs there as a prepared
 * batch of GEMM_F32 jobs followed by its post_scale / post_bias / ReLU, and only
 * the logits come back (one host wait per chunk).  The other path is the
 * reference's call pattern: per block one write, the GEMM_F32 jobs and one read,
 * the post-operation on the host.  Both give the same logits bit for bit.  Its
 * device-path statistics: transfer_ns the two copies, execute_ns the wait.
 */
#ifndef BNN_ENGINE_HIP_H
#define BNN_ENGINE_HIP_H

#include "bnn-engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Selects the path of a context: 0 the host call pattern, 1 the device path with
 * fused batches where the backend takes them (the default), 2 the device path with
 * prepared batches only.  qwen3: only before its first token (BNNE_EINVAL
 * otherwise).  bnn-mlp: between any two calls; its device path has no fused form,
 * so 1 and 2 both select it.  BNNE_EINVAL for other values; BNNE_ENOTSUP for other
 * architectures and for shapes the device path does not take (a bnn-mlp block
 * split over several shards). */
BNNE_Status BNNEX_ContextSetResident(BNNE_Context ctx, int enable);

/* The path in effect: 0 host, 1 device with fused batches, 2 device with
 * prepared batches (a bnn-mlp context's device path). */
int BNNEX_ContextIsResident(BNNE_Context ctx);

/* Greedy decoding: n_steps BNNE_Decode calls of one token each, the first of `token`,
 * every later one of the argmax of the previous logits (the first index of the largest
 * value, as bnn-infer-v2.c:48-54 picks it); out_tokens[i] receives the argmax after
 * step i.  The same tokens as that loop; on the device path every step, its argmax
 * included, stays on the device and the host waits once.  No EOG test: the caller
 * truncates at the first end-of-generation token (BNNE_ContextTruncate).  On success
 * the position advances by n_steps; on an error (BNNE_ECOMPUTE for non-finite logits
 * or norms, as BNNE_Decode) it is left where it was and out_tokens is undefined. */
BNNE_Status BNNEX_DecodeGreedy(BNNE_Context ctx, int32_t token, uint32_t n_steps, int32_t* out_tokens);

#ifdef __cplusplus
}
#endif
#endif
