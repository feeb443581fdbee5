// Device-resident Qwen3 decode: the whole token step runs on the GPU, on the
// accelerator device's stream.  Linear layers are fused BNNX batches of the HIP
// backend (q/k/v together, gate/up together, the lm_head chunks together), whose
// single launch also produces the layer's input row: the RMSNorm with the
// residual add, the attention output, or SiLU(gate)*up.  The q/k norms, RoPE, the
// KV cache and attention are one kernel of this engine.  Where the backend does
// not take fused batches (wider layers), prepared batches run beside this
// engine's RMSNorm and SiLU kernels instead.  Every kernel keeps the host step's
// operation order (each
// output's sums run sequentially in one lane, no FMA contraction, IEEE division
// and square root, and an expf that returns what the host C library's expf
// returns), so the logits are the ones the host step computes.
#ifndef BNNE_RESIDENT_H
#define BNNE_RESIDENT_H

#include "engine.hpp"

namespace bnne {

struct ResidentModel {  // host views of the model, used once to build the device state
    uint32_t C, H, Hk, HD, FF, L, V, kv_dim, n_ctx;
    float eps;
    const float* const* attn_norm;  // [L][C]
    const float* const* ffn_norm;   // [L][C]
    const float* const* q_norm;     // [L][HD]
    const float* const* k_norm;     // [L][HD]
    const float* final_norm;        // [C]
    const uint8_t* emb_bits;        // [V][C/8]
    const uint16_t* emb_scales;     // [V][C/128]
    const float* rope_cos;          // [n_ctx][HD/2]
    const float* rope_sin;
    const SignLinear* const* wq;  // [L] each
    const SignLinear* const* wk;
    const SignLinear* const* wv;
    const SignLinear* const* wo;
    const SignLinear* const* gate;
    const SignLinear* const* up;
    const SignLinear* const* down;
    const SignLinear* lm_head;
};

struct Resident;

// fused: run the linear layers as fused batches where the backend takes them
// (BNNX_BatchCreateFused), else as prepared batches with this engine's norm and
// SiLU kernels.
BNNE_Status resident_create(bnne_context* c, const ResidentModel& m, bool fused, Resident** out);
// Whether the step runs fused batches.
bool resident_fused(const Resident* r);
// One decode step of `token` at position `pos`; logits (host, V floats) only when
// non-null.  Enqueues everything, waits once.
BNNE_Status resident_step(bnne_context* c, Resident* r, const int32_t* tokens, uint32_t n, uint32_t pos0,
                          float* logits);
// Greedy decoding of n tokens on the device, as n calls of resident_step with logits,
// each followed by the caller's argmax (bnn-infer-v2.c:48-54) fed back as the next
// token: `token` at pos0, then each argmax; out_tokens[i] the argmax after step i.  The
// host waits once, after the last step.
BNNE_Status resident_greedy(bnne_context* c, Resident* r, int32_t token, uint32_t n, uint32_t pos0,
                            int32_t* out_tokens);
void resident_free(Resident* r);

}  // namespace bnne

#endif
