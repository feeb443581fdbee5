// Device-resident bnn-mlp classification: a classify call's rows go to the device once,
// the blocks run there, and only the last block's outputs come back: one host wait per
// chunk of rows instead of a write, a synchronous BNN_Execute and a read per block.  The
// blocks run as one chained batch of the backend (BNNX_BatchCreateChain: each block's
// GEMM_F32 and its post_scale * y + post_bias and ReLU, one launch for all of them), or,
// for blocks wider than a chain takes, as one prepared batch of GEMM_F32 jobs per block
// (each row of a job is that sample's GEMV_F32, as SignLinear::apply_rows computes it)
// followed by this engine's post-operation kernel (each operation rounded on its own as
// mlp.cpp's host loop does).  The logits equal the host call pattern's bit for bit.
#ifndef BNNE_MLP_DEVICE_H
#define BNNE_MLP_DEVICE_H

#include "engine.hpp"

namespace bnne {

struct MlpDeviceBlock {
    const SignLinear* weight;
    const float* post_scale;  // [weight->out()]
    const float* post_bias;   // [weight->out()]
    bool relu;
};

struct MlpDevice;

// State for chunks of up to `rows` rows.  BNNE_ENOTSUP when the backend has no device
// stream (BNNX_DeviceStream) or a block's weights are split over several shards.
BNNE_Status mlp_device_create(bnne_context* c, const MlpDeviceBlock* blocks, uint32_t count, uint32_t inputs,
                              uint32_t rows, MlpDevice** out);
// One chunk: input rows x inputs floats in, rows x classes logits out (rows <= the rows
// given at creation).  Enqueues everything on the device's stream and waits once.
BNNE_Status mlp_device_classify(bnne_context* c, MlpDevice* d, const float* input, uint32_t rows, float* logits);
void mlp_device_free(MlpDevice* d);

}  // namespace bnne

#endif
