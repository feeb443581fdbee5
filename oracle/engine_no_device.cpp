// Test infrastructure: the device-path entry points (engine/resident.h) for a build of
// the engine's host code without HIP, linked to the CPU oracle backend (oracle/bnn_cpu.c)
// so that the engine's host step runs -- and runs under AddressSanitizer and
// UndefinedBehaviorSanitizer -- on a machine without a GPU.  Every context then
// decodes on the host step and classifies with the host call pattern.  Not part of the
// product.
#include "mlp_device.h"
#include "resident.h"

namespace bnne {

struct Resident {};

BNNE_Status resident_create(bnne_context*, const ResidentModel&, bool, Resident** out) {
    *out = nullptr;
    return complain(BNNE_ENOTSUP, "this build of the engine has no device path");
}

bool resident_fused(const Resident*) { return false; }

BNNE_Status resident_step(bnne_context*, Resident*, const int32_t*, uint32_t, uint32_t, float*) {
    return complain(BNNE_ENOTSUP, "this build of the engine has no device path");
}

BNNE_Status resident_greedy(bnne_context*, Resident*, int32_t, uint32_t, uint32_t, int32_t*) {
    return complain(BNNE_ENOTSUP, "this build of the engine has no device path");
}

void resident_free(Resident*) {}

struct MlpDevice {};

BNNE_Status mlp_device_create(bnne_context*, const MlpDeviceBlock*, uint32_t, uint32_t, uint32_t, MlpDevice** out) {
    *out = nullptr;
    return complain(BNNE_ENOTSUP, "this build of the engine has no device path");
}

BNNE_Status mlp_device_classify(bnne_context*, MlpDevice*, const float*, uint32_t, float*) {
    return complain(BNNE_ENOTSUP, "this build of the engine has no device path");
}

void mlp_device_free(MlpDevice*) {}

}  // namespace bnne
