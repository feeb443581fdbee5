/*
 * Extensions exported by the HIP backend (libbnn_hip.so) beside the eleven
 * BNN_* entry points of bnn-accelerator.h.  None of them has a counterpart in
 * the reference API (bnn-accelerator/bnn-accelerator.h); a caller written for
 * the reference never needs them.  They exist for measurement and for callers
 * that issue many independent jobs at once.
 */
#ifndef BNN_ACCELERATOR_HIP_H
#define BNN_ACCELERATOR_HIP_H

#include "bnn-accelerator.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel kinds reported by BNNX_KernelTimingRead. */
enum {
    BNNX_KERNEL_PREP = 0,    /* row validation + quantisation + bit planes */
    BNNX_KERNEL_DOT = 1,     /* group dots + FP32 scale accumulation (the dominant kernel) */
    BNNX_KERNEL_SCATTER = 2, /* copy into odd (unaligned) output views */
    BNNX_KERNEL_GEMM = 3     /* multi-row jobs on the matrix cores */
};

/* The hipStream_t (as void*) on which every transfer and kernel of the device runs. */
BNN_Status BNNX_DeviceStream(BNN_Device device, void** out_stream);

/*
 * enable != 0: start recording HIP events around every kernel launch of the
 * device and reset the totals; enable == 0: stop.  Timing adds one event pair
 * and one synchronisation per launch, so leave it off outside measurement.
 */
BNN_Status BNNX_KernelTiming(BNN_Device device, int enable);

/* Total device time (ms) and launch count recorded for one kernel kind. */
BNN_Status BNNX_KernelTimingRead(BNN_Device device, uint32_t kind, double* total_ms, uint64_t* launches);

/*
 * Runs `count` independent jobs as one unit: one prep launch for every
 * activation row of every job, then one group-dot launch for every output tile.
 * Each job is checked exactly as BNN_Execute checks it, in order; the first
 * failing job's status is returned and nothing runs.  Input values of all jobs
 * are checked before any output is written: an illegal value anywhere gives
 * BNN_ERANGE and leaves every output unchanged.  Because the jobs run
 * concurrently, no job's output buffer may be any job's input buffer, and
 * outputs sharing a buffer may not overlap (BNN_EINVAL).  Only naturally
 * aligned views (4-byte F32, 2-byte I16 offsets and strides) and rows <= 4096
 * per job are accepted (otherwise BNN_ENOTSUP; BNN_Execute takes any view).
 * Synchronous, like BNN_Execute.
 */
BNN_Status BNNX_ExecuteBatch(BNN_Device device, const BNN_Job* jobs, uint32_t count);

/* Name of the HIP device behind the handle (e.g. "AMD Instinct MI355X") and its
 * gfx architecture string; either pointer may be NULL. */
BNN_Status BNNX_DeviceName(BNN_Device device, char* name, size_t name_bytes, char* arch, size_t arch_bytes);

#ifdef __cplusplus
}
#endif

#endif
