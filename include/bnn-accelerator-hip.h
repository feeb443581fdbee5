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

/*
 * BNN_DeviceOpen accepts index 0 only, as the reference's soft backend does
 * (soft-bnn-accelerator.c:317-318); index 0 is the process's first visible HIP
 * device.  This opens HIP device `hip_ordinal` (0 .. hipGetDeviceCount() - 1) with
 * the same semantics, for hosts with several GPUs; BNN_ENOTSUP for any other value.
 */
BNN_Status BNNX_DeviceOpenOrdinal(uint32_t hip_ordinal, BNN_Device* out_device);

/* The hipStream_t (as void*) on which every transfer and kernel of the device runs. */
BNN_Status BNNX_DeviceStream(BNN_Device device, void** out_stream);

/*
 * enable != 0: every kernel launch of the device records its own start and end
 * into a HIP event pair (hipExtLaunchKernel), and the totals are reset; enable == 0:
 * stop.  Events are resolved at the next synchronisation of the call or of
 * BNNX_DeviceSynchronize (and every 1024 launches).  Profiled dispatches run a few
 * percent slower, so leave timing off outside measurement.
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

/*
 * BNN_Execute that allocates nothing.  No counterpart in the reference API: it is
 * for callers that cannot allocate memory at call time (tight serving loops,
 * harnesses that forbid hipMalloc).  Same checks, statuses and results as
 * BNN_Execute for every job.  A multi-row job keeps its rows' quantised forms (and,
 * for an output view that is not naturally aligned, its staged output rows) in one
 * fixed 8 MiB device array per GPU, created with the library's code object and held
 * until the process ends; the rows run in chunks that fit it, on the bit-plane dot
 * kernels.  A job whose single row does not fit the array is rejected with
 * BNN_ENOMEM (none does within the 8192-feature limits of BNN_DeviceGetCaps).
 * Single-row outputs are not mirrored in host memory.  Every call on one GPU, from
 * any BNN_Device handle opened on it, shares that array; the call is synchronous and
 * holds a per-GPU lock while it uses the array, so calls from several threads or
 * handles on one GPU run one after another (devices stay independent, as
 * bnn-accelerator.h requires of BNN_Device handles).
 */
BNN_Status BNNX_ExecuteNoAlloc(BNN_Device device, const BNN_Job* job);

/*
 * Prepared batches: the checks and job tables of BNNX_ExecuteBatch done once, for
 * callers that run the same set of jobs many times (a model's layers, token after
 * token) and keep their activations on the device.
 *
 * BNNX_BatchCreate checks the jobs exactly as BNNX_ExecuteBatch does (same
 * statuses) and builds the batch; the jobs' buffers and matrices must outlive it.
 * BNNX_BatchLaunch enqueues the batch on the device's stream (BNNX_DeviceStream)
 * and returns without waiting.  It fails with BNN_EINVAL once any matrix or buffer
 * of the device has been destroyed after the batch was built (rebuild it), and
 * with BNN_ENOTSUP when an FP32 job meets a host rounding mode other than
 * FE_TONEAREST.  Input values are checked by the device: a job that meets an
 * illegal input writes nothing, and the next BNNX_DeviceSynchronize reports it.
 * BNNX_DeviceSynchronize waits for everything enqueued on the device's stream and
 * returns BNN_ERANGE if any batch launched since the previous synchronisation met
 * an illegal input (BNN_EIO on a device error).  A device with live batches cannot
 * be closed (BNN_EBUSY).  Calls on one device must not overlap.
 */
typedef struct bnnx_batch* BNNX_Batch;
BNN_Status BNNX_BatchCreate(BNN_Device device, const BNN_Job* jobs, uint32_t count, BNNX_Batch* out_batch);
BNN_Status BNNX_BatchLaunch(BNNX_Batch batch);
void BNNX_BatchDestroy(BNNX_Batch batch);
/* What BNNX_BatchLaunch would return before enqueuing (BNN_OK, BNN_EINVAL for a
 * stale batch, BNN_ENOTSUP for the rounding mode), without launching. */
BNN_Status BNNX_BatchCheck(BNNX_Batch batch);
BNN_Status BNNX_DeviceSynchronize(BNN_Device device);

/*
 * Fused batches: GEMV_F32 jobs (rows = 1) that all read one input row, where the
 * row is produced on the device by a pre-operation and quantised inside the same
 * single kernel launch that computes the dots -- no prep launch, no host work per
 * launch.  For decode loops whose linear layers read normalised or gated
 * device-resident vectors.  With x_i = a_i + b_i (just a_i when b is NULL):
 *   BNNX_PRE_ROW      input = the jobs' input row (every job must name the same view)
 *   BNNX_PRE_RMSNORM  rms = sqrtf((sum over i in index order of x_i * x_i) / width + eps),
 *                     input_i = x_i / rms * gain_i; a_out (if not NULL) receives x
 *   BNNX_PRE_SILU_MUL input_i = a_i / (1 + expf(-a_i)) * b_i  (expf of the host C library)
 * every product, quotient and sum rounded to binary32 separately.  The produced row
 * then goes through exactly what GEMV_F32 does with an input row (check,
 * quantisation, dots, FP32 accumulation in group order): results are bit-identical
 * to computing the row on the host and calling BNN_Execute.
 * a, b, gain, a_out are device addresses on the batch's device (BNNX_BufferDevicePointer
 * or memory allocated there) of `width` floats, valid whenever the batch runs; a_out
 * may not overlap a or b, and no job output may overlap any of them (BNN_EINVAL).
 * Every job must be GEMV_F32 with rows = 1, K = width <= 6144 and an aligned output
 * view (else BNN_ENOTSUP or the BNN_Execute status).  A non-finite produced row is
 * an illegal input (nothing written; BNNX_DeviceSynchronize reports BNN_ERANGE); when
 * the RMSNORM divisor is not finite or zero, err_code is also stored to *err (if err
 * is not NULL and *err is 0).  Launch, check, destroy and synchronise as any
 * prepared batch.
 */
enum { BNNX_PRE_ROW = 0, BNNX_PRE_RMSNORM = 1, BNNX_PRE_SILU_MUL = 2 };
typedef struct {
    int32_t kind;      /* BNNX_PRE_* */
    uint32_t width;    /* values in the row (the matrices' K) */
    const float* a;    /* RMSNORM: x; SILU_MUL: gate */
    const float* b;    /* RMSNORM: residual added to x first (NULL: none); SILU_MUL: up */
    const float* gain; /* RMSNORM */
    float* a_out;      /* RMSNORM: receives x (NULL: not stored) */
    float eps;         /* RMSNORM */
    int32_t* err;      /* RMSNORM: error word (NULL: none) */
    int32_t err_code;
} BNNX_PreOp;
BNN_Status BNNX_BatchCreateFused(BNN_Device device, const BNN_Job* jobs, uint32_t count, const BNNX_PreOp* pre,
                                 BNNX_Batch* out_batch);

/* A fused batch with an operation on pairs of its outputs (post == NULL or kind
 * BNNX_POST_NONE: BNNX_BatchCreateFused).  BNNX_POST_SILU_MUL: the 2m jobs are m pairs
 * (job p, job m + p) whose outputs have equal length n_p; besides writing every job's
 * output as usual, the batch stores
 *   out[o_p + i] = y_p[i] / (1 + expf(-y_p[i])) * y_(m+p)[i],   o_p = n_0 + ... + n_(p-1)
 * (each operation rounded to binary32 separately, expf of the host C library): the
 * SiLU(gate) * up of the qwen3 step (qwen3.c:491-495) for gate/up jobs, as one launch.
 * `out` is a device address of n_0 + ... + n_(m-1) floats that may not overlap any
 * operand or job output.  Statuses as BNNX_BatchCreateFused, plus BNN_EINVAL for an
 * odd job count, pairs of unequal length or a NULL out. */
enum { BNNX_POST_NONE = 0, BNNX_POST_SILU_MUL = 1 };
typedef struct {
    int32_t kind; /* BNNX_POST_* */
    float* out;   /* SILU_MUL: the products */
} BNNX_PostOp;
BNN_Status BNNX_BatchCreateFusedPost(BNN_Device device, const BNN_Job* jobs, uint32_t count, const BNNX_PreOp* pre,
                                     const BNNX_PostOp* post, BNNX_Batch* out_batch);

/*
 * Chained batches: GEMM_F32 layers applied in turn to every row of an input view.
 * Layer i computes, for each row, exactly what a GEMM_F32 job computes (check,
 * quantisation, group dots, FP32 accumulation in group order); when post_scale is
 * set its outputs then become out_o = post_scale[o] * y_o, then out_o + post_bias[o]
 * (each rounded to binary32 on its own); with relu a negative result becomes +0; and
 * the row is layer i + 1's input.  The last layer's results go to the output view.
 * The results equal separate GEMM_F32 jobs with the mapping done on the host (the
 * bnn-mlp classifier's blocks, bnn-mlp.c:173-198), bit for bit, in one launch: a
 * workgroup carries a row through every layer and the rows between layers never
 * leave the chip.  layers[i].matrix has K_i inputs and N_i outputs with
 * K_(i+1) = N_i (else BNN_EINVAL); at most 16 layers, K_i and N_i <= 4096 and
 * rows <= 4096 (else BNN_ENOTSUP).  post_scale and post_bias are device addresses of
 * N_i floats (BNNX_BufferDevicePointer or memory allocated there), both NULL or both
 * set (else BNN_EINVAL), valid whenever the batch runs.  input is an F32 view of
 * rows x K_0 values, output an F32 view of rows x N_last values in another buffer
 * (BNN_EINVAL), both with 4-byte aligned rows (BNN_ENOTSUP).  A row that meets a
 * non-finite value at a layer's input writes nothing more, and the next
 * BNNX_DeviceSynchronize reports BNN_ERANGE.  Launch, check, destroy and synchronise as
 * any prepared batch.
 */
typedef struct {
    BNN_Matrix matrix;
    const float* post_scale; /* [N_i] or NULL */
    const float* post_bias;  /* [N_i] or NULL */
    int32_t relu;
} BNNX_ChainLayer;
BNN_Status BNNX_BatchCreateChain(BNN_Device device, const BNNX_ChainLayer* layers, uint32_t count,
                                 BNN_BufferView input, BNN_BufferView output, uint32_t rows,
                                 BNNX_Batch* out_batch);

/* Device address of a buffer's memory, for kernels a caller runs on the device's
 * stream between batch launches.  Valid until BNN_BufferFree. */
BNN_Status BNNX_BufferDevicePointer(BNN_Buffer buffer, void** out_pointer);

/* Name of the HIP device behind the handle (e.g. "AMD Instinct MI355X") and its
 * gfx architecture string; either pointer may be NULL. */
BNN_Status BNNX_DeviceName(BNN_Device device, char* name, size_t name_bytes, char* arch, size_t arch_bytes);

#ifdef __cplusplus
}
#endif

#endif
