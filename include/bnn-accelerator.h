/*
 * BNN accelerator API, version 2 -- the drop-in C boundary of this backend.
 *
 * This header restates, in this project's own words, the C ABI declared by the
 * reference at bnn-accelerator/bnn-accelerator.h.  Every type, enumerator value,
 * struct member (order, type and therefore layout) and function signature is
 * kept identical, so that a caller compiled against the reference header
 * (bnn-sw-v2/linear.c, engine.c, bnn-infer-v2.c, tests/accelerator) links
 * unchanged against libbnn_hip.so.  The layout identity is checked by
 * oracle/abi_probe.c, which is compiled once against this header and once
 * against the reference header.
 *
 * Citations are "file:line" relative to the reference tree.
 */
#ifndef BNN_ACCELERATOR_H
#define BNN_ACCELERATOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bnn-accelerator.h:12.  Callers and backends are rebuilt together per version. */
#define BNN_API_VERSION 2u

/* bnn-accelerator.h:14-16.  Opaque handles; each backend defines the structs. */
typedef struct bnn_accel_device* BNN_Device;
typedef struct bnn_accel_matrix* BNN_Matrix;
typedef struct bnn_accel_buffer* BNN_Buffer;

/* bnn-accelerator.h:18-27 */
typedef enum {
    BNN_OK = 0,
    BNN_EINVAL = -1,   /* bad argument, handle, type or ownership */
    BNN_ENOMEM = -2,   /* allocation failed; outputs untouched */
    BNN_ENOTSUP = -3,  /* operation / configuration not offered by this backend */
    BNN_ERANGE = -4,   /* out-of-range view, size overflow or illegal input value */
    BNN_EBUSY = -5,    /* device still owns matrices or buffers */
    BNN_EIO = -6,      /* device failure; output may be partially written */
    BNN_ETIMEOUT = -7  /* device timeout; output may be partially written */
} BNN_Status;

/*
 * bnn-accelerator.h:29-41.
 *   GEMV / GEMM      : I8 activations -> per-group integer dots -> F32 sum of scale*dot.
 *   DOT_GROUPS       : I8 activations -> exact per-group I16 dots, no weight scale.
 *   GEMV_F32/GEMM_F32: F32 activations, quantised to I8 per full row by the backend,
 *                      then as GEMV/GEMM, then multiplied by the row scale.
 */
typedef enum {
    BNN_OP_GEMV = 1,
    BNN_OP_GEMM = 2,
    BNN_OP_DOT_GROUPS = 3,
    BNN_OP_GEMV_F32 = 4,
    BNN_OP_GEMM_F32 = 5
} BNN_Operation;

/* bnn-accelerator.h:43 */
typedef enum { BNN_TYPE_I8 = 1, BNN_TYPE_F32 = 2, BNN_TYPE_I16 = 3 } BNN_Type;

/* bnn-accelerator.h:45-52.  Capability bits; not the same numbers as BNN_Operation. */
typedef enum {
    BNN_CAP_GEMV = 1u << 0,
    BNN_CAP_GEMM = 1u << 1,
    BNN_CAP_DOT_GROUPS = 1u << 2,
    BNN_CAP_GEMV_F32 = 1u << 3,
    BNN_CAP_GEMM_F32 = 1u << 4
} BNN_OperationCaps;

/*
 * bnn-accelerator.h:54-69.  Logical limits of the whole backend (inclusive).
 * group_size is the one weight-scale group size the backend accepts.
 */
typedef struct {
    uint32_t api_version;
    uint32_t max_in_features;
    uint32_t max_out_features;
    uint32_t max_rows;
    uint32_t group_size;
    uint32_t supported_ops;
} BNN_Caps;

/*
 * bnn-accelerator.h:71-102.  Read-only W1 matrix, logical shape [out][in].
 * weight_bits: row-major, in/8 bytes per row; weight k of row o is bit (k & 7)
 *   of byte weight_bits[o * (in / 8) + (k >> 3)]; bit 1 means +1, bit 0 means -1.
 * scale_fp16: row-major [out][in / group_size] host-order binary16 bit patterns;
 *   every finite value is legal (negative, signed zero, subnormal); NaN/Inf are not.
 * All sizes non-zero; group_size a multiple of 8 in [8, 256] dividing in;
 * weight_bytes / scale_count must equal the sizes exactly; both arrays required.
 * After a successful MatrixCreate the caller may modify or free both arrays.
 */
typedef struct {
    uint32_t in_features;
    uint32_t out_features;
    uint32_t group_size;

    const uint8_t* weight_bits;
    size_t weight_bytes;

    const uint16_t* scale_fp16;
    size_t scale_count;
} BNN_MatrixDesc;

/*
 * bnn-accelerator.h:104-119.  Borrowed, stateless view of an untyped buffer.
 * offset and row_stride are bytes and may be unaligned; row_stride 0 means
 * tightly packed, otherwise it must be at least one logical row.  Every logical
 * row must lie inside the buffer and no size computation may overflow.
 */
typedef struct {
    BNN_Buffer buffer;
    BNN_Type type;
    size_t offset;
    size_t row_stride;
} BNN_BufferView;

/*
 * bnn-accelerator.h:121-161.  One job.  M = rows, K = in_features,
 * N = out_features, G = group_size, groups = K / G; all layouts row-major.
 *
 *   operation    input         output
 *   GEMV         [1][K] I8     [1][N] F32
 *   GEMM         [M][K] I8     [M][N] F32
 *   DOT_GROUPS   [M][K] I8     [M][N][groups] I16
 *   GEMV_F32     [1][K] F32    [1][N] F32
 *   GEMM_F32     [M][K] F32    [M][N] F32
 *
 * rows != 0; both GEMV operations need rows == 1.  Logical I8 inputs lie in
 * [-127, 127] (-128 is rejected).  D[m][n][g] = sum over group g of Q[m][k]*W[n][k]
 * is exact (|D| <= 32512 for G <= 256) and never wraps or saturates.
 * Z[m][n] = sum_g F32(scale[n][g]) * D[m][n][g]; I8 GEMV/GEMM return Z.
 * F32 operations quantise each full logical row: a = max|X|; NaN/Inf -> ERANGE;
 * s = 1 if a == 0 else F32(a / 127), replaced by the smallest positive subnormal
 * if that division rounds to zero; Q = clamp(round-half-away(F32(X / s)), -127, 127);
 * Y = F32(Z * s).  Internal K tiling must reuse the full-row quantisation.
 * Matrix and both buffers belong to the executing device; input and output
 * must be different buffer handles even when the views do not overlap.
 */
typedef struct {
    BNN_Operation operation;
    BNN_Matrix matrix;
    BNN_BufferView input;
    BNN_BufferView output;
    uint32_t rows;
} BNN_Job;

/*
 * bnn-accelerator.h:163-207.  Resources and concurrency:
 * - a failed create sets the output handle to NULL;
 * - calls on one device are serialised by the caller; devices are independent;
 *   transfers and Execute are synchronous;
 * - matrices and buffers are released before their device; Destroy/Free take NULL.
 */
BNN_Status BNN_DeviceOpen(uint32_t device_index, BNN_Device* out_device);
/* Returns BNN_EBUSY, leaving the device open, while matrices or buffers remain. */
BNN_Status BNN_DeviceClose(BNN_Device device);
BNN_Status BNN_DeviceGetCaps(BNN_Device device, BNN_Caps* out_caps);

BNN_Status BNN_MatrixCreate(BNN_Device device, const BNN_MatrixDesc* desc, BNN_Matrix* out_matrix);
void BNN_MatrixDestroy(BNN_Matrix matrix);

/* bytes > 0; contents start uninitialised; a buffer has no element type. */
BNN_Status BNN_BufferAlloc(BNN_Device device, size_t bytes, BNN_Buffer* out_buffer);
void BNN_BufferFree(BNN_Buffer buffer);
/*
 * Synchronous raw byte copies with bounds checks.  With bytes == 0 the pointer
 * may be NULL but offset must still lie in [0, buffer size].
 */
BNN_Status BNN_BufferWrite(BNN_Buffer buffer, size_t offset, const void* src, size_t bytes);
BNN_Status BNN_BufferRead(BNN_Buffer buffer, size_t offset, void* dst, size_t bytes);

/*
 * Synchronous: on BNN_OK the complete result is readable.  FP32 arithmetic is
 * round-to-nearest-even with subnormals kept; FP16 scales convert exactly; each
 * group product is rounded to FP32 and the products are added in increasing
 * group order without FMA.  Unknown operations -> BNN_ENOTSUP; view type
 * mismatch -> BNN_EINVAL.  Argument, input or allocation failures leave the
 * output unchanged; only BNN_EIO / BNN_ETIMEOUT may leave partial output.
 * Success writes logical output elements only, never row padding.
 */
BNN_Status BNN_Execute(BNN_Device device, const BNN_Job* job);

const char* BNN_StatusString(BNN_Status status);

#ifdef __cplusplus
}
#endif

#endif
