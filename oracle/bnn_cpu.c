/*
 * bnn_cpu.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference's
 * soft backend, used as the parity oracle and as the single-core CPU baseline.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker.  The product (libbnn_hip.so) never
 * links, loads or calls it.
 *
 * It implements the same eleven BNN_* entry points as the reference backend
 * (bnn-accelerator/soft-bnn-accelerator.c:310-626) with the same validation
 * order, the same status codes, and the same arithmetic:
 *   - binary16 -> binary32 exactly              (soft-bnn-accelerator.c:92-121)
 *   - one rounding per FP32 multiply/add/divide (soft-bnn-accelerator.c:127-140)
 *   - full-row absmax quantisation              (soft-bnn-accelerator.c:175-211)
 *   - per-group positive-bit sum, D = 2*pos - sum(x), FP32 accumulation in
 *     increasing group order                     (soft-bnn-accelerator.c:219-276)
 * The loop structure (a branch per weight bit, single thread) is kept so that
 * timing it stands in for timing the reference.
 *
 * Pinning (see tests/test_oracle_*.py): the reference's own contract test
 * (tests/accelerator/test_bnn_accelerator.c) passes against this file; the
 * RTL golden case (bnn-hw-v2/simple_test/tests/case/golden_*.hex) is
 * reproduced bit-exactly; soft-generated fixtures at the benchmark shapes match;
 * the half converter is checked exhaustively against numpy's float16; the
 * quantiser is checked against exact rational arithmetic.
 *
 * oracle_execute_parallel() is a second, faster evaluation of the same
 * function (byte lookup tables for D, pthreads over output features) for
 * parity checks at full benchmark sizes.  Integer D is exact either way and the
 * FP32 sequence per output is identical, so the results are bit-identical;
 * a test checks that against the scalar path.
 */
#include "bnn-accelerator.h"

#include <fenv.h>
#include <float.h>
#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if CHAR_BIT != 8
#error "8-bit bytes required"
#endif
#if FLT_RADIX != 2 || FLT_MANT_DIG != 24 || FLT_MAX_EXP != 128
#error "IEEE-754 binary32 float required"
#endif
#if !defined(FLT_EVAL_METHOD) || FLT_EVAL_METHOD != 0
#error "float expressions must be evaluated in float (FLT_EVAL_METHOD 0)"
#endif
#ifdef __FAST_MATH__
#error "build without fast-math"
#endif

#define CPU_MAX_FEATURES 8192u
#define CPU_GROUP 128u
#define CPU_MAX_GROUPS (CPU_MAX_FEATURES / CPU_GROUP)

#define EXPORT __attribute__((visibility("default")))

struct bnn_accel_device {
    size_t live_matrices;
    size_t live_buffers;
};

struct bnn_accel_matrix {
    BNN_Device device;
    uint32_t k;      /* in_features */
    uint32_t n;      /* out_features */
    uint32_t groups; /* k / 128 */
    uint8_t* bits;   /* [n][k/8], caller layout */
    uint16_t* half;  /* [n][groups] */
};

struct bnn_accel_buffer {
    BNN_Device device;
    size_t size;
    unsigned char* bytes;
};

/* ---- overflow-safe size arithmetic (soft-bnn-accelerator.c:49-77) ---- */

static int mul_size(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a)
        return 0;
    *out = a * b;
    return 1;
}

static int span_fits(size_t capacity, size_t offset, size_t bytes) {
    if (offset > capacity)
        return 0;
    return bytes <= capacity - offset;
}

/* Last row [offset + (rows-1)*stride, +row_bytes) inside capacity, without
 * forming (rows-1)*stride. */
static int rows_fit(size_t capacity, size_t offset, size_t stride, size_t row_bytes, uint32_t rows) {
    size_t room;
    if (rows == 0 || row_bytes == 0 || stride < row_bytes || offset > capacity)
        return 0;
    room = capacity - offset;
    if (row_bytes > room)
        return 0;
    return (uintmax_t)(rows - 1u) <= (uintmax_t)((room - row_bytes) / stride);
}

/* ---- numerics ---- */

/* Exact binary16 -> binary32 (soft-bnn-accelerator.c:92-121). */
EXPORT float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t fraction = h & 0x3ffu;
    uint32_t bits;
    float value;

    if (exponent == 31u) {
        bits = sign | 0x7f800000u | (fraction << 13);
    } else if (exponent != 0u) {
        bits = sign | ((exponent + 112u) << 23) | (fraction << 13);
    } else if (fraction == 0u) {
        bits = sign;
    } else {
        /* subnormal half: value = fraction * 2^-24; normalise the fraction */
        int e = -14;
        while ((fraction & 0x400u) == 0u) {
            fraction <<= 1;
            --e;
        }
        bits = sign | ((uint32_t)(e + 127) << 23) | ((fraction & 0x3ffu) << 13);
    }
    memcpy(&value, &bits, sizeof value);
    return value;
}

/* One rounding per operation: volatile stores plus -ffp-contract=off
 * (soft-bnn-accelerator.c:127-140). */
static float f32_mul(float a, float b) {
    volatile float r = a * b;
    return r;
}
static float f32_add(float a, float b) {
    volatile float r = a + b;
    return r;
}
static float f32_div(float a, float b) {
    volatile float r = a / b;
    return r;
}

static float read_f32(const unsigned char* p) {
    float v;
    memcpy(&v, p, sizeof v);
    return v;
}

/*
 * Full-row absmax quantisation (soft-bnn-accelerator.c:175-211; contract at
 * bnn-accelerator.h:141-149).  Input assumed finite.  Returns the row scale s.
 */
static float quantize_row_bytes(const unsigned char* row, uint32_t count, int8_t* q) {
    float a = 0.0f, s;
    uint32_t i;
    for (i = 0; i < count; ++i) {
        float v = fabsf(read_f32(row + (size_t)i * 4u));
        if (v > a)
            a = v;
    }
    if (a == 0.0f) {
        s = 1.0f;
    } else {
        s = f32_div(a, 127.0f);
        if (s == 0.0f)
            s = FLT_TRUE_MIN;
    }
    for (i = 0; i < count; ++i) {
        float r = roundf(f32_div(read_f32(row + (size_t)i * 4u), s)); /* half away from zero */
        if (r > 127.0f)
            r = 127.0f;
        if (r < -127.0f)
            r = -127.0f;
        q[i] = (int8_t)r;
    }
    return s;
}

EXPORT float oracle_quantize_row(const float* x, uint32_t count, int8_t* q) {
    return quantize_row_bytes((const unsigned char*)x, count, q);
}

/*
 * One row through the matrix, reference loop structure
 * (soft-bnn-accelerator.c:219-276).  y receives N floats or N*groups int16.
 */
static void row_product(const struct bnn_accel_matrix* m, const int8_t* x, unsigned char* y,
                        BNN_Operation op, float row_scale, int apply_row_scale) {
    int32_t group_sum[CPU_MAX_GROUPS];
    const size_t row_bytes = m->k / 8u;
    uint32_t g, n, k;

    for (g = 0; g < m->groups; ++g) {
        int32_t s = 0;
        for (k = g * CPU_GROUP; k < (g + 1u) * CPU_GROUP; ++k)
            s += x[k];
        group_sum[g] = s;
    }

    for (n = 0; n < m->n; ++n) {
        const uint8_t* w = m->bits + (size_t)n * row_bytes;
        float acc = 0.0f;
        for (g = 0; g < m->groups; ++g) {
            int32_t pos = 0, d;
            for (k = g * CPU_GROUP; k < (g + 1u) * CPU_GROUP; ++k)
                if ((w[k >> 3] >> (k & 7u)) & 1u)
                    pos += x[k];
            d = 2 * pos - group_sum[g]; /* |d| <= 16256 for G = 128 */
            if (op == BNN_OP_DOT_GROUPS) {
                int16_t d16 = (int16_t)d;
                memcpy(y + ((size_t)n * m->groups + g) * 2u, &d16, 2u);
            } else {
                float term = f32_mul(oracle_half_to_float(m->half[(size_t)n * m->groups + g]), (float)d);
                acc = f32_add(acc, term);
            }
        }
        if (op != BNN_OP_DOT_GROUPS) {
            float out = apply_row_scale ? f32_mul(acc, row_scale) : acc;
            memcpy(y + (size_t)n * 4u, &out, 4u);
        }
    }
}

static BNN_Status io_types(BNN_Operation op, BNN_Type* in, BNN_Type* out) {
    switch (op) {
    case BNN_OP_GEMV:
    case BNN_OP_GEMM:
        *in = BNN_TYPE_I8;
        *out = BNN_TYPE_F32;
        return BNN_OK;
    case BNN_OP_DOT_GROUPS:
        *in = BNN_TYPE_I8;
        *out = BNN_TYPE_I16;
        return BNN_OK;
    case BNN_OP_GEMV_F32:
    case BNN_OP_GEMM_F32:
        *in = BNN_TYPE_F32;
        *out = BNN_TYPE_F32;
        return BNN_OK;
    default:
        return BNN_ENOTSUP;
    }
}

/* Logical-input checks over all rows before anything is written
 * (soft-bnn-accelerator.c:278-308, 575-587). */
static BNN_Status check_rows(const unsigned char* base, size_t stride, uint32_t rows, uint32_t count,
                             int is_f32) {
    uint32_t r, i;
    for (r = 0; r < rows; ++r) {
        const unsigned char* row = base + (size_t)r * stride;
        for (i = 0; i < count; ++i) {
            if (is_f32) {
                if (!isfinite(read_f32(row + (size_t)i * 4u)))
                    return BNN_ERANGE;
            } else if ((int8_t)row[i] == INT8_MIN) {
                return BNN_ERANGE;
            }
        }
    }
    return BNN_OK;
}

/* ---- API (soft-bnn-accelerator.c:310-626) ---- */

EXPORT BNN_Status BNN_DeviceOpen(uint32_t device_index, BNN_Device* out_device) {
    float one = 1.0f;
    uint32_t one_bits;
    BNN_Device d;
    if (out_device == NULL)
        return BNN_EINVAL;
    *out_device = NULL;
    memcpy(&one_bits, &one, sizeof one_bits);
    if (device_index != 0u || one_bits != 0x3f800000u)
        return BNN_ENOTSUP;
    d = calloc(1, sizeof *d);
    if (d == NULL)
        return BNN_ENOMEM;
    *out_device = d;
    return BNN_OK;
}

EXPORT BNN_Status BNN_DeviceClose(BNN_Device device) {
    if (device == NULL)
        return BNN_EINVAL;
    if (device->live_matrices || device->live_buffers)
        return BNN_EBUSY;
    free(device);
    return BNN_OK;
}

/* Test hook: ORACLE_MAX_ROWS=n makes this backend report max_rows = n and reject jobs
 * with more rows (as the reference's remote backend does with its 128-row limit,
 * remote-bnn-accelerator.c:39,432,624), so that callers' row splitting can be tested. */
static uint32_t max_rows_limit(void) {
    const char* v = getenv("ORACLE_MAX_ROWS");
    const long n = v ? strtol(v, NULL, 10) : 0;
    return n > 0 && n < (long)UINT32_MAX ? (uint32_t)n : UINT32_MAX;
}

EXPORT BNN_Status BNN_DeviceGetCaps(BNN_Device device, BNN_Caps* out_caps) {
    if (device == NULL || out_caps == NULL)
        return BNN_EINVAL;
    memset(out_caps, 0, sizeof *out_caps);
    out_caps->api_version = BNN_API_VERSION;
    out_caps->max_in_features = CPU_MAX_FEATURES;
    out_caps->max_out_features = CPU_MAX_FEATURES;
    out_caps->max_rows = max_rows_limit();
    out_caps->group_size = CPU_GROUP;
    out_caps->supported_ops = BNN_CAP_GEMV | BNN_CAP_GEMM | BNN_CAP_DOT_GROUPS | BNN_CAP_GEMV_F32 |
                              BNN_CAP_GEMM_F32;
    return BNN_OK;
}

EXPORT BNN_Status BNN_MatrixCreate(BNN_Device device, const BNN_MatrixDesc* desc, BNN_Matrix* out_matrix) {
    size_t bits_bytes, scale_count, scale_bytes, i;
    struct bnn_accel_matrix* m;

    if (out_matrix == NULL)
        return BNN_EINVAL;
    *out_matrix = NULL;
    if (device == NULL || desc == NULL)
        return BNN_EINVAL;
    if (desc->in_features == 0u || desc->out_features == 0u || desc->group_size == 0u ||
        desc->group_size > 256u || (desc->group_size & 7u) != 0u)
        return BNN_EINVAL;
    if (desc->in_features > CPU_MAX_FEATURES || desc->out_features > CPU_MAX_FEATURES ||
        desc->group_size != CPU_GROUP)
        return BNN_ENOTSUP;
    if (desc->in_features % CPU_GROUP != 0u)
        return BNN_EINVAL;
    if (!mul_size(desc->out_features, desc->in_features / 8u, &bits_bytes) ||
        !mul_size(desc->out_features, desc->in_features / CPU_GROUP, &scale_count) ||
        !mul_size(scale_count, sizeof(uint16_t), &scale_bytes))
        return BNN_ERANGE;
    if (desc->weight_bits == NULL || desc->scale_fp16 == NULL || desc->weight_bytes != bits_bytes ||
        desc->scale_count != scale_count)
        return BNN_EINVAL;
    for (i = 0; i < scale_count; ++i)
        if ((desc->scale_fp16[i] & 0x7c00u) == 0x7c00u) /* NaN or Inf */
            return BNN_EINVAL;
    if (device->live_matrices == SIZE_MAX)
        return BNN_ERANGE;

    m = calloc(1, sizeof *m);
    if (m == NULL)
        return BNN_ENOMEM;
    m->bits = malloc(bits_bytes);
    m->half = malloc(scale_bytes);
    if (m->bits == NULL || m->half == NULL) {
        free(m->bits);
        free(m->half);
        free(m);
        return BNN_ENOMEM;
    }
    memcpy(m->bits, desc->weight_bits, bits_bytes);
    memcpy(m->half, desc->scale_fp16, scale_bytes);
    m->device = device;
    m->k = desc->in_features;
    m->n = desc->out_features;
    m->groups = desc->in_features / CPU_GROUP;
    device->live_matrices++;
    *out_matrix = m;
    return BNN_OK;
}

EXPORT void BNN_MatrixDestroy(BNN_Matrix matrix) {
    if (matrix == NULL)
        return;
    matrix->device->live_matrices--;
    free(matrix->bits);
    free(matrix->half);
    free(matrix);
}

EXPORT BNN_Status BNN_BufferAlloc(BNN_Device device, size_t bytes, BNN_Buffer* out_buffer) {
    struct bnn_accel_buffer* b;
    if (out_buffer == NULL)
        return BNN_EINVAL;
    *out_buffer = NULL;
    if (device == NULL || bytes == 0u)
        return BNN_EINVAL;
    if (device->live_buffers == SIZE_MAX)
        return BNN_ERANGE;
    b = calloc(1, sizeof *b);
    if (b == NULL)
        return BNN_ENOMEM;
    b->bytes = malloc(bytes);
    if (b->bytes == NULL) {
        free(b);
        return BNN_ENOMEM;
    }
    b->device = device;
    b->size = bytes;
    device->live_buffers++;
    *out_buffer = b;
    return BNN_OK;
}

EXPORT void BNN_BufferFree(BNN_Buffer buffer) {
    if (buffer == NULL)
        return;
    buffer->device->live_buffers--;
    free(buffer->bytes);
    free(buffer);
}

EXPORT BNN_Status BNN_BufferWrite(BNN_Buffer buffer, size_t offset, const void* src, size_t bytes) {
    if (buffer == NULL || (bytes != 0u && src == NULL))
        return BNN_EINVAL;
    if (!span_fits(buffer->size, offset, bytes))
        return BNN_ERANGE;
    if (bytes)
        memcpy(buffer->bytes + offset, src, bytes);
    return BNN_OK;
}

EXPORT BNN_Status BNN_BufferRead(BNN_Buffer buffer, size_t offset, void* dst, size_t bytes) {
    if (buffer == NULL || (bytes != 0u && dst == NULL))
        return BNN_EINVAL;
    if (!span_fits(buffer->size, offset, bytes))
        return BNN_ERANGE;
    if (bytes)
        memcpy(dst, buffer->bytes + offset, bytes);
    return BNN_OK;
}

EXPORT BNN_Status BNN_Execute(BNN_Device device, const BNN_Job* job) {
    const struct bnn_accel_matrix* m;
    BNN_Type in_type, out_type;
    size_t in_row, out_row, out_count, in_stride, out_stride;
    int8_t q[CPU_MAX_FEATURES];
    BNN_Status st;
    uint32_t r;

    if (device == NULL || job == NULL || job->matrix == NULL || job->input.buffer == NULL ||
        job->output.buffer == NULL || job->rows == 0u)
        return BNN_EINVAL;
    st = io_types(job->operation, &in_type, &out_type);
    if (st != BNN_OK)
        return st;
    if ((job->operation == BNN_OP_GEMV || job->operation == BNN_OP_GEMV_F32) && job->rows != 1u)
        return BNN_EINVAL;
    if (job->rows > max_rows_limit())
        return BNN_EINVAL;
    if (job->input.type != in_type || job->output.type != out_type)
        return BNN_EINVAL;
    m = job->matrix;
    if (m->device != device || job->input.buffer->device != device || job->output.buffer->device != device ||
        job->input.buffer == job->output.buffer)
        return BNN_EINVAL;

    if (!mul_size(m->k, in_type == BNN_TYPE_F32 ? 4u : 1u, &in_row))
        return BNN_ERANGE;
    if (job->operation == BNN_OP_DOT_GROUPS) {
        if (!mul_size(m->n, m->groups, &out_count) || !mul_size(out_count, 2u, &out_row))
            return BNN_ERANGE;
    } else if (!mul_size(m->n, 4u, &out_row)) {
        return BNN_ERANGE;
    }
    in_stride = job->input.row_stride ? job->input.row_stride : in_row;
    out_stride = job->output.row_stride ? job->output.row_stride : out_row;
    if (in_stride < in_row || out_stride < out_row)
        return BNN_EINVAL;
    if (!rows_fit(job->input.buffer->size, job->input.offset, in_stride, in_row, job->rows) ||
        !rows_fit(job->output.buffer->size, job->output.offset, out_stride, out_row, job->rows))
        return BNN_ERANGE;
    if (job->operation != BNN_OP_DOT_GROUPS && fegetround() != FE_TONEAREST)
        return BNN_ENOTSUP;

    st = check_rows(job->input.buffer->bytes + job->input.offset, in_stride, job->rows, m->k,
                    in_type == BNN_TYPE_F32);
    if (st != BNN_OK)
        return st;

    for (r = 0; r < job->rows; ++r) {
        const unsigned char* in = job->input.buffer->bytes + job->input.offset + (size_t)r * in_stride;
        unsigned char* out = job->output.buffer->bytes + job->output.offset + (size_t)r * out_stride;
        if (in_type == BNN_TYPE_F32) {
            float s = quantize_row_bytes(in, m->k, q);
            row_product(m, q, out, job->operation, s, 1);
        } else {
            row_product(m, (const int8_t*)in, out, job->operation, 0.0f, 0);
        }
    }
    return BNN_OK;
}

EXPORT const char* BNN_StatusString(BNN_Status status) {
    switch (status) {
    case BNN_OK:
        return "success";
    case BNN_EINVAL:
        return "invalid argument";
    case BNN_ENOMEM:
        return "out of memory";
    case BNN_ENOTSUP:
        return "unsupported operation or configuration";
    case BNN_ERANGE:
        return "buffer or input range error";
    case BNN_EBUSY:
        return "device still owns resources";
    case BNN_EIO:
        return "device I/O error";
    case BNN_ETIMEOUT:
        return "device timeout";
    default:
        return "unknown status";
    }
}

/* ====================================================================== */
/* Faster exact evaluation for large parity checks (same function).       */
/* ====================================================================== */

typedef struct {
    const uint8_t* bits;   /* [n][k/8] */
    const uint16_t* half;  /* [n][groups] */
    uint32_t k, n, groups;
    int op;
    uint32_t rows;
    const int8_t* q;       /* [rows][k] quantised rows */
    const float* row_scale;/* [rows] or NULL */
    void* out;             /* tight [rows][n] f32 or [rows][n][groups] i16 */
    uint32_t n_begin, n_end;
    const int16_t* table;  /* [rows][k/8][256] positive-bit sums */
    const int32_t* sums;   /* [rows][groups] */
} fast_task;

static void* fast_worker(void* arg) {
    const fast_task* t = arg;
    const uint32_t bytes_per_row = t->k / 8u;
    uint32_t r, n, g, b;
    for (r = 0; r < t->rows; ++r) {
        const int16_t* tab = t->table + (size_t)r * bytes_per_row * 256u;
        const int32_t* sums = t->sums + (size_t)r * t->groups;
        for (n = t->n_begin; n < t->n_end; ++n) {
            const uint8_t* w = t->bits + (size_t)n * bytes_per_row;
            float acc = 0.0f;
            for (g = 0; g < t->groups; ++g) {
                int32_t pos = 0, d;
                for (b = g * 16u; b < g * 16u + 16u; ++b)
                    pos += tab[(size_t)b * 256u + w[b]];
                d = 2 * pos - sums[g];
                if (t->op == BNN_OP_DOT_GROUPS) {
                    ((int16_t*)t->out)[((size_t)r * t->n + n) * t->groups + g] = (int16_t)d;
                } else {
                    float term = f32_mul(oracle_half_to_float(t->half[(size_t)n * t->groups + g]), (float)d);
                    acc = f32_add(acc, term);
                }
            }
            if (t->op != BNN_OP_DOT_GROUPS)
                ((float*)t->out)[(size_t)r * t->n + n] = t->row_scale ? f32_mul(acc, t->row_scale[r]) : acc;
        }
    }
    return NULL;
}

/*
 * Evaluate one job on tight host arrays with `threads` threads.
 *   op: BNN_OP_* ; input: [rows][k] int8 (I8 ops) or float (F32 ops);
 *   out: [rows][n] float or [rows][n][k/128] int16.
 * Returns BNN_ERANGE if any logical input is illegal (nothing written),
 * BNN_EINVAL on bad sizes, BNN_ENOMEM on allocation failure.
 */
EXPORT BNN_Status oracle_execute_parallel(int op, const uint8_t* bits, const uint16_t* half, uint32_t k,
                                          uint32_t n, uint32_t rows, const void* input, void* out,
                                          int threads) {
    const uint32_t groups = k / CPU_GROUP, bytes_per_row = k / 8u;
    int is_f32 = (op == BNN_OP_GEMV_F32 || op == BNN_OP_GEMM_F32);
    int8_t* q = NULL;
    float* rs = NULL;
    int16_t* table = NULL;
    int32_t* sums = NULL;
    pthread_t tid[256];
    fast_task task[256];
    BNN_Status st = BNN_OK;
    uint32_t r, i, b, v;
    int t, started = 0;

    if (k == 0u || k % CPU_GROUP || n == 0u || rows == 0u || op < 1 || op > 5)
        return BNN_EINVAL;
    if (threads < 1)
        threads = 1;
    if (threads > 256)
        threads = 256;
    st = check_rows(input, (size_t)k * (is_f32 ? 4u : 1u), rows, k, is_f32);
    if (st != BNN_OK)
        return st;

    q = malloc((size_t)rows * k);
    rs = is_f32 ? malloc((size_t)rows * sizeof *rs) : NULL;
    table = malloc((size_t)rows * bytes_per_row * 256u * sizeof *table);
    sums = malloc((size_t)rows * groups * sizeof *sums);
    if (!q || (is_f32 && !rs) || !table || !sums) {
        st = BNN_ENOMEM;
        goto done;
    }
    for (r = 0; r < rows; ++r) {
        int8_t* qr = q + (size_t)r * k;
        if (is_f32)
            rs[r] = quantize_row_bytes((const unsigned char*)input + (size_t)r * k * 4u, k, qr);
        else
            memcpy(qr, (const int8_t*)input + (size_t)r * k, k);
        for (i = 0; i < groups; ++i) {
            int32_t s = 0;
            for (b = 0; b < CPU_GROUP; ++b)
                s += qr[i * CPU_GROUP + b];
            sums[(size_t)r * groups + i] = s;
        }
        for (b = 0; b < bytes_per_row; ++b) {
            int16_t* row = table + ((size_t)r * bytes_per_row + b) * 256u;
            for (v = 0; v < 256u; ++v) {
                int32_t s = 0;
                for (i = 0; i < 8u; ++i)
                    if ((v >> i) & 1u)
                        s += qr[b * 8u + i];
                row[v] = (int16_t)s;
            }
        }
    }
    for (t = 0; t < threads; ++t) {
        fast_task* x = &task[t];
        x->bits = bits;
        x->half = half;
        x->k = k;
        x->n = n;
        x->groups = groups;
        x->op = op;
        x->rows = rows;
        x->q = q;
        x->row_scale = is_f32 ? rs : NULL;
        x->out = out;
        x->n_begin = (uint32_t)((uint64_t)n * (uint64_t)t / (uint64_t)threads);
        x->n_end = (uint32_t)((uint64_t)n * (uint64_t)(t + 1) / (uint64_t)threads);
        x->table = table;
        x->sums = sums;
    }
    for (t = 1; t < threads; ++t) {
        if (pthread_create(&tid[t], NULL, fast_worker, &task[t]) != 0)
            break;
        started = t;
    }
    fast_worker(&task[0]);
    for (t = 1; t <= started; ++t)
        pthread_join(tid[t], NULL);
    for (t = started + 1; t < threads; ++t) /* threads that failed to start */
        fast_worker(&task[t]);
done:
    free(q);
    free(rs);
    free(table);
    free(sums);
    return st;
}
