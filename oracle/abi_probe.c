/*
 * abi_probe.c -- TEST INFRASTRUCTURE.  Prints the layout of every type and the
 * value of every constant of the BNN accelerator API v2 header it is compiled
 * against.  Built twice by oracle/Makefile: against include/bnn-accelerator.h
 * (this project) and, where the reference tree is present, against the
 * reference's bnn-accelerator/bnn-accelerator.h.  tests/test_abi.py requires
 * the two outputs (and the committed tests/golden/abi_layout.txt) to be equal.
 */
#include "bnn-accelerator.h"

#include <stddef.h>
#include <stdio.h>

#define SZ(t) printf("sizeof %s %zu\n", #t, sizeof(t))
#define AL(t) printf("alignof %s %zu\n", #t, _Alignof(t))
#define OFF(t, f) printf("offsetof %s.%s %zu\n", #t, #f, offsetof(t, f))
#define VAL(c) printf("value %s %lld\n", #c, (long long)(c))

int main(void) {
    VAL(BNN_API_VERSION);
    VAL(BNN_OK); VAL(BNN_EINVAL); VAL(BNN_ENOMEM); VAL(BNN_ENOTSUP);
    VAL(BNN_ERANGE); VAL(BNN_EBUSY); VAL(BNN_EIO); VAL(BNN_ETIMEOUT);
    VAL(BNN_OP_GEMV); VAL(BNN_OP_GEMM); VAL(BNN_OP_DOT_GROUPS); VAL(BNN_OP_GEMV_F32); VAL(BNN_OP_GEMM_F32);
    VAL(BNN_TYPE_I8); VAL(BNN_TYPE_F32); VAL(BNN_TYPE_I16);
    VAL(BNN_CAP_GEMV); VAL(BNN_CAP_GEMM); VAL(BNN_CAP_DOT_GROUPS); VAL(BNN_CAP_GEMV_F32); VAL(BNN_CAP_GEMM_F32);
    SZ(BNN_Status); SZ(BNN_Operation); SZ(BNN_Type); SZ(BNN_OperationCaps);
    SZ(BNN_Device); SZ(BNN_Matrix); SZ(BNN_Buffer);
    SZ(BNN_Caps); AL(BNN_Caps);
    OFF(BNN_Caps, api_version); OFF(BNN_Caps, max_in_features); OFF(BNN_Caps, max_out_features);
    OFF(BNN_Caps, max_rows); OFF(BNN_Caps, group_size); OFF(BNN_Caps, supported_ops);
    SZ(BNN_MatrixDesc); AL(BNN_MatrixDesc);
    OFF(BNN_MatrixDesc, in_features); OFF(BNN_MatrixDesc, out_features); OFF(BNN_MatrixDesc, group_size);
    OFF(BNN_MatrixDesc, weight_bits); OFF(BNN_MatrixDesc, weight_bytes);
    OFF(BNN_MatrixDesc, scale_fp16); OFF(BNN_MatrixDesc, scale_count);
    SZ(BNN_BufferView); AL(BNN_BufferView);
    OFF(BNN_BufferView, buffer); OFF(BNN_BufferView, type); OFF(BNN_BufferView, offset);
    OFF(BNN_BufferView, row_stride);
    SZ(BNN_Job); AL(BNN_Job);
    OFF(BNN_Job, operation); OFF(BNN_Job, matrix); OFF(BNN_Job, input); OFF(BNN_Job, output);
    OFF(BNN_Job, rows);
    return 0;
}
