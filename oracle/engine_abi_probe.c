/* Test infrastructure: prints the layout of the engine API types (sizes, field
 * offsets, enumerator values) so that the restated include/bnn-engine.h can be
 * compared with the reference's bnn-sw-v2/bnn-engine.h.  Not part of the product. */
#include "bnn-engine.h"

#include <stddef.h>
#include <stdio.h>

#define SIZE(t) printf("sizeof %s %zu\n", #t, sizeof(t))
#define OFF(t, f) printf("offsetof %s.%s %zu\n", #t, #f, offsetof(t, f))
#define VAL(e) printf("value %s %ld\n", #e, (long)(e))

int main(void) {
    VAL(BNNE_API_VERSION);
    VAL(BNNE_MAX_RANK);
    VAL(BNNE_OK); VAL(BNNE_EINVAL); VAL(BNNE_ENOMEM); VAL(BNNE_ENOTSUP);
    VAL(BNNE_ERANGE); VAL(BNNE_EIO); VAL(BNNE_EFORMAT); VAL(BNNE_ECOMPUTE);
    VAL(BNNE_TASK_CLASSIFY); VAL(BNNE_TASK_LLM);
    SIZE(BNNE_Status); SIZE(BNNE_Task);
    SIZE(BNNE_ModelInfo);
    OFF(BNNE_ModelInfo, task); OFF(BNNE_ModelInfo, arch); OFF(BNNE_ModelInfo, load_ns);
    OFF(BNNE_ModelInfo, input_rank); OFF(BNNE_ModelInfo, input_dims); OFF(BNNE_ModelInfo, input_size);
    OFF(BNNE_ModelInfo, n_classes); OFF(BNNE_ModelInfo, n_vocab); OFF(BNNE_ModelInfo, n_ctx_train);
    OFF(BNNE_ModelInfo, bos_token); OFF(BNNE_ModelInfo, eos_token);
    SIZE(BNNE_ContextParams);
    OFF(BNNE_ContextParams, n_ctx); OFF(BNNE_ContextParams, n_batch); OFF(BNNE_ContextParams, enable_stats);
    SIZE(BNNE_Stats);
    OFF(BNNE_Stats, calls); OFF(BNNE_Stats, items); OFF(BNNE_Stats, total_ns); OFF(BNNE_Stats, quantize_ns);
    OFF(BNNE_Stats, transfer_ns); OFF(BNNE_Stats, execute_ns); OFF(BNNE_Stats, host_ns);
    OFF(BNNE_Stats, device_calls); OFF(BNNE_Stats, bytes_written); OFF(BNNE_Stats, bytes_read);
    OFF(BNNE_Stats, logical_macs); OFF(BNNE_Stats, executed_macs);
    return 0;
}
