/* Test infrastructure: a minimal driver of the BNN engine API (bnn-engine.h), linked
 * either with the reference engine sources (bnn-sw-v2, compiled where they lie) or
 * with this project's libbnn_engine.so, so that both engines can be run on the same
 * GGUF file and their outputs compared bit for bit.  Not part of the product.
 *
 *   engine_run llm MODEL.gguf IDS_FILE STEPS CTX
 *       prefill the prompt IDs, then STEPS greedy steps (no EOG stop); prints
 *       "step <i> <argmax> <fnv64 of the logits bytes>" per decode call and a
 *       "stats" line (BNNE_Stats fields)
 *   engine_run classify MODEL.gguf INPUT_F32 SAMPLES BATCH
 *       classifies SAMPLES rows of raw float32 input, BATCH per call; prints every
 *       logit as 8 hex digits (its float32 bit pattern), one sample per line
 * Built against this project's engine (OWN_ENGINE), an optional last argument
 * selects the llm decode path: "host" (the host call pattern), "prepared" (the
 * device path with prepared batches only) or "device" (the default: fused
 * batches); the path in effect is printed as "path host|prepared|device".
 */
#include "bnn-engine.h"
#ifdef OWN_ENGINE
#include "bnn-engine-hip.h"
#endif

#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t fnv64(const void* data, size_t n) {
    const unsigned char* p = data;
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

static int fail(const char* what, BNNE_Status st) {
    fprintf(stderr, "error: %s: %s (%s)\n", what, BNNE_StatusString(st), BNNE_LastError());
    return 2;
}

static uint32_t argmax(const float* v, uint32_t n) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; i++)
        if (v[i] > v[best])
            best = i;
    return best;
}

static int run_llm(BNNE_Model model, const char* ids_path, uint32_t steps, uint32_t ctx, int mode) {
    BNNE_ModelInfo info;
    BNNE_Status st = BNNE_ModelGetInfo(model, &info);
    if (st != BNNE_OK)
        return fail("BNNE_ModelGetInfo", st);
    int rc = 2;
    BNNE_Context c = NULL;
    int32_t* ids = malloc((size_t)ctx * sizeof *ids);
    float* logits = malloc((size_t)info.n_vocab * sizeof *logits);
    FILE* f = fopen(ids_path, "r");
    if (!ids || !logits || !f)
        goto done;
    uint32_t count = 0;
    long v;
    while (count < ctx && fscanf(f, "%ld", &v) == 1)
        ids[count++] = (int32_t)v;
    BNNE_ContextParams params;
    BNNE_ContextParamsInit(&params);
    params.n_ctx = ctx;
    st = BNNE_ContextCreate(model, &params, &c);
    if (st != BNNE_OK) {
        rc = fail("BNNE_ContextCreate", st);
        goto done;
    }
#ifdef OWN_ENGINE
    if ((st = BNNEX_ContextSetResident(c, mode)) != BNNE_OK) {
        rc = fail("BNNEX_ContextSetResident", st);
        goto done;
    }
    static const char* const kPath[] = {"host", "device", "prepared"};
    printf("path %s\n", kPath[BNNEX_ContextIsResident(c)]);
#else
    (void)mode;
#endif
    st = BNNE_Decode(c, ids, count, logits);
    if (st != BNNE_OK) {
        rc = fail("BNNE_Decode(prefill)", st);
        goto done;
    }
    int32_t next = (int32_t)argmax(logits, info.n_vocab);
    const int32_t first = next;
    printf("step 0 %d %016" PRIx64 "\n", next, fnv64(logits, (size_t)info.n_vocab * 4));
    for (uint32_t s = 1; s <= steps; s++) {
        st = BNNE_Decode(c, &next, 1, logits);
        if (st != BNNE_OK) {
            rc = fail("BNNE_Decode", st);
            goto done;
        }
        next = (int32_t)argmax(logits, info.n_vocab);
        printf("step %u %d %016" PRIx64 "\n", s, next, fnv64(logits, (size_t)info.n_vocab * 4));
        fflush(stdout);
    }
    BNNE_Stats stats;
    BNNE_ContextGetStats(c, &stats);
    printf("stats calls=%" PRIu64 " items=%" PRIu64 " total_ns=%" PRIu64 " transfer_ns=%" PRIu64
           " execute_ns=%" PRIu64 " host_ns=%" PRIu64 " device_calls=%" PRIu64 "\n",
           stats.calls, stats.items, stats.total_ns, stats.transfer_ns, stats.execute_ns, stats.host_ns,
           stats.device_calls);
#ifdef OWN_ENGINE
    /* the same steps again, as one BNNEX_DecodeGreedy call from the first generated token */
    if (steps > 0) {
        int32_t* greedy = malloc(steps * sizeof *greedy);
        if (!greedy)
            goto done;
        if ((st = BNNE_ContextTruncate(c, count)) != BNNE_OK ||
            (st = BNNEX_DecodeGreedy(c, first, steps, greedy)) != BNNE_OK) {
            free(greedy);
            rc = fail("BNNEX_DecodeGreedy", st);
            goto done;
        }
        printf("greedy");
        for (uint32_t s = 0; s < steps; s++)
            printf(" %d", greedy[s]);
        printf("\n");
        free(greedy);
    }
#else
    (void)first;
#endif
    rc = 0;
done:
    if (f)
        fclose(f);
    BNNE_ContextFree(c);
    free(ids);
    free(logits);
    return rc;
}

static int run_classify(BNNE_Model model, const char* input_path, uint32_t samples, uint32_t batch, int mode) {
    BNNE_ModelInfo info;
    BNNE_Status st = BNNE_ModelGetInfo(model, &info);
    if (st != BNNE_OK)
        return fail("BNNE_ModelGetInfo", st);
    int rc = 2;
    BNNE_Context c = NULL;
    float* x = malloc((size_t)samples * info.input_size * sizeof *x);
    float* logits = malloc((size_t)batch * info.n_classes * sizeof *logits);
    FILE* f = fopen(input_path, "rb");
    if (!x || !logits || !f || fread(x, sizeof *x, (size_t)samples * info.input_size, f) !=
                                   (size_t)samples * info.input_size)
        goto done;
    BNNE_ContextParams params;
    BNNE_ContextParamsInit(&params);
    params.n_batch = batch;
    st = BNNE_ContextCreate(model, &params, &c);
    if (st != BNNE_OK) {
        rc = fail("BNNE_ContextCreate", st);
        goto done;
    }
#ifdef OWN_ENGINE
    if (mode >= 0 && (st = BNNEX_ContextSetResident(c, mode)) != BNNE_OK) {
        rc = fail("BNNEX_ContextSetResident", st);
        goto done;
    }
    /* the path on stderr: stdout holds only the logits */
    fprintf(stderr, "path %s\n", BNNEX_ContextIsResident(c) ? "device" : "host");
#else
    (void)mode;
#endif
    for (uint32_t s0 = 0; s0 < samples; s0 += batch) {
        const uint32_t n = samples - s0 < batch ? samples - s0 : batch;
        st = BNNE_Classify(c, x + (size_t)s0 * info.input_size, n, logits);
        if (st != BNNE_OK) {
            rc = fail("BNNE_Classify", st);
            goto done;
        }
        for (uint32_t i = 0; i < n; i++) {
            for (uint32_t k = 0; k < info.n_classes; k++) {
                uint32_t bits;
                memcpy(&bits, &logits[(size_t)i * info.n_classes + k], 4);
                printf("%08x%c", bits, k + 1 == info.n_classes ? '\n' : ' ');
            }
        }
    }
    rc = 0;
done:
    if (f)
        fclose(f);
    BNNE_ContextFree(c);
    free(x);
    free(logits);
    return rc;
}

int main(int argc, char** argv) {
    /* BNNEX_ContextSetResident: 0 host, 1 device (fused), 2 prepared batches; the
     * context's default path when not given (-2) */
    int mode = -2;
    if (argc == 7)
        mode = strcmp(argv[6], "host") == 0 ? 0 : strcmp(argv[6], "prepared") == 0 ? 2
                                            : strcmp(argv[6], "device") == 0 ? 1 : -1;
    if ((argc != 6 && argc != 7) || mode == -1 || (strcmp(argv[1], "llm") != 0 && strcmp(argv[1], "classify") != 0)) {
        fprintf(stderr, "usage: %s llm MODEL IDS STEPS CTX | classify MODEL INPUT SAMPLES BATCH [host|device|prepared]\n", argv[0]);
        return 1;
    }
    BNN_Device dev = NULL;
    BNN_Status ds = BNN_DeviceOpen(0, &dev);
    if (ds != BNN_OK) {
        fprintf(stderr, "error: BNN_DeviceOpen: %s\n", BNN_StatusString(ds));
        return 2;
    }
    BNNE_Model model = NULL;
    BNNE_Status st = BNNE_ModelLoad(dev, argv[2], &model);
    if (st != BNNE_OK) {
        BNN_DeviceClose(dev);
        return fail("BNNE_ModelLoad", st);
    }
    const uint32_t a = (uint32_t)strtoul(argv[4], NULL, 10), b = (uint32_t)strtoul(argv[5], NULL, 10);
    const int rc = strcmp(argv[1], "llm") == 0 ? run_llm(model, argv[3], a, b, mode < 0 ? 1 : mode)
                                                   : run_classify(model, argv[3], a, b, mode);
    BNNE_ModelFree(model);
    BNN_DeviceClose(dev);
    return rc;
}
