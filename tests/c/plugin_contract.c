/*
 * Plugin-contract check for libxllm_hip_backend.so, driven like the
 * reference backend manager drives a plugin (src/core/backend_manager.c:
 * dlopen RTLD_NOW|RTLD_LOCAL :274, dlsym of the three entry points :283-285,
 * state INITIALIZING -> READY or ERROR :302-314, run only when READY :342) and
 * asserting the conventions of the reference's tests/test_backend_load.c:83-163.
 *
 *   plugin_contract <path/to/libxllm_hip_backend.so> [--gpu]
 *
 * Without --gpu: init may fail (no device); every NULL-argument convention
 * is still checked.  With --gpu: init must succeed, a garbage descriptor
 * (a 4-byte int, as test_backend_load.c:116-118 passes) must be refused, and
 * a real decode on device buffers must return 0 and match a CPU softmax
 * computed here.  Exit status 0 = all checks passed.
 */
#include <dlfcn.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "xllm_hip_backend.h"

typedef int (*InitFn)(NxtBackend *);
typedef int (*RunFn)(NxtBackend *, void *, void *);
typedef int (*FiniFn)(NxtBackend *);

static int failures = 0;
#define CHECK(cond, msg)                                              \
    do {                                                              \
        if (cond) {                                                   \
            printf("  ok   %s\n", msg);                               \
        } else {                                                      \
            printf("  FAIL %s (%s:%d)\n", msg, __FILE__, __LINE__);   \
            failures++;                                               \
        }                                                             \
    } while (0)

/* fp32 -> binary16, round to nearest even, for |f| in [2^-14, 65504] or 0:
 * the inputs below are multiples of 2^-9 in [-1, 1), all exact in binary16
 * (anything smaller than the normal range is flushed to a signed zero). */
static unsigned short to_half(float f) {
    unsigned int x;
    memcpy(&x, &f, 4);
    unsigned short sign = (unsigned short)((x >> 16) & 0x8000u);
    unsigned int ax = x & 0x7FFFFFFFu;
    if (ax < 0x38800000u) return sign; /* below 2^-14 */
    unsigned int odd = (ax >> 13) & 1u;
    ax += 0xC8000FFFu + odd;
    return sign | (unsigned short)(ax >> 13);
}

/* A seeded value in [-1, 1) that is a multiple of 2^-9. */
static float next_value(unsigned int *seed) {
    *seed = *seed * 1664525u + 1013904223u;
    return (float)((int)(*seed >> 22) - 512) / 512.0f;
}

static float from_half(unsigned short h) {
    unsigned int sign = (unsigned int)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    unsigned int bits = e ? (sign | ((e + 112u) << 23) | (m << 13)) : sign; /* no subnormals used */
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static int real_decode(RunFn run, NxtBackend *b) {
    enum { S = 2, H = 8, KVH = 2, D = 128, BS = 16, MAXB = 4, NB = 8 };
    const int lens[S] = {37, 60};
    const int table[S * MAXB] = {5, 1, 7, -1, 2, 0, 6, 3};
    const size_t q_n = (size_t)S * H * D, kv_n = (size_t)NB * KVH * BS * D;
    unsigned short *q = malloc(q_n * 2), *k = malloc(kv_n * 2), *v = malloc(kv_n * 2),
                   *o = malloc(q_n * 2);
    unsigned int seed = 12345u;
    for (size_t i = 0; i < q_n; i++) q[i] = to_half(next_value(&seed));
    for (size_t i = 0; i < kv_n; i++) {
        k[i] = to_half(next_value(&seed));
        v[i] = to_half(next_value(&seed));
    }
    void *dq, *dk, *dv, *dout, *dbt, *dsl;
    if (hipMalloc(&dq, q_n * 2) || hipMalloc(&dk, kv_n * 2) || hipMalloc(&dv, kv_n * 2) ||
        hipMalloc(&dout, q_n * 2) || hipMalloc(&dbt, sizeof(table)) || hipMalloc(&dsl, sizeof(lens))) {
        printf("  FAIL hipMalloc\n");
        return 1;
    }
    hipMemcpy(dq, q, q_n * 2, hipMemcpyHostToDevice);
    hipMemcpy(dk, k, kv_n * 2, hipMemcpyHostToDevice);
    hipMemcpy(dv, v, kv_n * 2, hipMemcpyHostToDevice);
    hipMemcpy(dbt, table, sizeof(table), hipMemcpyHostToDevice);
    hipMemcpy(dsl, lens, sizeof(lens), hipMemcpyHostToDevice);

    NxtPagedAttentionInput in;
    memset(&in, 0, sizeof(in));
    in.query = dq;
    in.key_cache = dk;
    in.value_cache = dv;
    in.block_tables = dbt;
    in.seq_lens = dsl;
    in.num_seqs = S;
    in.num_heads = H;
    in.head_size = D;
    in.num_kv_heads = KVH;
    in.scale = 1.0f / sqrtf((float)D);
    in.max_num_blocks_per_seq = MAXB;
    in.block_size = BS;
    in.dtype_size = 2;
    in.kv_block_stride = KVH * BS * D;
    in.kv_head_stride = BS * D;
    in.stream = NULL;
    CHECK(run(b, &in, dout) == 0, "run(real fp16 descriptor) == 0");
    hipDeviceSynchronize();
    hipMemcpy(o, dout, q_n * 2, hipMemcpyDeviceToHost);

    double worst = 0.0;
    for (int s = 0; s < S; s++) {
        for (int h = 0; h < H; h++) {
            const int kh = h / (H / KVH);
            double sc[64], m = -1e300, sum = 0.0, out[D];
            for (int t = 0; t < lens[s]; t++) {
                const size_t row = ((size_t)table[s * MAXB + t / BS] * KVH + kh) * BS * D + (t % BS) * D;
                double dot = 0.0;
                for (int d = 0; d < D; d++) dot += from_half(q[(s * H + h) * D + d]) * from_half(k[row + d]);
                sc[t] = dot * in.scale;
                if (sc[t] > m) m = sc[t];
            }
            for (int d = 0; d < D; d++) out[d] = 0.0;
            for (int t = 0; t < lens[s]; t++) sum += exp(sc[t] - m);
            for (int t = 0; t < lens[s]; t++) {
                const size_t row = ((size_t)table[s * MAXB + t / BS] * KVH + kh) * BS * D + (t % BS) * D;
                const double w = exp(sc[t] - m) / sum;
                for (int d = 0; d < D; d++) out[d] += w * from_half(v[row + d]);
            }
            for (int d = 0; d < D; d++) {
                const double g = from_half(o[(s * H + h) * D + d]);
                const double excess = fabs(g - out[d]) / (2e-3 + 1e-2 * fabs(out[d]));
                if (excess > worst) worst = excess;
            }
        }
    }
    printf("  worst |err| / (2e-3 + 1e-2|ref|) = %.3f\n", worst);
    CHECK(worst <= 1.0, "plugin output matches the CPU softmax within atol 2e-3 / rtol 1e-2");
    hipFree(dq); hipFree(dk); hipFree(dv); hipFree(dout); hipFree(dbt); hipFree(dsl);
    free(q); free(k); free(v); free(o);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s plugin.so [--gpu]\n", argv[0]);
        return 2;
    }
    const int gpu = argc > 2 && strcmp(argv[2], "--gpu") == 0;
    void *h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    CHECK(h != NULL, "dlopen(RTLD_NOW|RTLD_LOCAL)");
    if (!h) {
        printf("  dlerror: %s\n", dlerror());
        return 1;
    }
    InitFn init = (InitFn)dlsym(h, "nxt_backend_init");
    RunFn run = (RunFn)dlsym(h, "nxt_backend_run");
    FiniFn fini = (FiniFn)dlsym(h, "nxt_backend_fini");
    CHECK(init && run && fini, "dlsym nxt_backend_init/run/fini");
    if (!init || !run || !fini) return 1;
    /* the optional model symbols the manager resolves when it registers a
     * plugin (backend_manager.c:202-206), so the scheduler's poll can reach
     * instance_exec (scheduler.c:482-486) */
    static const char *const model_syms[] = {"nxt_model_init", "nxt_model_fini",
                                             "nxt_model_instance_init", "nxt_model_instance_fini",
                                             "nxt_model_instance_exec"};
    for (size_t i = 0; i < sizeof(model_syms) / sizeof(model_syms[0]); i++)
        CHECK(dlsym(h, model_syms[i]) != NULL, model_syms[i]);

    CHECK(init(NULL) == -1, "init(NULL) == -1");
    CHECK(fini(NULL) == -1, "fini(NULL) == -1");
    CHECK(run(NULL, NULL, NULL) == -1, "run(NULL, NULL, NULL) == -1");

    NxtBackend b;
    memset(&b, 0, sizeof(b));
    b.name = "hip_test";
    b.state = NXT_BACKEND_STATE_INITIALIZING;
    const int rc = init(&b);
    if (gpu) {
        CHECK(rc == 0, "init(valid) == 0 on the GPU");
    } else {
        CHECK(rc == 0 || rc == -1, "init(valid) returns 0 or -1");
    }
    if (rc == 0) {
        CHECK(b.state == NXT_BACKEND_STATE_READY, "state READY after init");
        CHECK(b.backend_state != NULL, "backend_state set after init");
        CHECK(run(&b, NULL, NULL) == -1, "run(b, NULL, NULL) == -1");
        int dummy_input = 0xDEAD, dummy_output = 0;
        CHECK(run(&b, &dummy_input, &dummy_output) == -1, "garbage descriptor refused with -1");
        if (gpu) real_decode(run, &b);
    } else {
        CHECK(b.state == NXT_BACKEND_STATE_ERROR, "state ERROR after a failed init");
        CHECK(b.backend_state == NULL, "no backend_state after a failed init");
        CHECK(run(&b, NULL, NULL) == -1, "run on an uninitialised backend == -1");
    }
    CHECK(fini(&b) == 0, "fini(b) == 0");
    CHECK(b.state == NXT_BACKEND_STATE_UNINITIALIZED, "state UNINITIALIZED after fini");
    CHECK(b.backend_state == NULL, "backend_state NULL after fini");
    CHECK(fini(&b) == 0, "double fini == 0");
    CHECK(dlclose(h) == 0, "dlclose");
    printf("%s (%d failure%s)\n", failures ? "FAILED" : "PASSED", failures, failures == 1 ? "" : "s");
    return failures ? 1 : 0;
}
