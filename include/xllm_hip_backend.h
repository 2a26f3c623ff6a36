/*
 * xLLM HIP backend plugin (libxllm_hip_backend.so) -- plugin C-ABI.
 *
 * Drop-in for the reference's CUDA backend plugin
 * (backends/cuda_backend.h:22-51, backends/cuda_backend.c:35-120): the
 * reference backend manager dlopen()s the .so (src/core/backend_manager.c:274,
 * RTLD_NOW|RTLD_LOCAL) and dlsym()s nxt_backend_init / nxt_backend_run /
 * nxt_backend_fini (:283-285), then drives them unchanged.
 *
 * Conventions kept from the reference plugin (pinned by its
 * tests/test_backend_load.c:83-163 and tests/test_backend.c:271-307):
 *   init(NULL) -> -1; init(b) -> 0, b->backend_state != NULL, b->state READY;
 *   run(NULL, ..) or a NULL input/output -> -1; run success -> 0;
 *   fini(NULL) -> -1; fini(b) frees the state, sets backend_state NULL and
 *   state UNINITIALIZED; a second fini returns 0.
 * Additions: run() validates the descriptor before launching (the reference
 * passes a 4-byte int as `input` in test_backend_load.c:116-118) and returns
 * -1 on a bad descriptor or launch failure; init() returns -1 (state ERROR)
 * when no HIP device is usable.
 *
 * Types: when the includer already has the reference's include/backend.h
 * (XLLM_BACKEND_H) or backends/cuda_backend.h (XLLM_CUDA_BACKEND_H), their
 * definitions are used; otherwise layout-identical mirrors are defined here.
 * Never include this header together with the manager-side prototype
 * `int nxt_backend_run(const char*, void*, void*)` (include/backend.h:211):
 * the plugin's symbol shares that name (cuda_backend.c:12-14 renames the
 * manager's one with a #define for the same reason).
 */
#ifndef XLLM_HIP_BACKEND_H_
#define XLLM_HIP_BACKEND_H_

#include <stdint.h>

#include "xllm_hip_operator_api.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef XLLM_BACKEND_H
/* Mirror of include/backend.h:35-41. */
typedef enum {
    NXT_BACKEND_STATE_UNINITIALIZED = 0,
    NXT_BACKEND_STATE_INITIALIZING = 1,
    NXT_BACKEND_STATE_READY = 2,
    NXT_BACKEND_STATE_ERROR = 3,
    NXT_BACKEND_STATE_UNLOADING = 4,
} NxtBackendState;

typedef struct NxtBackend NxtBackend;

/* Mirror of include/backend.h:128-137: eight function pointers (64 bytes on
 * LP64).  Only the first three are resolved from this plugin. */
typedef struct NxtBackendAPI {
    int (*backend_init)(NxtBackend *backend);
    int (*backend_run)(NxtBackend *backend, void *input, void *output);
    int (*backend_fini)(NxtBackend *backend);
    void *model_init;
    void *model_fini;
    void *instance_init;
    void *instance_fini;
    void *instance_exec;
} NxtBackendAPI;

/* Mirror of include/backend.h:141-151; offsets as documented by the
 * reference's tests/mock_cuda_backend.c:26-37 (name 0, so_path 8,
 * dl_handle 16, api 24, state 88, priority 92, model_count 96, models 104,
 * backend_state 112; sizeof 120). */
struct NxtBackend {
    char *name;
    char *so_path;
    void *dl_handle;
    NxtBackendAPI api;
    NxtBackendState state;
    int32_t priority;
    uint32_t model_count;
    void *models;
    void *backend_state;
};
#endif /* XLLM_BACKEND_H */

#ifndef XLLM_CUDA_BACKEND_H
/* Mirror of backends/cuda_backend.h:29-46 (sizeof 88 on LP64, scale at 56,
 * stream at 80): the `input` of nxt_backend_run; `output` is the device
 * [num_seqs][num_heads][head_size] result. */
typedef struct {
    const void *query;
    const void *key_cache;
    const void *value_cache;
    const int *block_tables;
    const int *seq_lens;
    int num_seqs;
    int num_heads;
    int head_size;
    int num_kv_heads;
    float scale;
    int max_num_blocks_per_seq;
    int block_size;
    int dtype_size;
    int kv_block_stride;
    int kv_head_stride;
    nxt_stream_t stream;
} NxtPagedAttentionInput;
#endif /* XLLM_CUDA_BACKEND_H */

/* Versioned descriptor for nxt_backend_run_ex (no counterpart in the
 * reference): the reference fields first, in the same order, then the dtype
 * code and the split-K partition length.  struct_size must be set to
 * sizeof(NxtPagedAttentionInputEx); later versions only append fields. */
typedef struct {
    uint32_t struct_size;
    uint32_t reserved;
    NxtPagedAttentionInput base;
    int kv_dtype;          /* NxtKvDtype */
    int partition_tokens;  /* 0 = automatic */
} NxtPagedAttentionInputEx;

/* Replace backends/cuda_backend.h:49-51 (cuda_backend.c:35, :71, :108). */
int nxt_backend_init(NxtBackend *backend);
int nxt_backend_run(NxtBackend *backend, void *input, void *output);
int nxt_backend_fini(NxtBackend *backend);

/* Additive: run with an explicit dtype (bf16) and partition length. */
int nxt_backend_run_ex(NxtBackend *backend, const NxtPagedAttentionInputEx *input,
                       void *output);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_BACKEND_H_ */
