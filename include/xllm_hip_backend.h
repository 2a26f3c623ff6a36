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

#include <stdbool.h>
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
typedef struct NxtModel NxtModel;
typedef struct NxtModelInstance NxtModelInstance;
typedef struct NxtInferRequest NxtInferRequest;

/* Mirrors of include/backend.h:13-33, 54-62, 66-113 and 155-189 (layouts as
 * the reference compiler lays them out on LP64: NxtTensor 48 bytes,
 * NxtModelConfig 120, NxtModel 168, NxtModelInstance 48, NxtInferRequest 56;
 * asserted in tests/c/layout_check.c). */
typedef enum {
    NXT_TYPE_BOOL = 1,
    NXT_TYPE_UINT8 = 2,
    NXT_TYPE_UINT16 = 3,
    NXT_TYPE_UINT32 = 4,
    NXT_TYPE_UINT64 = 5,
    NXT_TYPE_INT8 = 6,
    NXT_TYPE_INT16 = 7,
    NXT_TYPE_INT32 = 8,
    NXT_TYPE_INT64 = 9,
    NXT_TYPE_FP16 = 10,
    NXT_TYPE_FP32 = 11,
    NXT_TYPE_FP64 = 12,
    NXT_TYPE_BYTES = 13,
} NxtDataType;

typedef enum {
    NXT_MEM_CPU = 0,
    NXT_MEM_GPU = 1,
    NXT_MEM_CPU_PINNED = 2,
} NxtMemoryType;

typedef struct {
    const char *name;
    NxtDataType dtype;
    int64_t *shape;
    uint32_t dims_count;
    uint64_t byte_size;
    NxtMemoryType memory_type;
    int32_t memory_type_id;
} NxtTensor;

typedef enum {
    NXT_INSTANCE_KIND_GPU = 0,
    NXT_INSTANCE_KIND_CPU = 1,
} NxtInstanceKind;

typedef struct {
    uint32_t count;
    NxtInstanceKind kind;
    int32_t *gpus;
    uint32_t gpus_count;
} NxtInstanceGroup;

typedef struct {
    int policy; /* NxtVersionPolicy */
    uint32_t num_versions;
    int32_t *versions;
    uint32_t versions_count;
} NxtModelVersionConfig;

typedef struct {
    float preferred_batch_size_ratio;
    double max_queue_delay_ms;
    bool preserve_ordering;
    int32_t priority_levels;
} NxtDynamicBatchingConfig;

typedef struct {
    char *name;
    char *backend_name;
    char *model_path;
    int32_t max_batch_size;
    uint32_t input_count;
    NxtTensor **inputs;
    uint32_t output_count;
    NxtTensor **outputs;
    uint32_t instance_group_count;
    NxtInstanceGroup *instance_groups;
    NxtModelVersionConfig version_config;
    NxtDynamicBatchingConfig dynamic_batching;
} NxtModelConfig;

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
    NxtModel *models;
    void *backend_state;
};

struct NxtModel {
    char *name;
    int32_t version;
    NxtModelConfig config;
    NxtBackend *backend;
    NxtModelInstance *instances;
    uint32_t instance_count;
    NxtBackendState state;
    void *backend_state;
};

struct NxtModelInstance {
    NxtModel *model;
    char *name;
    NxtInstanceKind kind;
    int32_t device_id;
    void *instance_state;
    uint64_t exec_count;
    double total_exec_ms;
};

struct NxtInferRequest {
    const char *request_id;
    uint32_t batch_size;
    uint32_t input_count;
    NxtTensor *inputs;
    uint32_t requested_output_count;
    char **requested_output_names;
    uint64_t enqueue_time_ns;
    int32_t priority;
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

/* ------------------------------------------------ models and instances
 * The optional plugin symbols the reference manager resolves
 * (src/core/backend_manager.c:202-206), so that its scheduler's poll
 * (src/core/scheduler.c:477-488: instance_exec(model->instances, &request, 1)
 * for each scheduled request) reaches the decode path.
 *
 * nxt_model_init(model) is called by nxt_model_create
 * (backend_manager.c:389-398).  It reads the decode geometry from
 * model->config.inputs by name:
 *   "key_cache"     4 dims [num_blocks, num_kv_heads, block_size, head_size];
 *                   dtype NXT_TYPE_FP16, NXT_TYPE_FP32 or NXT_TYPE_BF16_HIP;
 *   "query"         2 dims [num_heads, head_size];
 *   "block_tables"  optional, 2 dims [*, max_blocks_per_seq] (default: every
 *                   page of the cache);
 * and model->config.max_batch_size (requests per exec, default 256).  It
 * creates one instance on the current HIP device (the reference creates
 * none, so model->instances would stay NULL), which holds the paged K/V
 * caches in HBM and the KV-cache index (xllm_hip_kv_index.h) of its
 * sequences.  Scale: 1/sqrt(head_size), as text_gen.c:732.
 *
 * A request carries no data pointers (NxtTensor has none), so its buffers
 * are bound by request_id before the exec that consumes them
 * (nxt_model_instance_bind).  exec then, for the batch of requests:
 *   1. admits a request seen for the first time with its tokens (prompt
 *      prefix matched against the cached sequences: shared pages reused,
 *      a partly matched page copied) or appends the tokens of a known one;
 *   2. writes the K/V rows of every new token that is not cached (one
 *      launch for the batch);
 *   3. runs the decode attention for the requests with a query (the
 *      prefix-aware form when the batch has shared prefixes) and writes each
 *      output;
 *   4. ends the requests marked release (their tokens stay in the tree for
 *      later prompts until evicted).
 * It returns when the device work is done (0), or -1 on an unbound request,
 * a bad binding or an exhausted cache; requests before the failing one stay
 * applied.  Bindings are consumed by the exec.  Not thread-safe. */
#define NXT_TYPE_BF16_HIP 256 /* bfloat16: no code in the reference's NxtDataType */

typedef struct {
    uint32_t struct_size;     /* sizeof(NxtDecodeIo) */
    int32_t num_tokens;       /* new tokens of the request (its prompt the first time) */
    const int32_t *token_ids; /* host [num_tokens] */
    const void *key;          /* device [num_tokens][num_kv_heads][head_size], cache dtype */
    const void *value;
    const void *query;        /* device [num_heads][head_size] of the last token, or NULL */
    void *output;             /* device [num_heads][head_size] (with query) */
    int32_t release;          /* end the request after this exec */
    int32_t reserved;
} NxtDecodeIo;

int nxt_model_init(NxtModel *model);
int nxt_model_fini(NxtModel *model);
int nxt_model_instance_init(NxtModelInstance *instance);
int nxt_model_instance_fini(NxtModelInstance *instance);
int nxt_model_instance_exec(NxtModelInstance *instance, NxtInferRequest **requests,
                            uint32_t request_count);
/* Additive: bind the buffers of the next exec of request_id (the
 * descriptor and its token ids are copied). */
int nxt_model_instance_bind(NxtModelInstance *instance, const char *request_id,
                            const NxtDecodeIo *io);

/* Additive, no counterpart in the reference: deferred execution, for the
 * reference scheduler's call pattern.  Its poll issues one
 * instance_exec(instance, &request, 1) per scheduled request
 * (scheduler.c:477-488), which as synchronous execs is one host-waited
 * decode launch sequence per request.  With deferred mode on, exec checks
 * the requests and queues them, returning 0; the queue runs as one
 * whole-batch exec (the steps above, one wait) when it is flushed:
 *   - by nxt_model_instance_flush, or an exec with request_count 0;
 *   - when a queued request is bound again or executed again (its next
 *     step began), before that bind or exec;
 *   - when the queue holds max_batch_size requests;
 *   - when deferred mode is switched off, and by nxt_model_instance_fini.
 * Outputs of queued requests are ready once the flush that ran them has
 * returned; its return value is the batch's (0, or -1 as for exec).
 * set_deferred returns 0, or the flush's status when switching off.  Off
 * by default: exec then runs and waits as above. */
int nxt_model_instance_set_deferred(NxtModelInstance *instance, int on);
int nxt_model_instance_flush(NxtModelInstance *instance);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_BACKEND_H_ */
