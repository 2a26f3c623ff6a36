/*
 * xLLM HIP backend plugin: nxt_backend_init / run / fini for MI355X.
 *
 * Replaces backends/cuda_backend.c:35-120 of the reference behind the same
 * dlopen ABI (resolved by src/core/backend_manager.c:283-285).  run() takes
 * the reference's NxtPagedAttentionInput (backends/cuda_backend.h:29-46) and
 * launches the paged-decode attention through nxt_paged_attention_ex, the C
 * entry point of the gfx950 kernels in the same shared object.
 *
 * Differences from the reference plugin, all stricter:
 *   - init() requires a usable gfx950 device (the kernels are built for that
 *     target only); otherwise it returns -1 and leaves the state ERROR.
 *   - run() checks the descriptor before launching: dtype_size, sizes, and
 *     that every tensor pointer is device memory (hipPointerGetAttributes), so
 *     a garbage descriptor (tests/test_backend_load.c:116-118 passes a 4-byte
 *     int) is refused with -1 instead of being launched.
 *   - fini() waits for the device and releases the split-K workspaces that
 *     this backend's runs allocated (not those of other backends, model
 *     instances or direct operator callers in the same process).
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "workspace.h"
#include "xllm_hip_backend.h"

#define XHIP_EXPORT __attribute__((visibility("default")))
#define XHIP_STATE_MAGIC 0x58484950u /* "XHIP" */

typedef struct {
    uint32_t magic;
    int device_id;
    int cu_count;
    char device_name[256];
    char arch_name[64];
    unsigned long long runs;
    unsigned long long failures;
} HipBackendState;

static int is_device_pointer(const void *ptr) {
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof(attr));
    if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
        (void)hipGetLastError(); /* clear the sticky error of the failed query */
        return 0;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

XHIP_EXPORT int nxt_backend_init(NxtBackend *backend) {
    if (!backend) return -1;

    HipBackendState *st = (HipBackendState *)calloc(1, sizeof(*st));
    if (!st) return -1;
    st->magic = XHIP_STATE_MAGIC;

    hipError_t err = hipGetDevice(&st->device_id);
    if (err != hipSuccess) {
        fprintf(stderr, "[hip_backend] hipGetDevice failed: %s\n", hipGetErrorString(err));
        free(st);
        backend->state = NXT_BACKEND_STATE_ERROR;
        return -1;
    }
    hipDeviceProp_t props;
    memset(&props, 0, sizeof(props));
    err = hipGetDeviceProperties(&props, st->device_id);
    if (err != hipSuccess) {
        fprintf(stderr, "[hip_backend] hipGetDeviceProperties failed: %s\n",
                hipGetErrorString(err));
        free(st);
        backend->state = NXT_BACKEND_STATE_ERROR;
        return -1;
    }
    st->cu_count = props.multiProcessorCount;
    snprintf(st->device_name, sizeof(st->device_name), "%.255s", props.name);
    snprintf(st->arch_name, sizeof(st->arch_name), "%.63s", props.gcnArchName);
    if (strncmp(st->arch_name, "gfx950", 6) != 0) {
        fprintf(stderr, "[hip_backend] device %d is %s; this plugin is built for gfx950 only\n",
                st->device_id, st->arch_name);
        free(st);
        backend->state = NXT_BACKEND_STATE_ERROR;
        return -1;
    }

    backend->backend_state = st;
    backend->state = NXT_BACKEND_STATE_READY;
    fprintf(stderr, "[hip_backend] initialized device=%d cu=%d gpu=%s arch=%s (%s)\n",
            st->device_id, st->cu_count, st->device_name, st->arch_name, nxt_attn_version());
    return 0;
}

/* Shared by run() and run_ex(): check the descriptor, then launch. */
static int launch(HipBackendState *st, const NxtPagedAttentionInput *pa, void *output,
                  int kv_dtype, int partition_tokens) {
    if (pa->num_seqs < 0 || pa->num_heads <= 0 || pa->num_kv_heads <= 0 ||
        pa->head_size <= 0 || pa->block_size <= 0 || pa->max_num_blocks_per_seq <= 0) {
        fprintf(stderr, "[hip_backend] run: bad sizes in input descriptor\n");
        return -1;
    }
    if (pa->num_seqs > 0) {
        const void *ptrs[6] = {output, pa->query, pa->key_cache, pa->value_cache,
                               pa->block_tables, pa->seq_lens};
        for (int i = 0; i < 6; i++) {
            if (!ptrs[i] || !is_device_pointer(ptrs[i])) {
                fprintf(stderr, "[hip_backend] run: tensor %d is not device memory\n", i);
                return -1;
            }
        }
    }
    /* the workspaces this run allocates belong to this backend (its fini
     * frees them, and no other backend's) */
    const void *prev_owner = xhip_set_workspace_owner(st);
    int rc = nxt_paged_attention_ex(output, pa->query, pa->key_cache, pa->value_cache,
                                    pa->block_tables, pa->seq_lens, pa->num_seqs, pa->num_heads,
                                    pa->head_size, pa->num_kv_heads, pa->scale,
                                    pa->max_num_blocks_per_seq, pa->block_size, pa->dtype_size,
                                    pa->kv_block_stride, pa->kv_head_stride, pa->stream, kv_dtype,
                                    partition_tokens);
    (void)xhip_set_workspace_owner(prev_owner);
    st->runs++;
    if (rc != NXT_ATTN_OK) {
        st->failures++;
        fprintf(stderr, "[hip_backend] run: %s\n", nxt_attn_last_error());
        return -1;
    }
    return 0;
}

static HipBackendState *state_of(NxtBackend *backend) {
    if (!backend || !backend->backend_state) return NULL;
    HipBackendState *st = (HipBackendState *)backend->backend_state;
    return st->magic == XHIP_STATE_MAGIC ? st : NULL;
}

XHIP_EXPORT int nxt_backend_run(NxtBackend *backend, void *input, void *output) {
    HipBackendState *st = state_of(backend);
    if (!st) return -1;
    if (!input || !output) return -1;
    const NxtPagedAttentionInput *pa = (const NxtPagedAttentionInput *)input;
    int kv_dtype;
    if (pa->dtype_size == 2)
        kv_dtype = NXT_KV_FP16;
    else if (pa->dtype_size == 4)
        kv_dtype = NXT_KV_FP32;
    else {
        fprintf(stderr, "[hip_backend] run: dtype_size %d is not 2 or 4\n", pa->dtype_size);
        return -1;
    }
    return launch(st, pa, output, kv_dtype, 0);
}

XHIP_EXPORT int nxt_backend_run_ex(NxtBackend *backend, const NxtPagedAttentionInputEx *input,
                                   void *output) {
    HipBackendState *st = state_of(backend);
    if (!st) return -1;
    if (!input || !output) return -1;
    if (input->struct_size < sizeof(NxtPagedAttentionInputEx)) {
        fprintf(stderr, "[hip_backend] run_ex: struct_size %u < %zu\n", input->struct_size,
                sizeof(NxtPagedAttentionInputEx));
        return -1;
    }
    return launch(st, &input->base, output, input->kv_dtype, input->partition_tokens);
}

XHIP_EXPORT int nxt_backend_fini(NxtBackend *backend) {
    if (!backend) return -1;
    HipBackendState *st = (HipBackendState *)backend->backend_state;
    if (st) {
        fprintf(stderr, "[hip_backend] unloading device=%d runs=%llu failures=%llu\n",
                st->device_id, st->runs, st->failures);
        /* after a wait for the device: only what this backend's runs allocated */
        (void)xhip_release_owner_workspaces(st);
        free(st);
        backend->backend_state = NULL;
    }
    backend->state = NXT_BACKEND_STATE_UNINITIALIZED;
    return 0;
}
