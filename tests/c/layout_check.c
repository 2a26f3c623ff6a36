/* Compile-time check that the plugin ABI mirrors of include/xllm_hip_backend.h
 * have the reference's layouts (include/backend.h:128-151,
 * backends/cuda_backend.h:29-46, offsets per tests/mock_cuda_backend.c:26-37). */
#include <stddef.h>

#include "xllm_hip_backend.h"

_Static_assert(sizeof(NxtBackendAPI) == 64, "NxtBackendAPI is 8 pointers");
_Static_assert(offsetof(NxtBackend, name) == 0, "name");
_Static_assert(offsetof(NxtBackend, so_path) == 8, "so_path");
_Static_assert(offsetof(NxtBackend, dl_handle) == 16, "dl_handle");
_Static_assert(offsetof(NxtBackend, api) == 24, "api");
_Static_assert(offsetof(NxtBackend, state) == 88, "state");
_Static_assert(offsetof(NxtBackend, priority) == 92, "priority");
_Static_assert(offsetof(NxtBackend, model_count) == 96, "model_count");
_Static_assert(offsetof(NxtBackend, models) == 104, "models");
_Static_assert(offsetof(NxtBackend, backend_state) == 112, "backend_state");
_Static_assert(sizeof(NxtBackend) == 120, "sizeof NxtBackend");
_Static_assert(sizeof(NxtPagedAttentionInput) == 88, "sizeof NxtPagedAttentionInput");
_Static_assert(offsetof(NxtPagedAttentionInput, scale) == 56, "scale");
_Static_assert(offsetof(NxtPagedAttentionInput, stream) == 80, "stream");
_Static_assert(offsetof(NxtPagedAttentionInputEx, base) == 8, "Ex.base");
_Static_assert(sizeof(NxtPagedAttentionInputEx) == 104, "sizeof NxtPagedAttentionInputEx");

/* include/backend.h:54-189, offsets as the reference header compiles (an
 * offsetof probe over the reference's own include/backend.h). */
_Static_assert(sizeof(NxtTensor) == 48, "sizeof NxtTensor");
_Static_assert(offsetof(NxtTensor, shape) == 16, "NxtTensor.shape");
_Static_assert(offsetof(NxtTensor, byte_size) == 32, "NxtTensor.byte_size");
_Static_assert(offsetof(NxtTensor, memory_type_id) == 44, "NxtTensor.memory_type_id");
_Static_assert(sizeof(NxtModelConfig) == 120, "sizeof NxtModelConfig");
_Static_assert(offsetof(NxtModelConfig, max_batch_size) == 24, "config.max_batch_size");
_Static_assert(offsetof(NxtModelConfig, inputs) == 32, "config.inputs");
_Static_assert(offsetof(NxtModelConfig, instance_groups) == 64, "config.instance_groups");
_Static_assert(offsetof(NxtModelConfig, version_config) == 72, "config.version_config");
_Static_assert(offsetof(NxtModelConfig, dynamic_batching) == 96, "config.dynamic_batching");
_Static_assert(sizeof(NxtModel) == 168, "sizeof NxtModel");
_Static_assert(offsetof(NxtModel, config) == 16, "model.config");
_Static_assert(offsetof(NxtModel, backend) == 136, "model.backend");
_Static_assert(offsetof(NxtModel, instances) == 144, "model.instances");
_Static_assert(offsetof(NxtModel, instance_count) == 152, "model.instance_count");
_Static_assert(offsetof(NxtModel, state) == 156, "model.state");
_Static_assert(offsetof(NxtModel, backend_state) == 160, "model.backend_state");
_Static_assert(sizeof(NxtModelInstance) == 48, "sizeof NxtModelInstance");
_Static_assert(offsetof(NxtModelInstance, instance_state) == 24, "instance.instance_state");
_Static_assert(offsetof(NxtModelInstance, total_exec_ms) == 40, "instance.total_exec_ms");
_Static_assert(sizeof(NxtInferRequest) == 56, "sizeof NxtInferRequest");
_Static_assert(offsetof(NxtInferRequest, inputs) == 16, "request.inputs");
_Static_assert(offsetof(NxtInferRequest, enqueue_time_ns) == 40, "request.enqueue_time_ns");
_Static_assert(offsetof(NxtInferRequest, priority) == 48, "request.priority");
_Static_assert(sizeof(NxtDecodeIo) == 56, "sizeof NxtDecodeIo");

int main(void) { return 0; }
