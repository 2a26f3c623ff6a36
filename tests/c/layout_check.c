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

int main(void) { return 0; }
