/*
 * Library-internal workspace control, shared by the plugin (hip_backend.c),
 * the model instance (model_instance.cpp) and the operator layer
 * (paged_decode_api.cpp), which owns the workspace cache.  Hidden symbols:
 * not part of the exported C-ABI.
 */
#ifndef XLLM_HIP_WORKSPACE_H
#define XLLM_HIP_WORKSPACE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Tags the workspaces this host thread allocates from now on with `owner`
 * (NULL: no owner); returns the previous tag.  The plugin brackets each run
 * with it, so its fini releases exactly what its runs allocated. */
__attribute__((visibility("hidden"))) const void *xhip_set_workspace_owner(const void *owner);

/* Frees the workspaces allocated under `owner`, after waiting for their
 * devices.  Returns 0, or -1 when a device wait failed. */
__attribute__((visibility("hidden"))) int xhip_release_owner_workspaces(const void *owner);

/* Frees every workspace of one stream handle on one device (all kinds and
 * threads), after waiting for the device: for a caller about to destroy
 * that stream.  Returns 0, or -1 when the device wait failed. */
__attribute__((visibility("hidden"))) int xhip_release_stream_workspaces(int device, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_WORKSPACE_H */
