/*
 * xLLM paged-decode attention for AMD MI355X (gfx950) -- operator C-ABI.
 *
 * Drop-in for the paged-attention part of the reference's operator API
 * (include/operator_api.h:29-116 of ahua2020qq/xLLMs): same symbol names, same
 * argument order and meaning, `void*` tensors, opaque stream.  All three
 * reference entry points map to ONE implementation (hand-written gfx950
 * kernels in libxllm_hip_backend.so); there is no per-entry-point kernel
 * family and no multi-backend dispatch.
 *
 * Semantics (what every entry point computes), with G = num_heads/num_kv_heads:
 *   for s < num_seqs, h < num_heads, L = seq_lens[s]:
 *     O[s,h,:] = sum_{t<L} softmax_t(scale * <Q[s,h,:], K_t>) * V_t
 *   where K_t / V_t is row (t % block_size) of kv head h/G in physical block
 *   block_tables[s*max_num_blocks_per_seq + t/block_size], i.e. at element
 *   offset blk*kv_block_stride + (h/G)*kv_head_stride + (t%block_size)*head_size.
 *   Q and O are [num_seqs][num_heads][head_size].  Arithmetic is fp32; O is
 *   written in the input dtype.
 * Contract points the reference leaves undefined, fixed here:
 *   - seq_lens[s] <= 0 writes a zero row; seq_lens[s] is clamped to
 *     max_num_blocks_per_seq*block_size.
 *   - block-table entries are read only for t < L; a negative entry is never
 *     dereferenced and its tokens contribute nothing.
 *   - K/V slots past L in the last block are never read (they may hold NaN).
 *   - Unsupported shapes never compute a wrong size silently: the call does
 *     nothing on the device and records an error, readable through
 *     nxt_attn_last_status()/nxt_attn_last_error() on the calling thread.
 * Supported: head_size in {32,64,80,96,112,128,192,256}; num_heads %
 * num_kv_heads == 0 with G <= 64 for fp16/bf16 at head_size % 32 == 0 and
 * block_size >= 16, else G <= 32; block_size a power of two in [1, 1024];
 * max_num_blocks_per_seq*block_size <= 2^28; 16-byte aligned tensors and
 * strides (every real KV cache layout).
 *
 * Calls are asynchronous on `stream` (NULL = the default stream) and never
 * synchronise, except the rare call that must grow the split-K workspace of
 * that stream, which first waits for the stream.  Threads: the library keeps
 * one workspace per (device, stream queue); a call holds it from lookup until
 * its launches are enqueued, so calls from several host threads on one
 * stream handle are enqueued one after the other, calls on different streams
 * are independent, and hipStreamPerThread gets one workspace per thread.
 * Do not destroy a stream while calls on it are pending.
 */
#ifndef XLLM_HIP_OPERATOR_API_H_
#define XLLM_HIP_OPERATOR_API_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef XLLM_OPERATOR_API_H_
/* Opaque stream handle: a hipStream_t.  Same type as the reference's
 * include/operator_api.h:29. */
typedef void *nxt_stream_t;
#endif

/* Replaces nxt_paged_attention, include/operator_api.h:63-72 (implemented
 * there by operators/page_attention.cu:170-322).  dtype_size 2 = fp16,
 * 4 = fp32, as the reference header documents (operator_api.h:14-16, :59). */
void nxt_paged_attention(void *out, const void *query, const void *key_cache,
                         const void *value_cache, const int *block_tables,
                         const int *seq_lens, int num_seqs, int num_heads, int head_size,
                         int num_kv_heads, float scale, int max_num_blocks_per_seq,
                         int block_size, int dtype_size, int kv_block_stride,
                         int kv_head_stride, nxt_stream_t stream);

/* Replaces nxt_paged_attention_v2, include/operator_api.h:84-93 (implemented
 * there by operators/page_attention_v2.cu:262-348).  Same computation. */
void nxt_paged_attention_v2(void *out, const void *query, const void *key_cache,
                            const void *value_cache, const int *block_tables,
                            const int *seq_lens, int num_seqs, int num_heads,
                            int head_size, int num_kv_heads, float scale,
                            int max_num_blocks_per_seq, int block_size, int dtype_size,
                            int kv_block_stride, int kv_head_stride, nxt_stream_t stream);

/* Replaces nxt_paged_attention_flash, include/operator_api.h:106-115
 * (implemented there by operators/flashinfer_adapter.cu:329-433, only under
 * USE_FLASHINFER).  Exported unconditionally; same computation. */
void nxt_paged_attention_flash(void *out, const void *query, const void *key_cache,
                               const void *value_cache, const int *block_tables,
                               const int *seq_lens, int num_seqs, int num_heads,
                               int head_size, int num_kv_heads, float scale,
                               int max_num_blocks_per_seq, int block_size,
                               int dtype_size, int kv_block_stride, int kv_head_stride,
                               nxt_stream_t stream);

/* ---- Additive extensions (no counterpart in the reference) -------------- */

/* KV / query / output element type.  The reference's dtype_size cannot name
 * bf16 (operator_api.h:14-16; NxtDataType in include/backend.h:13-27 has no
 * BF16), so the extended entry point takes an explicit code. */
typedef enum {
    NXT_KV_FP16 = 1,
    NXT_KV_BF16 = 2,
    NXT_KV_FP32 = 3,
} NxtKvDtype;

/* Status codes returned by the extended entry points and recorded for the
 * void ones. */
enum {
    NXT_ATTN_OK = 0,
    NXT_ATTN_E_INVALID = -1,     /* NULL pointer / negative or inconsistent size */
    NXT_ATTN_E_UNSUPPORTED = -2, /* head_size, group, block_size, alignment     */
    NXT_ATTN_E_HIP = -3,         /* HIP runtime / launch failure                */
    NXT_ATTN_E_NOMEM = -4,       /* split-K workspace allocation failed         */
};

/* Same computation as nxt_paged_attention, with the dtype named explicitly
 * (dtype_size must agree: 2 for FP16/BF16, 4 for FP32) and the split-K
 * granularity: partition_tokens = 0 lets the library spread the batch
 * evenly over one resident round of wavefronts; otherwise it is the token
 * range each wavefront streams (a power of two >= the kernel tile, 16 tokens
 * for fp16/bf16 head_size 128), e.g. to check that results do not depend on
 * where sequences are cut.  Returns NXT_ATTN_OK or a negative status.
 * Graph capture: the split-K workspace is the library's, per (device,
 * stream); a captured call holds its address, so the library keeps every
 * buffer a capture used alive (a later larger call on the stream allocates
 * a new one beside it) until nxt_attn_release_workspaces().  A call under
 * capture that would need a larger workspace than its stream has returns
 * NXT_ATTN_E_UNSUPPORTED without launching: make one call of the shape on
 * that stream before capturing. */
int nxt_paged_attention_ex(void *out, const void *query, const void *key_cache,
                           const void *value_cache, const int *block_tables,
                           const int *seq_lens, int num_seqs, int num_heads,
                           int head_size, int num_kv_heads, float scale,
                           int max_num_blocks_per_seq, int block_size, int dtype_size,
                           int kv_block_stride, int kv_head_stride, nxt_stream_t stream,
                           int kv_dtype, int partition_tokens);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, checks and result as
 * nxt_paged_attention_ex, but the split-K partials live in a fixed per-device
 * scratch array of 66 MiB that the library holds until the process ends,
 * instead of the library's per-stream workspace: the call makes no hipMalloc
 * or hipFree.  Every automatic plan (partition_tokens = 0) fits on a 256-CU
 * MI355X, so results equal nxt_paged_attention_ex's bit for bit (on a
 * device with more CUs an automatic plan is cut to fewer wavefronts to fit:
 * correct, but not bit-identical); a plan that needs more scratch (an
 * explicit partition_tokens over a large batch) returns
 * NXT_ATTN_E_UNSUPPORTED without launching.  Every call on one device
 * shares that device's scratch, so the library orders them on the GPU: a
 * call's stream waits for the device's previous no-alloc call (an event
 * recorded after it; the first call on a device creates that event) unless
 * that call went to the same queue.  The host does not block.  A call made
 * while its stream is being captured goes into the caller's graph unordered:
 * replays of graphs that hold no-alloc calls must not overlap one another or
 * eager no-alloc calls on the same device (replay them on one stream, or
 * wait for them). */
int nxt_paged_attention_noalloc(void *out, const void *query, const void *key_cache,
                                const void *value_cache, const int *block_tables,
                                const int *seq_lens, int num_seqs, int num_heads,
                                int head_size, int num_kv_heads, float scale,
                                int max_num_blocks_per_seq, int block_size, int dtype_size,
                                int kv_block_stride, int kv_head_stride, nxt_stream_t stream,
                                int kv_dtype, int partition_tokens);

/* Wavefronts the automatic split-K plan launches for this shape (needs a
 * current HIP device for its CU count and the kernel occupancy), or a
 * negative status. */
int nxt_paged_attention_auto_waves(int num_seqs, int num_heads, int head_size,
                                   int num_kv_heads, int max_num_blocks_per_seq,
                                   int block_size, int kv_dtype);

/* Status and message of the last paged-attention call made by this thread. */
int nxt_attn_last_status(void);
const char *nxt_attn_last_error(void);

/* Profiling hook: when set, every later launch from the calling thread
 * stamps `start_event` and `partition_done_event` (hipEvent_t handles owned
 * by the caller) with the start and the end of its partition kernel, on the
 * stream it runs on (hipExtLaunchKernel's kernel events), so the kernel can
 * be timed without event packets queued around it.  NULL, NULL clears the
 * hook.  Meant for benchmarks and tracing. */
void nxt_attn_set_trace_events(void *start_event, void *partition_done_event);

/* Waits for and frees every cached split-K and cascade workspace of this
 * process, including the ones kept alive for captured graphs: call it only
 * when no graph captured over an allocating entry point runs again.  The
 * library also frees a stream's workspaces when it evicts the least
 * recently used of more than 64 (device, stream) entries, and the
 * hipStreamPerThread workspaces of a thread when that thread exits. */
int nxt_attn_release_workspaces(void);

/* Library version string, e.g. "xllm-hip-attn 0.1.0 gfx950". */
const char *nxt_attn_version(void);

/* ------------------------------------------------ prefix-aware (cascade) decode
 * No counterpart in the reference: its decode reads every sequence's pages
 * even where sequences share them (radix-shared prefixes,
 * src/core/prefix_sharing.c).  Same result as nxt_paged_attention_ex (same
 * arguments and layouts, within the dtype's rounding), but the pages of a
 * shared prefix are read once per 32 (sequence, query head) rows of the
 * sequences that share them (16 for fp32 or head_size > 128) instead of
 * once per sequence.
 *   prefix_group[num_seqs]  device int32: group of each sequence, -1 = none
 *   prefix_blocks[max_groups] device int32: the number of leading pages (full
 *                           pages, block_size tokens each) that every member
 *                           of the group has in common, same physical ids.
 * A sequence whose entry does not fit (group id out of range, a prefix
 * longer than its table or its length) is decoded without sharing.
 * max_groups = 0 is the ordinary decode.  num_seqs <= 8192, max_groups <=
 * num_seqs.  Allocates (once, per stream) a workspace for its plan and the
 * fp32 pass outputs; asynchronous on `stream`. */
int nxt_paged_attention_cascade(void *out, const void *query, const void *key_cache,
                                const void *value_cache, const int *block_tables,
                                const int *seq_lens, const int *prefix_group,
                                const int *prefix_blocks, int max_groups, int num_seqs,
                                int num_heads, int head_size, int num_kv_heads, float scale,
                                int max_num_blocks_per_seq, int block_size, int kv_block_stride,
                                int kv_head_stride, int kv_dtype, nxt_stream_t stream);

/* Finds the shared prefixes of a batch from its block tables, for callers
 * without a radix tree: sequences whose first page is the same physical
 * page form a group (two or more members); the group's prefix_blocks is the
 * longest run of leading pages all members share with its lowest-numbered
 * member, counting pages full in both.  Writes prefix_group[num_seqs],
 * prefix_blocks[] and *num_groups (device memory; ids < num_seqs / 2 + 1,
 * numbered by lowest member).  num_seqs <= 4096.  Meant to run once per
 * batch composition, not per decode step. */
int nxt_paged_prefix_groups(const int *block_tables, const int *seq_lens, int num_seqs,
                            int max_num_blocks_per_seq, int block_size, int *prefix_group,
                            int *prefix_blocks, int *num_groups, nxt_stream_t stream);

/* ---------------------------------------------------------- KV append
 * The step before the decode attention: store the new token's K and V rows
 * in the paged cache.  The reference has no GPU counterpart; its CPU decode
 * loop copies the rows into a contiguous cache at position cur_len and then
 * attends over cur_len + 1 tokens (examples/text_gen.c:1274-1281).  Here
 * the cache is the operator-API page layout [num_blocks][num_kv_heads]
 * [block_size][head_size] with the same strides (elements) as
 * nxt_paged_attention, and the new rows are key / value
 * [num_tokens][num_kv_heads][head_size] in the cache dtype.  The caller owns
 * every buffer and guarantees that page ids and slots lie inside the cache.
 * Asynchronous on `stream`; bytes are copied exactly.  Returns NXT_ATTN_OK
 * or a negative status (also recorded for nxt_attn_last_status). */

/* Decode: token s (row s of key / value) of sequence s goes to page
 * block_tables[s][positions[s] / block_size], slot positions[s] %
 * block_size.  A negative position, a position at or past
 * max_num_blocks_per_seq * block_size, or a negative page id skips it. */
int nxt_paged_kv_append(void *key_cache, void *value_cache, const void *key,
                        const void *value, const int *block_tables, const int *positions,
                        int num_seqs, int num_kv_heads, int head_size,
                        int max_num_blocks_per_seq, int block_size, int kv_block_stride,
                        int kv_head_stride, int kv_dtype, nxt_stream_t stream);

/* Prefill / general: token i goes to flat slot slot_mapping[i] (page =
 * slot / block_size, offset = slot % block_size); a negative slot skips it. */
int nxt_paged_kv_write_slots(void *key_cache, void *value_cache, const void *key,
                             const void *value, const int *slot_mapping, int num_tokens,
                             int num_kv_heads, int head_size, int block_size,
                             int kv_block_stride, int kv_head_stride, int kv_dtype,
                             nxt_stream_t stream);

/* Copy-on-write of a partly shared page: the K and V rows (every kv head) of
 * slot src_slots[i] are copied to slot dst_slots[i] of the same caches; a
 * negative source or destination skips the pair.  No destination may be the
 * source of another pair in the same call.  The reference has no counterpart
 * (its radix tree hands out shared pages only, prefix_sharing.c:211-265);
 * nxt_kv_seq_admit (xllm_hip_kv_index.h) produces the lists. */
int nxt_paged_kv_copy_slots(void *key_cache, void *value_cache, const int *src_slots,
                            const int *dst_slots, int num_tokens, int num_kv_heads, int head_size,
                            int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype,
                            nxt_stream_t stream);

/* ---------------------------------------------------------- activations
 * The MLP activations of the reference's operator API (include/operator_api.h:
 * 118-150, implemented there by operators/activation_kernels.cu:52-239).
 * Same names, argument order and meaning: input is [num_tokens][2*d] for the
 * gated ops (row = gate | up, the gate being the first d elements) and
 * [num_tokens][d] for the element-wise ones; out is [num_tokens][d].
 * dtype_size 2 = fp16, 4 = fp32.  Per element, in fp32:
 *   silu(x)      = x / (1 + exp(-x))
 *   gelu(x)      = (x * 0.5) * (1 + erf(x / sqrt(2)))
 *   gelu_tanh(x) = (0.5 * x) * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))
 * The activation is rounded to the element type and, for the gated ops,
 * multiplied by the other operand in the element type (one rounding of the
 * exact product), as the reference does (activation_kernels.cu:24-48, :65-69).
 * Contract points the reference leaves undefined, fixed here: num_tokens or
 * d of 0 does nothing (the reference's launch of 0 threads fails silently);
 * a negative size, a NULL tensor or a dtype_size other than 2 / 4 (the
 * reference treats every value but 2 as fp32) does nothing and records an
 * error for nxt_attn_last_status(); offsets are 64-bit (no wrap at 2^32
 * elements).  out must not overlap input, except that an element-wise op may
 * run in place (out == input).  Asynchronous on `stream`. */

/* Replaces nxt_silu_and_mul, include/operator_api.h:122-125:
 * out = silu(gate) * up. */
void nxt_silu_and_mul(void *out, const void *input, int num_tokens, int d, int dtype_size,
                      nxt_stream_t stream);

/* Replaces nxt_mul_and_silu, include/operator_api.h:127-130:
 * out = gate * silu(up). */
void nxt_mul_and_silu(void *out, const void *input, int num_tokens, int d, int dtype_size,
                      nxt_stream_t stream);

/* Replaces nxt_gelu_and_mul, include/operator_api.h:132-135:
 * out = gelu(gate) * up (erf form). */
void nxt_gelu_and_mul(void *out, const void *input, int num_tokens, int d, int dtype_size,
                      nxt_stream_t stream);

/* Replaces nxt_gelu_tanh_and_mul, include/operator_api.h:137-140:
 * out = gelu_tanh(gate) * up. */
void nxt_gelu_tanh_and_mul(void *out, const void *input, int num_tokens, int d, int dtype_size,
                           nxt_stream_t stream);

/* Replaces nxt_gelu_elementwise, include/operator_api.h:142-145:
 * out = gelu(input). */
void nxt_gelu_elementwise(void *out, const void *input, int num_tokens, int d, int dtype_size,
                          nxt_stream_t stream);

/* Replaces nxt_silu_elementwise, include/operator_api.h:147-150:
 * out = silu(input). */
void nxt_silu_elementwise(void *out, const void *input, int num_tokens, int d, int dtype_size,
                          nxt_stream_t stream);

/* Additive: the six activations above behind one entry point, with the
 * element type named explicitly (NxtKvDtype codes, so bf16 too) and a 64-bit
 * token count.  Returns NXT_ATTN_OK or a negative status. */
typedef enum {
    NXT_ACT_SILU_AND_MUL = 1,
    NXT_ACT_MUL_AND_SILU = 2,
    NXT_ACT_GELU_AND_MUL = 3,
    NXT_ACT_GELU_TANH_AND_MUL = 4,
    NXT_ACT_GELU = 5,
    NXT_ACT_SILU = 6,
} NxtActivationOp;

int nxt_activation_ex(int op, void *out, const void *input, int64_t num_tokens, int d, int dtype,
                      nxt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_OPERATOR_API_H_ */
