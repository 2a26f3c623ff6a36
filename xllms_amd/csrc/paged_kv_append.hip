// KV append for the paged cache: writes the K/V rows of new tokens into
// their page slots, the step that precedes the decode attention (the
// reference's CPU decode loop does it with two memcpys into a contiguous
// cache at position cur_len, examples/text_gen.c:1274-1278).
//
// Layout: the new rows are key/value [num_tokens][num_kv_heads][row_bytes]
// (one row = head_size elements of any dtype, a multiple of 16 bytes); the
// caches are the operator-API pages [num_blocks][num_kv_heads][block_size]
// [head_size] addressed with kv_block_stride / kv_head_stride in bytes here.
// Token i goes to page slot_of(i) / block_size, offset slot_of(i) %
// block_size, where slot_of comes either from `slots` (prefill: one flat
// slot per token) or from `block_tables` + `positions` (decode: token s of
// sequence s at position positions[s]).  A negative slot, position or page
// id skips the token.  In copy mode (`src_slots`) the rows come from another
// slot of the same caches: the copy-on-write of a partly shared page.  HBM-bound byte copy: each lane moves 16 bytes of K
// and 16 of V with one load and one store each; a wavefront covers four
// 256-byte rows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paged_kv_append.h"

namespace xhip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void paged_kv_append_kernel(const KvAppendParams p) {
    const long long n_chunks = (long long)p.num_tokens * p.num_kv_heads * p.row_chunks;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n_chunks; i += stride) {
        const int c = (int)(i % p.row_chunks);
        const long long row = i / p.row_chunks;  // token * num_kv_heads + kv head
        const int h = (int)(row % p.num_kv_heads);
        const int tok = (int)(row / p.num_kv_heads);
        long long slot;
        if (p.slots) {
            slot = p.slots[tok];
        } else {
            const int pos = p.positions[tok];
            if (pos < 0 || pos >= p.max_ctx) continue;
            const int blk = p.block_tables[(size_t)tok * p.max_blocks + (pos >> p.bs_shift)];
            slot = blk < 0 ? -1 : (long long)blk * p.block_size + (pos & (p.block_size - 1));
        }
        if (slot < 0) continue;
        const long long blk = slot >> p.bs_shift;
        const long long off = slot & (p.block_size - 1);
        const size_t dst = (size_t)(blk * p.kv_block_stride_bytes + h * p.kv_head_stride_bytes +
                                    off * p.row_bytes) + (size_t)c * 16;
        size_t src;
        if (p.src_slots) {  // copy inside the cache, page slot to page slot
            const long long from = p.src_slots[tok];
            if (from < 0) continue;
            src = (size_t)((from >> p.bs_shift) * p.kv_block_stride_bytes +
                           h * p.kv_head_stride_bytes +
                           (from & (p.block_size - 1)) * p.row_bytes) + (size_t)c * 16;
        } else if (p.key_rows) {  // each token's rows at their own address
            const size_t o = (size_t)h * p.row_bytes + (size_t)c * 16;
            const u32x4 k = *(const u32x4 *)(p.key_rows[tok] + o);
            const u32x4 v = *(const u32x4 *)(p.value_rows[tok] + o);
            *(u32x4 *)((char *)p.key_cache + dst) = k;
            *(u32x4 *)((char *)p.value_cache + dst) = v;
            continue;
        } else {
            src = (size_t)row * p.row_bytes + (size_t)c * 16;
        }
        const u32x4 k = *(const u32x4 *)((const char *)p.key + src);
        const u32x4 v = *(const u32x4 *)((const char *)p.value + src);
        *(u32x4 *)((char *)p.key_cache + dst) = k;
        *(u32x4 *)((char *)p.value_cache + dst) = v;
    }
}

hipError_t launch_kv_append(const KvAppendParams &p, hipStream_t stream) {
    const long long n_chunks = (long long)p.num_tokens * p.num_kv_heads * p.row_chunks;
    if (n_chunks == 0) return hipSuccess;
    long long blocks = (n_chunks + 255) / 256;
    if (blocks > 65536) blocks = 65536;  // grid-stride beyond
    paged_kv_append_kernel<<<(unsigned)blocks, 256, 0, stream>>>(p);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void gather_rows_kernel(char *dst, const char *const *src,
                                                          int chunks, int n) {
    const long long total = (long long)n * chunks;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int r = (int)(i / chunks), c = (int)(i % chunks);
        *(u32x4 *)(dst + i * 16) = *(const u32x4 *)(src[r] + (size_t)c * 16);
    }
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(char *const *dst, const char *src,
                                                           int chunks, int n) {
    const long long total = (long long)n * chunks;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int r = (int)(i / chunks), c = (int)(i % chunks);
        *(u32x4 *)(dst[r] + (size_t)c * 16) = *(const u32x4 *)(src + i * 16);
    }
}

static unsigned copy_grid(long long chunks) {
    long long blocks = (chunks + 255) / 256;
    return (unsigned)(blocks > 4096 ? 4096 : blocks);
}

hipError_t launch_gather_rows(void *dst, const char *const *src, int row_bytes, int n,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int chunks = row_bytes / 16;
    gather_rows_kernel<<<copy_grid((long long)n * chunks), 256, 0, stream>>>((char *)dst, src,
                                                                              chunks, n);
    return hipGetLastError();
}

hipError_t launch_scatter_rows(char *const *dst, const void *src, int row_bytes, int n,
                               hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int chunks = row_bytes / 16;
    scatter_rows_kernel<<<copy_grid((long long)n * chunks), 256, 0, stream>>>(
        dst, (const char *)src, chunks, n);
    return hipGetLastError();
}

}  // namespace xhip
