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
// slot of the same caches: the copy-on-write of a partly shared page.
// HBM-bound byte copy: each lane moves one 16-byte chunk of K and the same
// chunk of V, with one load and one store each, from 32-bit indices (a
// multiply-high division by the row's chunks and by the kv heads; a 64-bit
// grid-stride version with three 64-bit divisions per chunk copied at 66%
// of the HBM peak).  The new rows are read once: nontemporal loads.
// Launches hold fewer than 2^31 chunks each (tokens split across launches).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paged_kv_append.h"

namespace xhip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kKvAppendBlock = 64;  // one wavefront per workgroup
constexpr long long kKvAppendMaxChunks = (1LL << 31) - 1;

// Chunk i of a launch's K/V rows to its page slot.
__device__ __forceinline__ void append_chunk(const KvAppendParams &p, uint32_t i) {
    if (i >= p.chunks) return;
    const uint32_t row_l = div_by(i, p.row_div);  // row of the launch: token * kv heads + head
    const int c = (int)(i - row_l * (uint32_t)p.row_chunks);
    const uint32_t tok_l = div_by(row_l, p.head_div);
    const int h = (int)(row_l - tok_l * (uint32_t)p.num_kv_heads);
    const int tok = p.tok0 + (int)tok_l;
    long long slot;
    if (p.slots) {
        slot = p.slots[tok];
    } else {
        const int pos = p.positions[tok];
        if (pos < 0 || pos >= p.max_ctx) return;
        const int blk = p.block_tables[(size_t)tok * p.max_blocks + (pos >> p.bs_shift)];
        slot = blk < 0 ? -1 : (long long)blk * p.block_size + (pos & (p.block_size - 1));
    }
    if (slot < 0) return;
    const long long blk = slot >> p.bs_shift;
    const long long off = slot & (p.block_size - 1);
    const size_t dst = (size_t)(blk * p.kv_block_stride_bytes + h * p.kv_head_stride_bytes +
                                off * p.row_bytes) + (size_t)c * 16;
    u32x4 k, v;
    if (p.src_slots) {  // copy inside the cache, page slot to page slot
        const long long from = p.src_slots[tok];
        if (from < 0) return;
        const size_t src = (size_t)((from >> p.bs_shift) * p.kv_block_stride_bytes +
                                    h * p.kv_head_stride_bytes +
                                    (from & (p.block_size - 1)) * p.row_bytes) + (size_t)c * 16;
        k = *(const u32x4 *)((const char *)p.key + src);
        v = *(const u32x4 *)((const char *)p.value + src);
    } else if (p.key_rows) {  // each token's rows at their own address
        const size_t o = (size_t)h * p.row_bytes + (size_t)c * 16;
        k = __builtin_nontemporal_load((const u32x4 *)(p.key_rows[tok] + o));
        v = __builtin_nontemporal_load((const u32x4 *)(p.value_rows[tok] + o));
    } else {
        const size_t src = ((size_t)tok * p.num_kv_heads + h) * p.row_bytes + (size_t)c * 16;
        k = __builtin_nontemporal_load((const u32x4 *)((const char *)p.key + src));
        v = __builtin_nontemporal_load((const u32x4 *)((const char *)p.value + src));
    }
    *(u32x4 *)((char *)p.key_cache + dst) = k;
    *(u32x4 *)((char *)p.value_cache + dst) = v;
}

__global__ __launch_bounds__(kKvAppendBlock) void paged_kv_append_kernel(const KvAppendParams p) {
    append_chunk(p, blockIdx.x * kKvAppendBlock + threadIdx.x);
}

hipError_t launch_kv_append(const KvAppendParams &params, hipStream_t stream) {
    KvAppendParams p = params;
    const long long per_token = (long long)p.num_kv_heads * p.row_chunks;
    if (p.num_tokens <= 0 || per_token <= 0) return hipSuccess;
    p.row_div = div_magic((uint32_t)p.row_chunks);
    p.head_div = div_magic((uint32_t)p.num_kv_heads);
    const long long tok_per_launch = kKvAppendMaxChunks / per_token;
    for (long long t0 = 0; t0 < p.num_tokens; t0 += tok_per_launch) {
        const long long n = p.num_tokens - t0 < tok_per_launch ? p.num_tokens - t0 : tok_per_launch;
        p.tok0 = (int)t0;
        p.chunks = (uint32_t)(n * per_token);
        const long long blocks = ((long long)p.chunks + kKvAppendBlock - 1) / kKvAppendBlock;
        paged_kv_append_kernel<<<(unsigned)blocks, kKvAppendBlock, 0, stream>>>(p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Staging copy by the device: n16 16-byte chunks from host-pinned memory
// (read over the host link) into device memory.  The model instance stages
// each exec's arrays this way instead of with a DMA copy: a small copy went
// through the DMA engine in ~6.7 us plus its submission, this kernel's reads
// take one host-link round trip.
//
// One thread's share of a staging copy: 16-byte chunk i of the staged
// bytes, to the tables' head or to dst; the first workgroup also stores the
// table entries.
__device__ __forceinline__ void stage_chunks(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst,
                                             long long n16, unsigned blocks,
                                             const StageTables &t) {
    const long long stride = (long long)blocks * 256;
    const long long head16 = t.head_bytes / 16;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = src[i];
        if (i < head16)
            ((u32x4 *)t.head)[i] = v;
        else
            dst[i - head16] = v;
    }
    if (blockIdx.x == 0)
        for (int j = threadIdx.x; j < t.count; j += 256) t.table[t.pairs[2 * j]] = t.pairs[2 * j + 1];
}

__global__ __launch_bounds__(256) void stage_copy_kernel(const u32x4 *__restrict__ src,
                                                         u32x4 *__restrict__ dst, long long n16,
                                                         const StageTables t) {
    stage_chunks(src, dst, n16, gridDim.x, t);
}

static StageTables no_tables() {
    StageTables t;
    t.head = nullptr;
    t.head_bytes = 0;
    t.pairs = nullptr;
    t.count = 0;
    t.table = nullptr;
    return t;
}

static bool tables_ok(const StageTables &t, size_t bytes) {
    return t.head_bytes >= 0 && (size_t)t.head_bytes <= bytes && (t.head_bytes & 15) == 0 &&
           (t.head_bytes == 0 || t.head) && t.count >= 0 && (t.count == 0 || (t.pairs && t.table));
}

hipError_t launch_stage_copy(void *dst, const void *host_src, size_t bytes, hipStream_t stream,
                             const StageTables *tables) {
    const StageTables t = tables ? *tables : no_tables();
    if (bytes == 0 && t.count == 0) return hipSuccess;
    if ((bytes | (uintptr_t)dst | (uintptr_t)host_src) & 15) return hipErrorInvalidValue;
    if (!tables_ok(t, bytes)) return hipErrorInvalidValue;
    const long long n16 = (long long)(bytes / 16);
    long long blocks = (n16 + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    stage_copy_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const u32x4 *)host_src, (u32x4 *)dst,
                                                             n16, t);
    return hipGetLastError();
}

// The staging copy and a K/V append in one launch: workgroups [0,
// copy_blocks) copy the staged arrays, the others write the new rows, whose
// slots and row pointers `p` reads from the host-pinned staging buffer
// itself (its device copy is being made by the same launch).  One launch
// fewer per exec: a launch costs ~2.5 us of host time (HIP runtime, as
// measured on the MI355X hosts).
__global__ __launch_bounds__(256) void stage_append_kernel(const u32x4 *__restrict__ src,
                                                           u32x4 *__restrict__ dst, long long n16,
                                                           unsigned copy_blocks,
                                                           const KvAppendParams p,
                                                           const StageTables t) {
    if (blockIdx.x < copy_blocks) {
        stage_chunks(src, dst, n16, copy_blocks, t);
        return;
    }
    append_chunk(p, (blockIdx.x - copy_blocks) * 256 + threadIdx.x);
}

hipError_t launch_stage_copy_append(void *dst, const void *host_src, size_t bytes,
                                    const KvAppendParams &params, hipStream_t stream,
                                    const StageTables *tables) {
    KvAppendParams p = params;
    const StageTables t = tables ? *tables : no_tables();
    const long long per_token = (long long)p.num_kv_heads * p.row_chunks;
    const long long chunks = (long long)p.num_tokens * per_token;
    if (bytes == 0 || chunks <= 0 || chunks > (1LL << 24)) {  // (the separate launches)
        hipError_t e = launch_stage_copy(dst, host_src, bytes, stream, tables);
        return e != hipSuccess ? e : launch_kv_append(params, stream);
    }
    if ((bytes | (uintptr_t)dst | (uintptr_t)host_src) & 15) return hipErrorInvalidValue;
    if (!tables_ok(t, bytes)) return hipErrorInvalidValue;
    p.row_div = div_magic((uint32_t)p.row_chunks);
    p.head_div = div_magic((uint32_t)p.num_kv_heads);
    p.tok0 = 0;
    p.chunks = (uint32_t)chunks;
    const long long n16 = (long long)(bytes / 16);
    long long copy_blocks = (n16 + 255) / 256;
    if (copy_blocks > 1024) copy_blocks = 1024;
    const long long blocks = copy_blocks + (chunks + 255) / 256;
    stage_append_kernel<<<(unsigned)blocks, 256, 0, stream>>>(
        (const u32x4 *)host_src, (u32x4 *)dst, n16, (unsigned)copy_blocks, p, t);
    return hipGetLastError();
}

// Completion word of a model-instance exec: one thread stores `value` to a
// host-coherent word with system scope.  Queued after an exec's launches it
// runs once they have all finished, and the host sees the word change
// ~2 us before hipStreamSynchronize on the same stream returns (measured on
// MI355X: a small kernel plus this signal and a host poll 9.3 us, the
// kernel plus hipStreamSynchronize 11.5 us).
__global__ __launch_bounds__(64) void exec_signal_kernel(unsigned *word, unsigned value) {
    if (threadIdx.x == 0) __hip_atomic_store(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_exec_signal(unsigned *word, unsigned value, hipStream_t stream) {
    exec_signal_kernel<<<1, 64, 0, stream>>>(word, value);
    return hipGetLastError();
}

}  // namespace xhip
