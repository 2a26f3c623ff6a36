// Read-only probe of a decode batch's K/V access pattern (measurement tool
// for bench.py, not part of the operator library): every valid 16-token tile
// of every (sequence, kv head) is read exactly as the MFMA partition kernel
// reads it -- K then V, 16-byte nontemporal buffer loads, one tile in flight
// while the previous one is consumed -- over the same number of resident
// wavefronts, with no arithmetic beyond folding the loaded words into one
// word per wavefront.  Its rate is the ceiling the decode kernel's own
// access pattern allows on this device.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "stream_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOob = 0x80000000u;
constexpr int kWaves = 4;  // wavefronts per workgroup

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const char *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7FFFFFFF, 0x00020000);
}

template <int LOADS>
struct Tile {
    u32x4 k[LOADS], v[LOADS];
};

// Tile i of the flattened list: row bytes `row_bytes`, valid rows in the
// low 5 bits of the descriptor, page byte offset in the rest.
template <int LOADS>
__device__ __forceinline__ void load_tile(const char *kbase, const char *vbase,
                                          const long long *desc, long long i, long long n,
                                          int row_bytes, int lane, Tile<LOADS> &t) {
    long long d = i < n ? desc[i] : 0;
    const int rows = (int)(d & 31);
    const long long off = d >> 5;
    const __amdgpu_buffer_rsrc_t rk = rsrc(kbase + off), rv = rsrc(vbase + off);
#pragma unroll
    for (int c = 0; c < LOADS; c++) {
        const int byte = (c * 64 + lane) * 16;
        const bool ok = i < n && byte < rows * row_bytes;
        const uint32_t o = ok ? (uint32_t)byte : kOob;
        t.k[c] = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)o, 0, 2);
    }
#pragma unroll
    for (int c = 0; c < LOADS; c++) {
        const int byte = (c * 64 + lane) * 16;
        const bool ok = i < n && byte < rows * row_bytes;
        const uint32_t o = ok ? (uint32_t)byte : kOob;
        t.v[c] = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)o, 0, 2);
    }
}

template <int LOADS>
__global__ __launch_bounds__(64 * kWaves) void stream_probe_kernel(
    const char *kbase, const char *vbase, const long long *desc, long long n, int row_bytes,
    int waves, uint32_t *sink) {
    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const long long per = (n + waves - 1) / waves;
    const long long lo = (long long)w * per;
    const long long hi = lo + per < n ? lo + per : n;
    uint32_t acc = 0;
    if (lo < hi) {
        Tile<LOADS> a, b;
        load_tile<LOADS>(kbase, vbase, desc, lo, hi, row_bytes, lane, a);
        for (long long i = lo; i < hi; i++) {
            load_tile<LOADS>(kbase, vbase, desc, i + 1, hi, row_bytes, lane, b);
#pragma unroll
            for (int c = 0; c < LOADS; c++)
                acc ^= a.k[c][0] ^ a.k[c][1] ^ a.k[c][2] ^ a.k[c][3] ^ a.v[c][0] ^ a.v[c][1] ^
                       a.v[c][2] ^ a.v[c][3];
            a = b;
        }
    }
    sink[(size_t)w * 64 + lane] = acc;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int xllm_stream_probe(
    const void *key_cache, const void *value_cache, const long long *tile_desc,
    long long num_tiles, int tile_bytes, int waves, unsigned *sink, void *stream) {
    if (!key_cache || !value_cache || !tile_desc || !sink || num_tiles < 0 || waves <= 0 ||
        waves % kWaves)
        return -1;
    const int row_bytes = tile_bytes / 16;
    const dim3 grid(waves / kWaves), block(64 * kWaves);
    const hipStream_t st = (hipStream_t)stream;
    switch (tile_bytes) {  // 16 rows of head_size x 2 bytes: 1, 2 or 4 KB
    case 1024: hipLaunchKernelGGL(stream_probe_kernel<1>, grid, block, 0, st, (const char *)key_cache, (const char *)value_cache, tile_desc, num_tiles, row_bytes, waves, sink); break;
    case 2048: hipLaunchKernelGGL(stream_probe_kernel<2>, grid, block, 0, st, (const char *)key_cache, (const char *)value_cache, tile_desc, num_tiles, row_bytes, waves, sink); break;
    case 4096: hipLaunchKernelGGL(stream_probe_kernel<4>, grid, block, 0, st, (const char *)key_cache, (const char *)value_cache, tile_desc, num_tiles, row_bytes, waves, sink); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
