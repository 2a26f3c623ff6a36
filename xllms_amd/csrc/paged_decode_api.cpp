// C-ABI of the paged-decode attention: argument validation, the split-K plan,
// per-(device, stream) workspace, and the launch of the gfx950 kernels.
//
// Entry points replace include/operator_api.h:63-115 of the reference (see
// include/xllm_hip_operator_api.h for the contract).  Host-side only; the
// kernels live in paged_decode_{f16,bf16,f32}.hip.
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "activation.h"
#include "paged_decode_cascade.h"
#include "paged_decode_launch.h"
#include "paged_decode_params.h"
#include "paged_decode_rows.h"
#include "noalloc_gate.h"
#include "paged_decode_scratch.h"
#include "paged_kv_append.h"
#include "workspace.h"
#include "workspace_cache.h"
#include "wg_trace.h"
#include "xllm_hip_operator_api.h"

namespace {

using xhip::DecodeParams;

thread_local int t_status = NXT_ATTN_OK;
thread_local char t_message[512] = "ok";
thread_local hipEvent_t t_trace_start = nullptr;
thread_local hipEvent_t t_trace_partition = nullptr;
// Per-workgroup timestamp buffer of the instrumented measurement build
// (wg_trace.h); the product build never sets it.
thread_local unsigned long long *t_wg_trace = nullptr;

int set_status(int status, const char *fmt, ...) {
    t_status = status;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_message, sizeof(t_message), fmt, ap);
    va_end(ap);
    return status;
}

int ok() {
    t_status = NXT_ATTN_OK;
    snprintf(t_message, sizeof(t_message), "ok");
    return NXT_ATTN_OK;
}

// ---------------------------------------------------------------- workspace
// Device calls of the workspace cache (workspace_cache.h).
struct HipDev {
    // runs fn with `device` current, restoring the caller's device
    template <class Fn> static int on_device(int device, Fn &&fn) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) return 1;
        if (cur != device && hipSetDevice(device) != hipSuccess) return 1;
        const hipError_t e = fn();
        if (cur != device) (void)hipSetDevice(cur);
        return e == hipSuccess ? 0 : 1;
    }
    static int sync_stream(int, void *stream) {
        return hipStreamSynchronize((hipStream_t)stream) == hipSuccess ? 0 : 1;
    }
    static int sync_device(int device) {
        return on_device(device, [] { return hipDeviceSynchronize(); });
    }
    static int alloc(int, void **ptr, size_t bytes) {  // the caller's device is current
        return hipMalloc(ptr, bytes) == hipSuccess ? 0 : 1;
    }
    static int release(int device, void *ptr) {
        return on_device(device, [ptr] { return hipFree(ptr); });
    }
    static bool per_thread(void *stream) { return stream == (void *)hipStreamPerThread; }
    static bool capturing(void *stream) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        return cs == hipStreamCaptureStatusActive;
    }
};

using WsCache = xhip::WorkspaceCache<HipDev>;

// Event calls of the no-alloc gate (noalloc_gate.h).
struct HipGateDev {
    static int create_event(void **ev) {
        return hipEventCreateWithFlags((hipEvent_t *)ev, hipEventDisableTiming) == hipSuccess ? 0
                                                                                              : 1;
    }
    static int record(void *ev, void *stream) {
        return hipEventRecord((hipEvent_t)ev, (hipStream_t)stream) == hipSuccess ? 0 : 1;
    }
    static int wait(void *stream, void *ev) {
        return hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)ev, 0) == hipSuccess ? 0 : 1;
    }
    static bool capturing(void *stream) { return HipDev::capturing(stream); }
    static bool per_thread(void *stream) { return HipDev::per_thread(stream); }
};
using NoAllocGate = xhip::NoAllocGate<HipGateDev>;
NoAllocGate g_noalloc_gate;
using xhip::kWsCascade;
using xhip::kWsSplitK;

WsCache g_ws;
thread_local const void *t_ws_owner = nullptr;

// Takes (device, stream, kind)'s workspace of at least `bytes` for one call;
// it stays locked to this thread until `lease` is destroyed, after the
// call's launches are enqueued.
int get_workspace(int device, hipStream_t stream, size_t bytes, WsCache::Lease *lease,
                  int kind = kWsSplitK) {
    const int rc = g_ws.acquire(device, (void *)stream, kind, bytes, t_ws_owner, lease);
    if (rc == WsCache::kSyncFailed)
        return set_status(NXT_ATTN_E_HIP, "hipStreamSynchronize before growing the workspace failed");
    if (rc == WsCache::kNoMemory)
        return set_status(NXT_ATTN_E_NOMEM, "workspace of %zu bytes: hipMalloc failed", bytes);
    if (rc == WsCache::kCaptureGrow)
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "stream is capturing and this call needs a %zu-byte workspace the stream "
                          "does not have yet: make one call of this shape on the stream before "
                          "the capture (or use nxt_paged_attention_noalloc)",
                          bytes);
    return NXT_ATTN_OK;
}

// ------------------------------------------------------------- device info
constexpr int kMaxDevices = 64;
std::mutex g_dev_mu;
int g_cu_count[kMaxDevices];

int cu_count(int device) {
    if (device < 0 || device >= kMaxDevices) return 256;
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if (g_cu_count[device] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            n <= 0)
            n = 256;
        g_cu_count[device] = n;
    }
    return g_cu_count[device];
}

// ---------------------------------------------------------------- geometry
bool supported_head_size(int d) {
    switch (d) {
    case 32: case 64: case 80: case 96: case 112: case 128: case 192: case 256: return true;
    default: return false;
    }
}

int pow2_ceil(int x) {
    int r = 1;
    while (r < x) r <<= 1;
    return r;
}

bool is_pow2(long long x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int x) {
    int r = 0;
    while ((1 << r) < x) r++;
    return r;
}

int elem_bytes(int kv_dtype) { return kv_dtype == NXT_KV_FP32 ? 4 : 2; }

// The MFMA tile path serves fp16/bf16 with head_size % 32 == 0 and pages of
// at least one 16-token tile; every other shape takes the VALU tile path.
bool use_mfma(int kv_dtype, int head_size, int block_size) {
    return kv_dtype != NXT_KV_FP32 && head_size % 32 == 0 && block_size >= 16;
}

// Tokens per tile of the kernel instantiation: 16 on the MFMA path, else
// kLoadsPerTile loads of 64/lanes-per-row rows (mirrors xhip::Geometry).
int tile_tokens(int head_size, int kv_dtype, bool mfma) {
    if (mfma) return 16;
    const int vec = 16 / elem_bytes(kv_dtype);
    const int row_lanes = pow2_ceil(head_size / vec);
    return (64 / row_lanes) * xhip::kLoadsPerTile;
}

struct HeadTiling {
    int head_tile;   // query heads per wavefront
    int head_tiles;  // wavefronts per (seq, kv head, partition)
};

// Largest GQA group of a tile path: the MFMA path splits any group into
// head tiles (segments of their own); the VALU path's tiles stop at 32.
int max_group(bool mfma) {
    return mfma ? xhip::kMfmaMaxGroup : xhip::kMaxHeadTile * xhip::kWavesPerGroup;
}

bool head_tiling(int group, bool mfma, int head_size, HeadTiling *t) {
    if (group <= 0 || group > max_group(mfma)) return false;
    if (mfma) {
        // groups of 17-32 heads: one wavefront with two row blocks reads each
        // K/V tile once for all of them (head_size <= 128), else two
        // wavefronts of one block each
        const bool wide = group > xhip::kMfmaHeads && head_size <= xhip::kMfmaWideMaxHeadSize;
        t->head_tile = wide ? 2 * xhip::kMfmaHeads : xhip::kMfmaHeads;
        t->head_tiles = (group + t->head_tile - 1) / t->head_tile;
        return true;
    }
    if (group <= xhip::kMaxHeadTile) {
        t->head_tile = pow2_ceil(group);
        t->head_tiles = 1;
        return true;
    }
    // ceil, not a power of two: every head tile holds at least one head (a
    // tile past the group would be a segment with no columns to merge)
    t->head_tile = xhip::kMaxHeadTile;
    t->head_tiles = (group + xhip::kMaxHeadTile - 1) / xhip::kMaxHeadTile;
    return t->head_tiles <= xhip::kWavesPerGroup;
}

// Smallest stream-K range, in split units, the automatic plan gives a
// wavefront: it binds only batches too small to fill the launch, whose time
// is the chain of dependent loads in each range.  Config 1 (8 sequences)
// measured 14.3-14.6 / 14.8 / 14.9 / 16.0-16.1 us per step at 2 / 3 / 4 / 6.
constexpr int kMinTilesPerWave = 2;


int partition_occupancy(int kv_dtype, int head_size, int head_tile, bool mfma, size_t lds) {
    switch (kv_dtype) {
    case NXT_KV_FP16: return xhip::partition_occupancy_f16(head_size, head_tile, mfma, lds);
    case NXT_KV_BF16: return xhip::partition_occupancy_bf16(head_size, head_tile, mfma, lds);
    default: return xhip::partition_occupancy_f32(head_size, head_tile, mfma, lds);
    }
}

// Wavefronts per CU of the MFMA partition kernel's plan: eight (2 per SIMD).
// Measured on MI355X against the twelve that fit: 4-10% less time on configs
// 2, 3 and 4 (fewer concurrent page streams per HBM channel, and an even
// finish across wavefronts).
constexpr int kMfmaWavesPerCu = 8;

int waves_per_group(bool mfma) { return mfma ? xhip::kMfmaWavesPerGroup : xhip::kWavesPerGroup; }

// Wavefronts of the automatic plan: one resident round of the partition
// kernel on every CU, but no more than the batch could keep busy with
// kMinTilesPerWave units each.
long long auto_waves(int kv_dtype, int head_size, int head_tile, bool mfma, int nseq,
                     long long ub_tiles, int cus) {
    const size_t lds = (size_t)(nseq + 1) * sizeof(int);
    const int occ = partition_occupancy(kv_dtype, head_size, head_tile, mfma, lds);
    if (occ <= 0) return 0;
    const int wpg = waves_per_group(mfma);
    int per_cu = occ * wpg;
    if (mfma && per_cu > kMfmaWavesPerCu) per_cu = kMfmaWavesPerCu;
    long long w = (long long)cus * per_cu;
    // On the MFMA path a batch bounded below kSmallBatchUnits units per
    // wavefront of that round gets one workgroup per CU instead: its wavefronts are short
    // chains of dependent loads, and a second workgroup on a CU waits behind
    // the first's.  Measured on MI355X (fp16, 32 / 8 heads, d = 128, step
    // times): 1 x 8192 tokens 18.5 -> 17.0 us, 4 x 2048 and 8 x 1024 18.4 ->
    // 16.9 us, 2 x 8192 22.5 -> 21.6 us; 1 x 2048 and batches above the bound
    // unchanged.
    constexpr long long kSmallBatchUnits = 8;
    if (mfma && ub_tiles < kSmallBatchUnits * w && per_cu > wpg) w = (long long)cus * wpg;
    const long long need = (ub_tiles + kMinTilesPerWave - 1) / kMinTilesPerWave;
    if (need < w) w = need;
    w = (w + wpg - 1) / wpg * wpg;
    return w > 0 ? w : wpg;
}

constexpr long long kMaxWaves = 1LL << 22;
constexpr long long kMaxLaunchTiles = 1LL << 30;  // bounds the partial workspace of explicit plans

// Split units an automatic plan charges each segment on top of its tiles
// (paged_decode_params.h): on MI355X a segment's first tile computes ~1.5
// tiles' time after the piece begins (block ids, then K, then the softmax
// chain), and a batch of fresh one-tile sequences otherwise piles dozens of
// such starts on one wavefront.  Explicit partition_tokens plans charge 0,
// so each wavefront's range is exactly partition_tokens of K/V.
constexpr int kSegmentCost = 2;

const char *dtype_name(int kv_dtype) {
    switch (kv_dtype) {
    case NXT_KV_FP16: return "fp16";
    case NXT_KV_BF16: return "bf16";
    case NXT_KV_FP32: return "fp32";
    default: return "?";
    }
}

// Partial-output mode of a pass (cascade decode): fp32 rows + log-sum-exp
// instead of `out`, and the K/V load policy.
struct PartialOut {
    float *out_f32;
    float *out_lse;
    int cached_seqs;  // leading sequences whose K/V loads are cacheable
    int skip_empty;   // rows of empty sequences are never read: leave them unwritten
};

// Prefix fold of a pass (cascade suffix pass): DecodeParams::fold_row.
struct PrefixFold {
    const int *row;  // [num_seqs]
    const float *out;
    const float *lse;
    int rows, kr;
};

// A caller-provided split-K workspace (the allocation-free entry point's
// fixed device scratch) used instead of the workspace cache.
struct FixedWs {
    void *ptr;
    size_t bytes;
};

// Per-sequence query and output rows (device arrays of num_seqs row
// pointers, each row block [num_heads][head_size], 16-byte aligned) instead
// of the contiguous query / out arrays: the model instance's requests keep
// their own buffers.
struct RowPtrs {
    const char *const *q;
    char *const *o;
};

// New-token fold of a one-sequence launch (DecodeParams::nt_fold): the
// sequence's cached tokens are attended in partial-output mode (po), and the
// merge folds in the new token and writes `out`.
struct NewTokenFold {
    const void *k, *v;  // the token's rows, [num_kv_heads][head_size], device
    int *table;         // block-table entry that receives `page` (null: none)
    int *lens;          // length entry that receives `len`
    int slot, page, len;
};

// The fields of a launch's DecodeParams that come straight from its batch.
void fill_batch(DecodeParams &p, const void *query, const void *key_cache, const void *value_cache,
                const int *block_tables, const int *seq_lens, int nseq, int num_heads,
                int num_kv_heads, int head_tiles, int max_num_blocks_per_seq, int block_size,
                int kv_block_stride, int kv_head_stride, float scale) {
    const long long max_ctx = (long long)max_num_blocks_per_seq * block_size;
    p.q = query;
    p.k = key_cache;
    p.v = value_cache;
    p.block_tables = block_tables;
    p.seq_lens = seq_lens;
    p.kv_block_stride = kv_block_stride;
    p.kv_head_stride = kv_head_stride;
    p.num_seqs = nseq;
    p.num_heads = num_heads;
    p.num_kv_heads = num_kv_heads;
    p.group = num_heads / num_kv_heads;
    p.head_tiles = head_tiles;
    p.max_blocks = max_num_blocks_per_seq;
    p.block_size = block_size;
    p.bs_shift = ilog2(block_size);
    p.max_ctx = (int)max_ctx;
    p.scale_log2 = scale * 1.4426950408889634f;
}

int run(void *out, const void *query, const void *key_cache, const void *value_cache,
        const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
        int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
        int kv_block_stride, int kv_head_stride, nxt_stream_t stream_handle, int kv_dtype,
        int partition_tokens, const PartialOut *po = nullptr, const PrefixFold *fold = nullptr,
        const FixedWs *fixed = nullptr, const RowPtrs *rows = nullptr,
        const NewTokenFold *nt = nullptr) {
    // ---- argument checks (host only; nothing is read from the device)
    if (kv_dtype != NXT_KV_FP16 && kv_dtype != NXT_KV_BF16 && kv_dtype != NXT_KV_FP32)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "kv_dtype %d is not FP16/BF16/FP32", kv_dtype);
    if (dtype_size != elem_bytes(kv_dtype))
        return set_status(NXT_ATTN_E_INVALID, "dtype_size %d does not match %s", dtype_size,
                          dtype_name(kv_dtype));
    if (num_seqs < 0) return set_status(NXT_ATTN_E_INVALID, "num_seqs %d < 0", num_seqs);
    if (num_heads <= 0 || num_kv_heads <= 0)
        return set_status(NXT_ATTN_E_INVALID, "num_heads %d / num_kv_heads %d must be > 0",
                          num_heads, num_kv_heads);
    if (num_heads % num_kv_heads)
        return set_status(NXT_ATTN_E_INVALID, "num_heads %d is not a multiple of num_kv_heads %d",
                          num_heads, num_kv_heads);
    if (!supported_head_size(head_size))
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "head_size %d not in {32,64,80,96,112,128,192,256}", head_size);
    if (max_num_blocks_per_seq <= 0)
        return set_status(NXT_ATTN_E_INVALID, "max_num_blocks_per_seq %d must be > 0",
                          max_num_blocks_per_seq);
    if (block_size <= 0) return set_status(NXT_ATTN_E_INVALID, "block_size %d", block_size);
    if (!is_pow2(block_size) || block_size > 1024)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "block_size %d is not a power of two <= 1024",
                          block_size);
    if (kv_block_stride < 0 || kv_head_stride < 0)
        return set_status(NXT_ATTN_E_INVALID, "negative kv stride (%d, %d)", kv_block_stride,
                          kv_head_stride);
    if (!isfinite(scale)) return set_status(NXT_ATTN_E_INVALID, "scale is not finite");
    const long long max_ctx = (long long)max_num_blocks_per_seq * block_size;
    if (max_ctx > (1LL << 28))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "context bound %lld tokens too large", max_ctx);
    const int group = num_heads / num_kv_heads;
    const bool mfma = use_mfma(kv_dtype, head_size, block_size);
    HeadTiling tiling;
    if (!head_tiling(group, mfma, head_size, &tiling))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "GQA group %d > %d", group, max_group(mfma));
    if (nt && (num_seqs != 1 || !po || !out || rows || fold || partition_tokens ||
               !(head_size == 32 || head_size == 64 || head_size == 128) || !nt->k || !nt->v ||
               !nt->lens))
        return set_status(NXT_ATTN_E_INVALID, "bad new-token fold launch");
    if (num_seqs == 0) return ok();
    const void *out_any = po ? (const void *)po->out_f32 : rows ? (const void *)rows->o : out;
    const void *q_any = rows ? (const void *)rows->q : query;
    if (!out_any || !q_any || !key_cache || !value_cache || !block_tables || !seq_lens ||
        (po && !po->out_lse))
        return set_status(NXT_ATTN_E_INVALID, "NULL tensor pointer");
    const int eb = elem_bytes(kv_dtype);
    if (((uintptr_t)(po ? out_any : rows ? nullptr : out) | (uintptr_t)(rows ? nullptr : query) |
         (uintptr_t)key_cache | (uintptr_t)value_cache) & 15)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "tensors must be 16-byte aligned");
    if (rows && (((uintptr_t)rows->q | (uintptr_t)rows->o) & 7))
        return set_status(NXT_ATTN_E_INVALID, "row pointer tables must be 8-byte aligned");
    if ((((long long)kv_block_stride * eb) & 15) || (((long long)kv_head_stride * eb) & 15))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "kv strides must be multiples of 16 bytes");
    if ((uintptr_t)block_tables & 3 || (uintptr_t)seq_lens & 3)
        return set_status(NXT_ATTN_E_INVALID, "int32 tables must be 4-byte aligned");

    const int tile = tile_tokens(head_size, kv_dtype, mfma);
    if (partition_tokens != 0 && (!is_pow2(partition_tokens) || partition_tokens < tile))
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "partition_tokens %d must be a power of two >= %d for head_size %d %s",
                          partition_tokens, tile, head_size, dtype_name(kv_dtype));

    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return set_status(NXT_ATTN_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    hipStream_t stream = (hipStream_t)stream_handle;
    const int cus = cu_count(device);
    const int segs = num_kv_heads * tiling.head_tiles;
    const int seg_cost = partition_tokens == 0 ? kSegmentCost : 0;
    const long long units_per_seg = (max_ctx + tile - 1) / tile + seg_cost;

    // Batches go in consecutive launches of at most kMaxSeqsPerLaunch
    // sequences (the per-workgroup prefix scan of the partition kernel lives
    // in LDS) and at most kMaxLaunchTiles split units by the context bound
    // (unit indices are 32-bit on the device).
    const long long seq_units = (long long)segs * units_per_seg;
    if (seq_units >= kMaxLaunchTiles)
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "one sequence bounds %lld tiles (kv heads x context); limit %lld",
                          seq_units, kMaxLaunchTiles);
    const long long fit = kMaxLaunchTiles / seq_units;
    const int per_launch = fit < xhip::kMaxSeqsPerLaunch ? (int)fit : xhip::kMaxSeqsPerLaunch;
    for (int s0 = 0; s0 < num_seqs; s0 += per_launch) {
        const int nseq = num_seqs - s0 < per_launch ? num_seqs - s0 : per_launch;
        const long long ub_tiles = (long long)nseq * seq_units;
        long long waves;
        int min_tpw;
        if (partition_tokens == 0) {
            waves = auto_waves(kv_dtype, head_size, tiling.head_tile, mfma, nseq, ub_tiles, cus);
            if (waves <= 0)
                return set_status(NXT_ATTN_E_HIP, "no occupancy for head_size %d %s", head_size,
                                  dtype_name(kv_dtype));
            min_tpw = kMinTilesPerWave;
        } else {
            min_tpw = partition_tokens / tile;
            waves = (ub_tiles + min_tpw - 1) / min_tpw;
            const int wpg = waves_per_group(mfma);
            waves = (waves + wpg - 1) / wpg * wpg;
            if (waves > kMaxWaves)
                return set_status(NXT_ATTN_E_UNSUPPORTED,
                                  "partition_tokens %d gives %lld wavefronts; raise it",
                                  partition_tokens, waves);
        }

        // Small batches on the VALU tile path: one round of workgroups over
        // the segments (paged_decode_segment_kernel) when they fit one per
        // CU, S of them per segment.  A workgroup streams its share of a
        // segment through one CU (~68 GB/s measured on MI355X), so a segment
        // is split while each share keeps at least kSegSplitBytes of K/V,
        // which one CU streams in about the time the merge launch then
        // needed takes (~2.3 us).  With S = 1 there is no split-K workspace
        // and no merge.  (Each load of a tile must lie in one page:
        // block_size >= its rows.)
        long long seg_split = 0;  // 0: the stream-K plan
        if (!mfma && partition_tokens == 0 && !po && !fold &&
            tiling.head_tile <= xhip::kSegMaxHeadTile && block_size >= tile / xhip::kLoadsPerTile &&
            (long long)nseq * segs <= cus) {
            constexpr long long kSegSplitBytes = 160 << 10;
            const long long cap = (long long)xhip::kSegWaves * xhip::kSegTiles * xhip::kSegRounds;
            const long long seg_tiles = (max_ctx + tile - 1) / tile;
            const long long seg_bytes = max_ctx * head_size * elem_bytes(kv_dtype) * 2;
            long long S = 1;
            while (S < 4 && (long long)nseq * segs * S * 2 <= cus &&
                   (seg_bytes / (S * 2) >= kSegSplitBytes || seg_tiles > S * cap))
                S *= 2;
            if (seg_tiles <= S * cap) seg_split = S;
        }
        const bool seg_launch = seg_split > 0;

        const size_t eb_total = (size_t)elem_bytes(kv_dtype);
        // workspace: fp32 partials o, their (m, l), the unit prefix; under a
        // split segment launch, one partial per workgroup
        const size_t pre_bytes = seg_launch ? 0 : (size_t)(nseq + 1) * sizeof(int);
        long long slots = seg_launch ? (seg_split > 1 ? nseq * segs * seg_split : 0)
                                     : 2 * waves;
        auto o_size = [&](long long n) {
            return ((size_t)n * tiling.head_tile * head_size * sizeof(float) + 255) & ~(size_t)255;
        };
        auto ml_size = [&](long long n) {
            return ((size_t)n * tiling.head_tile * 2 * sizeof(float) + 255) & ~(size_t)255;
        };
        if (fixed && partition_tokens == 0 && !seg_launch &&
            o_size(slots) + ml_size(slots) + pre_bytes > fixed->bytes) {
            // An automatic plan larger than the fixed scratch (a device with
            // more CUs than the scratch was sized for): fewer wavefronts, each
            // with a longer range.  Correct, though its cut points (and so
            // the last bits of the result) differ from the allocating entry
            // points' plan.
            const size_t per_wave =
                2 * (size_t)tiling.head_tile * ((size_t)head_size + 2) * sizeof(float);
            const int wpg = waves_per_group(mfma);
            const size_t room = fixed->bytes > pre_bytes + 512 ? fixed->bytes - pre_bytes - 512 : 0;
            long long w = (long long)(room / per_wave) / wpg * wpg;
            if (w >= wpg && w < waves) {
                waves = w;
                slots = 2 * waves;
            }
        }
        if (fixed && o_size(slots) + ml_size(slots) + pre_bytes > fixed->bytes)
            return set_status(NXT_ATTN_E_UNSUPPORTED,
                              "this plan needs %zu bytes of split-K scratch; the allocation-free "
                              "entry point has %zu%s",
                              o_size(slots) + ml_size(slots) + pre_bytes, fixed->bytes,
                              partition_tokens ? " (raise partition_tokens)" : "");
        const size_t o_bytes = o_size(slots);
        const size_t ml_bytes = ml_size(slots);
        WsCache::Lease lease;  // held until this chunk's launches are enqueued
        void *ws = nullptr;
        if (seg_launch && seg_split == 1) {
            // (no workspace)
        } else if (fixed) {
            ws = fixed->ptr;  // launches of one stream run in order: chunks reuse it
        } else {
            int st = get_workspace(device, stream, o_bytes + ml_bytes + pre_bytes, &lease);
            if (st != NXT_ATTN_OK) return st;
            ws = lease.ptr();
        }

        const size_t row0 = (size_t)s0 * num_heads * head_size * eb_total;
        DecodeParams p;
        memset(&p, 0, sizeof(p));
        p.out = out && !rows ? (char *)out + row0 : nullptr;
        p.q_rows = rows ? rows->q + s0 : nullptr;
        p.o_rows = rows ? rows->o + s0 : nullptr;
        if (po) {
            p.out_f32 = po->out_f32 + (size_t)s0 * num_heads * head_size;
            p.out_lse = po->out_lse + (size_t)s0 * num_heads;
            p.cached_seqs = po->cached_seqs > s0 ? po->cached_seqs - s0 : 0;
            p.skip_empty = po->skip_empty;
        }
        if (fold) {
            p.fold_row = fold->row + s0;
            p.fold_out = fold->out;
            p.fold_lse = fold->lse;
            p.fold_rows = fold->rows;
            p.fold_kr = fold->kr;
        }
        fill_batch(p, rows ? nullptr : (const char *)query + row0, key_cache, value_cache,
                   block_tables + (size_t)s0 * max_num_blocks_per_seq, seq_lens + s0, nseq,
                   num_heads, num_kv_heads, tiling.head_tiles, max_num_blocks_per_seq, block_size,
                   kv_block_stride, kv_head_stride, scale);
        p.ws_o = ws ? (float *)ws : nullptr;
        p.ws_ml = ws ? (float *)((char *)ws + o_bytes) : nullptr;
        p.ws_prefix = ws && !seg_launch ? (int *)((char *)ws + o_bytes + ml_bytes) : nullptr;
        p.wg_trace = t_wg_trace;
        p.segment_launch = seg_launch ? 1 : 0;
        p.segment_split = seg_launch ? (int)seg_split : 1;
        p.num_waves = (int)waves;
        p.min_tiles_per_wave = min_tpw;
        p.seg_cost = seg_cost;
        // the partition kernel combines cut segments inside its workgroups
        // (same predicate as the kernel instantiation's)
        p.wg_fix = mfma && xhip::mfma_wg_fixup(tiling.head_tile, head_size) != 0 ? 1 : 0;
        // One merge workgroup per segment once the segments alone fill two
        // workgroups per CU, or once the (segment, column chunk) grid would
        // launch more than four workgroups per CU (each costs ~2 ns of
        // dispatch; 32-head tiles have 32 chunks per segment at head_size
        // 128).  Fewer, longer segments of few heads (few sequences, long
        // contexts) take the chunk grid, whose 8 threads per column split
        // the many partials.
        const int mheads = group < tiling.head_tile ? group : tiling.head_tile;
        const long long chunks = (mheads * (head_size / 4) + xhip::kMergeCols - 1) / xhip::kMergeCols;
        p.merge_per_segment =
            ((long long)nseq * segs >= 2LL * cus || (long long)nseq * segs * chunks > 4LL * cus) ? 1
                                                                                                : 0;
        if (nt) {  // the fold lives in the chunk-grid merge
            p.merge_per_segment = 0;
            p.nt_fold = 1;
            p.nt_k = nt->k;
            p.nt_v = nt->v;
            p.nt_table = nt->table;
            p.nt_lens = nt->lens;
            p.nt_slot = nt->slot;
            p.nt_page = nt->page;
            p.nt_len = nt->len;
        }

        switch (kv_dtype) {
        case NXT_KV_FP16:
            e = xhip::launch_decode_f16(p, head_size, tiling.head_tile, mfma, stream,
                                        t_trace_start, t_trace_partition);
            break;
        case NXT_KV_BF16:
            e = xhip::launch_decode_bf16(p, head_size, tiling.head_tile, mfma, stream,
                                         t_trace_start, t_trace_partition);
            break;
        default:
            e = xhip::launch_decode_f32(p, head_size, tiling.head_tile, mfma, stream,
                                        t_trace_start, t_trace_partition);
            break;
        }
        if (e != hipSuccess)
            return set_status(NXT_ATTN_E_HIP, "kernel launch: %s", hipGetErrorString(e));
    }
    return ok();
}

// ------------------------------------------------------------ cascade decode
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int cascade_run(void *out, const void *query, const void *key_cache, const void *value_cache,
                const int *block_tables, const int *seq_lens, const int *prefix_group,
                const int *prefix_blocks, int max_groups, int num_seqs, int num_heads,
                int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
                int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype,
                nxt_stream_t stream_handle, const RowPtrs *rowp = nullptr) {
    if (max_groups < 0) return set_status(NXT_ATTN_E_INVALID, "max_groups %d < 0", max_groups);
    const int eb = (kv_dtype == NXT_KV_FP16 || kv_dtype == NXT_KV_BF16) ? 2 : 4;
    if (max_groups == 0 || num_seqs <= 0)  // nothing shared: the ordinary decode
        return run(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
                   head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, eb,
                   kv_block_stride, kv_head_stride, stream_handle, kv_dtype, 0, nullptr, nullptr,
                   nullptr, rowp);
    if (!prefix_group || !prefix_blocks)
        return set_status(NXT_ATTN_E_INVALID, "NULL prefix_group / prefix_blocks");
    if (num_seqs > xhip::kMaxSeqsPerLaunch || max_groups > num_seqs)
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "cascade batch of %d sequences / %d groups (limits %d, num_seqs)",
                          num_seqs, max_groups, xhip::kMaxSeqsPerLaunch);
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads ||
        !(rowp ? (const void *)rowp->o : out) || max_num_blocks_per_seq <= 0 || !is_pow2(block_size))
        return set_status(NXT_ATTN_E_INVALID, "bad cascade arguments");
    const int group = num_heads / num_kv_heads;
    // Query rows per kv head of a prefix-batch sequence: 64 (two 32-head
    // tiles, neighbouring segments of one sequence, which read the same
    // shared pages at the same offsets on one XCD) where the MFMA path serves
    // 32 heads per wavefront, else a multiple of the 16-head tile.
    constexpr int kCascadeWideRows = 4 * xhip::kCascadeRows;
    const bool wide = use_mfma(kv_dtype, head_size, block_size) &&
                      head_size <= xhip::kMfmaWideMaxHeadSize && group <= kCascadeWideRows;
    const int rows = wide ? kCascadeWideRows
                          : (group + xhip::kCascadeRows - 1) / xhip::kCascadeRows *
                                xhip::kCascadeRows;
    const long long v_max = ((long long)num_seqs * group + rows - 1) / rows + max_groups;
    const size_t mb = (size_t)max_num_blocks_per_seq;
    const size_t KR = (size_t)num_kv_heads * rows;
    if (v_max > xhip::kMaxSeqsPerLaunch)
        return set_status(NXT_ATTN_E_UNSUPPORTED,
                          "cascade prefix batch of %lld sequences (limit %d): fewer sequences "
                          "or groups per call",
                          v_max, xhip::kMaxSeqsPerLaunch);
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return set_status(NXT_ATTN_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    hipStream_t stream = (hipStream_t)stream_handle;

    // The MFMA path with 32-row prefix tiles runs both batches in one
    // partition launch of `fw` wavefronts and one merge
    // (paged_decode_cascade_attn.h); otherwise the two batches go through
    // run() one after the other, the suffix batch folding in the prefix rows.
    HeadTiling stile{};
    long long fw = 0;
    bool inplan = false;  // the partition launch plans both batches itself
    if (wide && supported_head_size(head_size) &&
        head_tiling(group, true, head_size, &stile)) {
        const long long tiles = ((long long)max_num_blocks_per_seq * block_size + 15) / 16 + kSegmentCost;
        const bool fits = v_max * (long long)num_kv_heads * (rows / 32) * tiles < kMaxLaunchTiles &&
                          (long long)num_seqs * num_kv_heads * stile.head_tiles * tiles <
                              kMaxLaunchTiles;
        const int rs = stile.head_tile / xhip::kMfmaHeads;
        auto occupancy = [&](bool ip, size_t lds) {
            return kv_dtype == NXT_KV_FP16 ? xhip::cascade_attn_occupancy_f16(head_size, rs, ip, lds)
                                           : xhip::cascade_attn_occupancy_bf16(head_size, rs, ip, lds);
        };
        int occ = 0;
        if (fits && max_groups <= xhip::kInPlanGroupsMax) {
            // (only where it keeps two workgroups per CU)
            occ = occupancy(true, xhip::inplan_lds_bytes(num_seqs, (int)v_max, max_groups));
            inplan = occ >= 2;
        }
        if (fits && !inplan) occ = occupancy(false, (size_t)(v_max + num_seqs + 2) * sizeof(int));
        if (occ > 0) {
            int per_cu = occ * xhip::kMfmaWavesPerGroup;
            if (per_cu > kMfmaWavesPerCu) per_cu = kMfmaWavesPerCu;
            fw = (long long)cu_count(device) * per_cu;
            if (fw < 2 * xhip::kMfmaWavesPerGroup) fw = 2 * xhip::kMfmaWavesPerGroup;
        }
    }
    // workspace layout (each piece 256-byte aligned)
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    // (the in-kernel plan needs only the batches' lengths and p_row of the
    // plan's arrays)
    const size_t pn = inplan ? 0 : 1;
    const size_t o_gc = take(4 * (size_t)max_groups * pn), o_gf = take(4 * (size_t)max_groups * pn),
                 o_gv = take(4 * (size_t)max_groups * pn), o_gm = take(4 * (size_t)max_groups * pn),
                 o_ms = take(4 * (size_t)num_seqs * pn), o_rk = take(4 * (size_t)num_seqs * pn),
                 o_vg = take(4 * (size_t)v_max * pn), o_vl = take(4 * (size_t)v_max),
                 o_vb = take(4 * (size_t)v_max * mb * pn),
                 o_vq = take((size_t)v_max * KR * head_size * eb * pn),
                 o_sl = take(4 * (size_t)num_seqs), o_sb = take(4 * (size_t)num_seqs * mb * pn),
                 o_po = take(4 * (size_t)v_max * KR * head_size), o_pl = take(4 * (size_t)v_max * KR),
                 o_pr = take(4 * (size_t)num_seqs), o_vd = take(4 * 8 * (size_t)v_max * pn),
                 o_spb = take(4 * (size_t)num_seqs * pn);
    // one launch over both batches: each batch's split-K workspace (partials
    // for up to every wavefront, unit prefix), and the suffix batch's rows
    const size_t gts = (size_t)stile.head_tile;
    const size_t o_xo = fw ? take(4 * 2 * (size_t)fw * 32 * head_size) : 0,
                 o_xm = fw ? take(4 * 2 * (size_t)fw * 32 * 2) : 0,
                 o_xp = fw ? take(4 * ((size_t)v_max + 2)) : 0,
                 o_yo = fw ? take(4 * 2 * (size_t)fw * gts * head_size) : 0,
                 o_ym = fw ? take(4 * 2 * (size_t)fw * gts * 2) : 0,
                 o_yp = fw ? take(4 * ((size_t)num_seqs + 1)) : 0,
                 o_so = fw ? take(4 * (size_t)num_seqs * num_heads * head_size) : 0,
                 o_sl2 = fw ? take(4 * (size_t)num_seqs * num_heads) : 0;
    // held over the plan and both passes (they read what the plan wrote)
    WsCache::Lease lease;
    int st = get_workspace(device, stream, off, &lease, kWsCascade);
    if (st != NXT_ATTN_OK) return st;
    char *w = (char *)lease.ptr();
    xhip::CascadeParams c;
    memset(&c, 0, sizeof(c));
    c.block_tables = block_tables;
    c.seq_lens = seq_lens;
    c.q = query;
    c.q_rows = rowp ? rowp->q : nullptr;
    c.out = out;
    c.prefix_group = prefix_group;
    c.prefix_blocks = prefix_blocks;
    c.num_seqs = num_seqs;
    c.num_heads = num_heads;
    c.num_kv_heads = num_kv_heads;
    c.group = group;
    c.head_size = head_size;
    c.elem_bytes = eb;
    c.kv_dtype = kv_dtype;
    c.max_blocks = max_num_blocks_per_seq;
    c.block_size = block_size;
    c.max_ctx = (int)((long long)max_num_blocks_per_seq * block_size);
    c.max_groups = max_groups;
    c.rows = rows;
    c.v_max = (int)v_max;
    c.g_count = (int *)(w + o_gc);
    c.g_first = (int *)(w + o_gf);
    c.g_vbase = (int *)(w + o_gv);
    c.g_moff = (int *)(w + o_gm);
    c.member_seq = (int *)(w + o_ms);
    c.rank = (int *)(w + o_rk);
    c.v_group = (int *)(w + o_vg);
    c.v_lens = (int *)(w + o_vl);
    c.v_bt = (int *)(w + o_vb);
    c.v_q = w + o_vq;
    c.s_lens = (int *)(w + o_sl);
    c.s_bt = (int *)(w + o_sb);
    c.p_row = (int *)(w + o_pr);
    c.v_desc = (int *)(w + o_vd);
    c.s_pblk = (int *)(w + o_spb);
    // plan -> prefix pass (R gathered query rows per kv head, cacheable K/V:
    // the rows of a group read the same pages) -> suffix pass, whose members
    // start from their prefix rows and which writes the output; or, with the
    // in-kernel plan, one partition launch that plans both batches itself
    if (!inplan) {
        e = xhip::launch_cascade_plan(c, stream);
        if (e != hipSuccess)
            return set_status(NXT_ATTN_E_HIP, "cascade plan launch: %s", hipGetErrorString(e));
    }
    if (fw) {
        DecodeParams pp, ps;
        memset(&pp, 0, sizeof(pp));
        memset(&ps, 0, sizeof(ps));
        // (in-kernel plan: the batches' lengths are the workspace arrays the
        // partition launch fills for the merge; tables and query rows are
        // the caller's, read in place)
        fill_batch(pp, inplan ? nullptr : c.v_q, key_cache, value_cache,
                   inplan ? block_tables : c.v_bt, c.v_lens, (int)v_max, (int)KR, num_kv_heads,
                   rows / 32, max_num_blocks_per_seq, block_size, kv_block_stride,
                   kv_head_stride, scale);
        fill_batch(ps, rowp ? nullptr : query, key_cache, value_cache,
                   inplan ? block_tables : c.s_bt, c.s_lens, num_seqs, num_heads, num_kv_heads,
                   stile.head_tiles, max_num_blocks_per_seq, block_size, kv_block_stride,
                   kv_head_stride, scale);
        ps.out = rowp ? nullptr : out;  // the merge's output rows
        ps.q_rows = rowp ? rowp->q : nullptr;
        ps.o_rows = rowp ? rowp->o : nullptr;
        for (DecodeParams *q : {&pp, &ps}) {
            q->num_waves = (int)fw;
            q->min_tiles_per_wave = kMinTilesPerWave;
            q->seg_cost = kSegmentCost;
            q->wg_fix = 1;
            q->skip_empty = 1;  // merged from the other batch, or zeros, by the merge
        }
        pp.wg_trace = ps.wg_trace = t_wg_trace;
        pp.pair_tiles = 1;  // the two 32-row head tiles share each range
        pp.wg_fix = 0;
        pp.out_f32 = (float *)(w + o_po);
        pp.out_lse = (float *)(w + o_pl);
        pp.cached_seqs = (int)v_max;  // a group's rows read its pages close in time
        pp.ws_o = (float *)(w + o_xo);
        pp.ws_ml = (float *)(w + o_xm);
        pp.ws_prefix = (int *)(w + o_xp);
        ps.out_f32 = (float *)(w + o_so);
        ps.out_lse = (float *)(w + o_sl2);
        ps.ws_o = (float *)(w + o_yo);
        ps.ws_ml = (float *)(w + o_ym);
        ps.ws_prefix = (int *)(w + o_yp);
        if (kv_dtype == NXT_KV_FP16) {
            // fp16 states, in the same (fp32-sized) buffers
            for (DecodeParams *q : {&pp, &ps}) {
                q->out_h = q->out_f32;
                q->ws_h = q->ws_o;
                q->out_f32 = nullptr;
                q->ws_o = nullptr;
            }
        }
        const int rs = stile.head_tile / xhip::kMfmaHeads;
        const xhip::CascadeInPlan ip{seq_lens, block_tables, prefix_group, prefix_blocks,
                                     max_groups};
        const xhip::CascadeInPlan *ipp = inplan ? &ip : nullptr;
        e = kv_dtype == NXT_KV_FP16
                ? xhip::launch_cascade_attn_f16(pp, ps, c.p_row, rows, head_size, rs, ipp, stream,
                                                t_trace_start, t_trace_partition)
                : xhip::launch_cascade_attn_bf16(pp, ps, c.p_row, rows, head_size, rs, ipp,
                                                 stream, t_trace_start, t_trace_partition);
        if (e != hipSuccess)
            return set_status(NXT_ATTN_E_HIP, "cascade attention launch: %s", hipGetErrorString(e));
        return ok();
    }
    // (the prefix batch's empty sequences are the reserved ones no group
    // uses: nothing reads their rows)
    const PartialOut pre{(float *)(w + o_po), (float *)(w + o_pl), (int)v_max, 1};
    st = run(nullptr, c.v_q, key_cache, value_cache, c.v_bt, c.v_lens, (int)v_max,
             num_kv_heads * rows, head_size, num_kv_heads, scale, max_num_blocks_per_seq,
             block_size, eb, kv_block_stride, kv_head_stride, stream_handle, kv_dtype, 0, &pre);
    if (st != NXT_ATTN_OK) return st;
    const PrefixFold fold{c.p_row, (const float *)(w + o_po), (const float *)(w + o_pl), rows,
                          (int)KR};
    return run(out, query, key_cache, value_cache, c.s_bt, c.s_lens, num_seqs, num_heads,
               head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, eb,
               kv_block_stride, kv_head_stride, stream_handle, kv_dtype, 0, nullptr, &fold,
               nullptr, rowp);
}

// KV append (decode: block_tables + positions; prefill: slots).
int kv_append_run(void *key_cache, void *value_cache, const void *key, const void *value,
                  const int *slots, const int *block_tables, const int *positions, int num_tokens,
                  int num_kv_heads, int head_size, int max_num_blocks_per_seq, int block_size,
                  int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream_handle,
                  const int *src_slots = nullptr) {
    if (kv_dtype != NXT_KV_FP16 && kv_dtype != NXT_KV_BF16 && kv_dtype != NXT_KV_FP32)
        return set_status(NXT_ATTN_E_INVALID, "kv_dtype %d is not FP16/BF16/FP32", kv_dtype);
    if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || kv_block_stride < 0 ||
        kv_head_stride < 0 || (!slots && max_num_blocks_per_seq <= 0))
        return set_status(NXT_ATTN_E_INVALID, "bad sizes (tokens %d, kv heads %d, block_size %d)",
                          num_tokens, num_kv_heads, block_size);
    if (!supported_head_size(head_size))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "head_size %d not supported", head_size);
    if (!is_pow2(block_size) || block_size > 1024)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "block_size %d is not a power of two <= 1024",
                          block_size);
    const long long max_ctx = slots ? 0 : (long long)max_num_blocks_per_seq * block_size;
    if (max_ctx > (1LL << 28))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "context bound %lld tokens too large", max_ctx);
    if (num_tokens == 0) return ok();
    if (!key_cache || !value_cache || !key || !value || (!slots && (!block_tables || !positions)))
        return set_status(NXT_ATTN_E_INVALID, "NULL pointer");
    const int eb = elem_bytes(kv_dtype);
    const long long bstride = (long long)kv_block_stride * eb, hstride = (long long)kv_head_stride * eb;
    if (((uintptr_t)key_cache | (uintptr_t)value_cache | (uintptr_t)key | (uintptr_t)value) & 15 ||
        (bstride & 15) || (hstride & 15))
        return set_status(NXT_ATTN_E_UNSUPPORTED, "tensors and kv strides must be 16-byte aligned");
    xhip::KvAppendParams p;
    memset(&p, 0, sizeof(p));
    p.key_cache = key_cache;
    p.value_cache = value_cache;
    p.key = key;
    p.value = value;
    p.slots = slots;
    p.src_slots = src_slots;
    p.block_tables = block_tables;
    p.positions = positions;
    p.kv_block_stride_bytes = bstride;
    p.kv_head_stride_bytes = hstride;
    p.num_tokens = num_tokens;
    p.num_kv_heads = num_kv_heads;
    p.row_bytes = head_size * eb;
    p.row_chunks = p.row_bytes / 16;
    p.block_size = block_size;
    p.bs_shift = ilog2(block_size);
    p.max_blocks = max_num_blocks_per_seq;
    p.max_ctx = (int)max_ctx;
    const hipError_t e = xhip::launch_kv_append(p, (hipStream_t)stream_handle);
    if (e != hipSuccess)
        return set_status(NXT_ATTN_E_HIP, "kv append launch: %s", hipGetErrorString(e));
    return ok();
}

int dtype_from_size(int dtype_size) {
    if (dtype_size == 2) return NXT_KV_FP16;
    if (dtype_size == 4) return NXT_KV_FP32;
    return 0;
}

// ------------------------------------------------------------- activations
// Largest number of 16-byte output chunks one vector launch covers: one lane
// per chunk, and a launch's work-items and the kernel's indices are 32-bit.
constexpr long long kActMaxChunks = (1LL << 31) - 1;

int activation_run(int op, void *out, const void *input, long long num_tokens, int d, int dtype,
                   nxt_stream_t stream_handle) {
    if (op < NXT_ACT_SILU_AND_MUL || op > NXT_ACT_SILU)
        return set_status(NXT_ATTN_E_INVALID, "activation op %d is not an NxtActivationOp", op);
    if (dtype != NXT_KV_FP16 && dtype != NXT_KV_BF16 && dtype != NXT_KV_FP32)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "dtype %d is not FP16/BF16/FP32", dtype);
    if (num_tokens < 0 || d < 0)
        return set_status(NXT_ATTN_E_INVALID, "num_tokens %lld / d %d must be >= 0", num_tokens, d);
    if (num_tokens == 0 || d == 0) return ok();
    if (!out || !input) return set_status(NXT_ATTN_E_INVALID, "NULL tensor pointer");
    const int eb = elem_bytes(dtype);
    if (((uintptr_t)out | (uintptr_t)input) % (uintptr_t)eb)
        return set_status(NXT_ATTN_E_INVALID, "tensors must be aligned to their element size");
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return set_status(NXT_ATTN_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    const int cus = cu_count(device);
    const long long row_bytes = (long long)d * eb;
    const bool vec = row_bytes % 16 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)input % 16) == 0;
    const int in_row_mult = xhip::act_is_gated(op) ? 2 : 1;
    xhip::ActivationParams p;
    memset(&p, 0, sizeof(p));
    p.d = d;
    p.dtype = dtype;
    p.op = op;
    if (!vec) {
        p.out = out;
        p.input = input;
        p.num_tokens = num_tokens;
        e = xhip::launch_activation(p, false, cus, (hipStream_t)stream_handle);
        if (e != hipSuccess)
            return set_status(NXT_ATTN_E_HIP, "activation launch: %s", hipGetErrorString(e));
        return ok();
    }
    // Vector path: rows split into launches of < 2^31 output chunks each.
    const long long rc = row_bytes / 16;
    const long long rows_per_launch = kActMaxChunks / rc;
    p.row_chunks = xhip::div_magic((uint32_t)rc);
    for (long long t0 = 0; t0 < num_tokens; t0 += rows_per_launch) {
        const long long rows = num_tokens - t0 < rows_per_launch ? num_tokens - t0 : rows_per_launch;
        p.out = (char *)out + t0 * row_bytes;
        p.input = (const char *)input + t0 * row_bytes * in_row_mult;
        p.num_tokens = rows;
        p.chunks = (uint32_t)(rows * rc);
        e = xhip::launch_activation(p, true, cus, (hipStream_t)stream_handle);
        if (e != hipSuccess)
            return set_status(NXT_ATTN_E_HIP, "activation launch: %s", hipGetErrorString(e));
    }
    return ok();
}

void activation_legacy(int op, void *out, const void *input, int num_tokens, int d, int dtype_size,
                       nxt_stream_t stream) {
    const int dtype = dtype_from_size(dtype_size);
    if (!dtype) {
        set_status(NXT_ATTN_E_UNSUPPORTED, "dtype_size %d is not 2 (fp16) or 4 (fp32)", dtype_size);
        return;
    }
    (void)activation_run(op, out, input, num_tokens, d, dtype, stream);
}

void run_legacy(void *out, const void *query, const void *key_cache, const void *value_cache,
                const int *block_tables, const int *seq_lens, int num_seqs, int num_heads,
                int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
                int block_size, int dtype_size, int kv_block_stride, int kv_head_stride,
                nxt_stream_t stream) {
    const int kv_dtype = dtype_from_size(dtype_size);
    if (!kv_dtype) {
        set_status(NXT_ATTN_E_UNSUPPORTED, "dtype_size %d is not 2 (fp16) or 4 (fp32)", dtype_size);
        return;
    }
    (void)run(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
              head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, dtype_size,
              kv_block_stride, kv_head_stride, stream, kv_dtype, 0);
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) void nxt_paged_attention(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
    int kv_block_stride, int kv_head_stride, nxt_stream_t stream) {
    run_legacy(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
               head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, dtype_size,
               kv_block_stride, kv_head_stride, stream);
}

__attribute__((visibility("default"))) void nxt_paged_attention_v2(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
    int kv_block_stride, int kv_head_stride, nxt_stream_t stream) {
    run_legacy(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
               head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, dtype_size,
               kv_block_stride, kv_head_stride, stream);
}

__attribute__((visibility("default"))) void nxt_paged_attention_flash(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
    int kv_block_stride, int kv_head_stride, nxt_stream_t stream) {
    run_legacy(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
               head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, dtype_size,
               kv_block_stride, kv_head_stride, stream);
}

__attribute__((visibility("default"))) int nxt_paged_attention_ex(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
    int kv_block_stride, int kv_head_stride, nxt_stream_t stream, int kv_dtype,
    int partition_tokens) {
    return run(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs, num_heads,
               head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, dtype_size,
               kv_block_stride, kv_head_stride, stream, kv_dtype, partition_tokens);
}

__attribute__((visibility("default"))) int nxt_paged_attention_noalloc(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size, int dtype_size,
    int kv_block_stride, int kv_head_stride, nxt_stream_t stream, int kv_dtype,
    int partition_tokens) {
    // shape checks before the scratch lookup (pointer checks follow in the
    // real run, still before any launch)
    if (num_seqs < 0) return set_status(NXT_ATTN_E_INVALID, "num_seqs %d < 0", num_seqs);
    const int st = run(out, query, key_cache, value_cache, block_tables, seq_lens, 0, num_heads,
                       head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size,
                       dtype_size, kv_block_stride, kv_head_stride, stream, kv_dtype,
                       partition_tokens);
    if (st != NXT_ATTN_OK || num_seqs == 0) return st;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return set_status(NXT_ATTN_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    FixedWs fixed{nullptr, 0};
    e = xhip::noalloc_scratch(device, &fixed.ptr, &fixed.bytes);
    if (e != hipSuccess)
        return set_status(NXT_ATTN_E_HIP, "scratch address of device %d: %s", device,
                          hipGetErrorString(e));
    // calls on one device run one after another on the GPU (noalloc_gate.h)
    NoAllocGate::Pass pass;
    if (g_noalloc_gate.enter(device, stream, &pass) != NoAllocGate::kOk)
        return set_status(NXT_ATTN_E_HIP,
                          "ordering after the device's previous no-alloc call failed");
    const int rc = run(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs,
                       num_heads, head_size, num_kv_heads, scale, max_num_blocks_per_seq,
                       block_size, dtype_size, kv_block_stride, kv_head_stride, stream, kv_dtype,
                       partition_tokens, nullptr, nullptr, &fixed);
    if (pass.done() != NoAllocGate::kOk && rc == NXT_ATTN_OK)
        return set_status(NXT_ATTN_E_HIP, "recording the no-alloc call's completion event failed");
    return rc;
}

__attribute__((visibility("default"))) int nxt_paged_attention_auto_waves(
    int num_seqs, int num_heads, int head_size, int num_kv_heads, int max_num_blocks_per_seq,
    int block_size, int kv_dtype) {
    if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
        !supported_head_size(head_size) || max_num_blocks_per_seq <= 0 || block_size <= 0 ||
        (kv_dtype != NXT_KV_FP16 && kv_dtype != NXT_KV_BF16 && kv_dtype != NXT_KV_FP32))
        return NXT_ATTN_E_INVALID;
    if (!is_pow2(block_size)) return NXT_ATTN_E_UNSUPPORTED;
    const bool mfma = use_mfma(kv_dtype, head_size, block_size);
    HeadTiling tiling;
    if (!head_tiling(num_heads / num_kv_heads, mfma, head_size, &tiling))
        return NXT_ATTN_E_UNSUPPORTED;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return NXT_ATTN_E_HIP;
    const int nseq = num_seqs < xhip::kMaxSeqsPerLaunch ? num_seqs : xhip::kMaxSeqsPerLaunch;
    const int tile = tile_tokens(head_size, kv_dtype, mfma);
    const long long ub = (long long)nseq * num_kv_heads * tiling.head_tiles *
                         (((long long)max_num_blocks_per_seq * block_size + tile - 1) / tile +
                          kSegmentCost);
    const long long w = auto_waves(kv_dtype, head_size, tiling.head_tile, mfma, nseq, ub,
                                   cu_count(device));
    return w > 0 ? (int)w : NXT_ATTN_E_HIP;
}

__attribute__((visibility("default"))) int nxt_paged_kv_append(
    void *key_cache, void *value_cache, const void *key, const void *value,
    const int *block_tables, const int *positions, int num_seqs, int num_kv_heads, int head_size,
    int max_num_blocks_per_seq, int block_size, int kv_block_stride, int kv_head_stride,
    int kv_dtype, nxt_stream_t stream) {
    return kv_append_run(key_cache, value_cache, key, value, nullptr, block_tables, positions,
                         num_seqs, num_kv_heads, head_size, max_num_blocks_per_seq, block_size,
                         kv_block_stride, kv_head_stride, kv_dtype, stream);
}

__attribute__((visibility("default"))) int nxt_paged_kv_write_slots(
    void *key_cache, void *value_cache, const void *key, const void *value,
    const int *slot_mapping, int num_tokens, int num_kv_heads, int head_size, int block_size,
    int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream) {
    if (!slot_mapping && num_tokens > 0) return set_status(NXT_ATTN_E_INVALID, "NULL slot_mapping");
    return kv_append_run(key_cache, value_cache, key, value, slot_mapping, nullptr, nullptr,
                         num_tokens, num_kv_heads, head_size, 0, block_size, kv_block_stride,
                         kv_head_stride, kv_dtype, stream);
}

__attribute__((visibility("default"))) int nxt_paged_kv_copy_slots(
    void *key_cache, void *value_cache, const int *src_slots, const int *dst_slots, int num_tokens,
    int num_kv_heads, int head_size, int block_size, int kv_block_stride, int kv_head_stride,
    int kv_dtype, nxt_stream_t stream) {
    if ((!src_slots || !dst_slots) && num_tokens > 0)
        return set_status(NXT_ATTN_E_INVALID, "NULL slot list");
    return kv_append_run(key_cache, value_cache, key_cache, value_cache, dst_slots, nullptr,
                         nullptr, num_tokens, num_kv_heads, head_size, 0, block_size,
                         kv_block_stride, kv_head_stride, kv_dtype, stream, src_slots);
}

#define XLLM_ACTIVATION_ENTRY(name, op)                                                            \
    __attribute__((visibility("default"))) void name(void *out, const void *input, int num_tokens, \
                                                     int d, int dtype_size, nxt_stream_t stream) { \
        activation_legacy(op, out, input, num_tokens, d, dtype_size, stream);                      \
    }
XLLM_ACTIVATION_ENTRY(nxt_silu_and_mul, NXT_ACT_SILU_AND_MUL)
XLLM_ACTIVATION_ENTRY(nxt_mul_and_silu, NXT_ACT_MUL_AND_SILU)
XLLM_ACTIVATION_ENTRY(nxt_gelu_and_mul, NXT_ACT_GELU_AND_MUL)
XLLM_ACTIVATION_ENTRY(nxt_gelu_tanh_and_mul, NXT_ACT_GELU_TANH_AND_MUL)
XLLM_ACTIVATION_ENTRY(nxt_gelu_elementwise, NXT_ACT_GELU)
XLLM_ACTIVATION_ENTRY(nxt_silu_elementwise, NXT_ACT_SILU)
#undef XLLM_ACTIVATION_ENTRY

__attribute__((visibility("default"))) int nxt_activation_ex(int op, void *out, const void *input,
                                                             int64_t num_tokens, int d, int dtype,
                                                             nxt_stream_t stream) {
    return activation_run(op, out, input, num_tokens, d, dtype, stream);
}

}  // extern "C"

namespace {

// nxt_paged_attention_cascade's checks and run, with contiguous query / out
// or per-sequence rows (rowp).
int cascade_entry(void *out, const void *query, const RowPtrs *rowp, const void *key_cache,
                  const void *value_cache, const int *block_tables, const int *seq_lens,
                  const int *prefix_group, const int *prefix_blocks, int max_groups, int num_seqs,
                  int num_heads, int head_size, int num_kv_heads, float scale,
                  int max_num_blocks_per_seq, int block_size, int kv_block_stride,
                  int kv_head_stride, int kv_dtype, nxt_stream_t stream) {
    // the ordinary path's argument checks, without launching anything
    const int eb = (kv_dtype == NXT_KV_FP16 || kv_dtype == NXT_KV_BF16) ? 2 : 4;
    int st = run(out, query, key_cache, value_cache, block_tables, seq_lens, 0, num_heads,
                 head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size, eb,
                 kv_block_stride, kv_head_stride, stream, kv_dtype, 0);
    if (st != NXT_ATTN_OK) return st;
    if (num_seqs < 0) return set_status(NXT_ATTN_E_INVALID, "num_seqs %d < 0", num_seqs);
    if (num_seqs == 0) return ok();
    // the checks run() makes only for a non-empty batch: the cascade plan
    // reads these arrays before any pass of run() is reached
    const void *o_any = rowp ? (const void *)rowp->o : out;
    const void *q_any = rowp ? (const void *)rowp->q : query;
    if (!o_any || !q_any || !key_cache || !value_cache || !block_tables || !seq_lens)
        return set_status(NXT_ATTN_E_INVALID, "NULL tensor pointer");
    if (max_groups > 0 && (!prefix_group || !prefix_blocks))
        return set_status(NXT_ATTN_E_INVALID, "NULL prefix_group / prefix_blocks");
    if (((uintptr_t)(rowp ? nullptr : out) | (uintptr_t)(rowp ? nullptr : query) |
         (uintptr_t)key_cache | (uintptr_t)value_cache) & 15)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "tensors must be 16-byte aligned");
    if (rowp && (((uintptr_t)rowp->q | (uintptr_t)rowp->o) & 7))
        return set_status(NXT_ATTN_E_INVALID, "row pointer tables must be 8-byte aligned");
    if (((uintptr_t)block_tables | (uintptr_t)seq_lens | (uintptr_t)prefix_group |
         (uintptr_t)prefix_blocks) & 3)
        return set_status(NXT_ATTN_E_INVALID, "int32 arrays must be 4-byte aligned");
    return cascade_run(out, query, key_cache, value_cache, block_tables, seq_lens, prefix_group,
                       prefix_blocks, max_groups, num_seqs, num_heads, head_size, num_kv_heads,
                       scale, max_num_blocks_per_seq, block_size, kv_block_stride,
                       kv_head_stride, kv_dtype, stream, rowp);
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int nxt_paged_attention_cascade(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_tables, const int *seq_lens, const int *prefix_group,
    const int *prefix_blocks, int max_groups, int num_seqs, int num_heads, int head_size,
    int num_kv_heads, float scale, int max_num_blocks_per_seq, int block_size,
    int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream) {
    return cascade_entry(out, query, nullptr, key_cache, value_cache, block_tables, seq_lens,
                         prefix_group, prefix_blocks, max_groups, num_seqs, num_heads, head_size,
                         num_kv_heads, scale, max_num_blocks_per_seq, block_size,
                         kv_block_stride, kv_head_stride, kv_dtype, stream);
}

__attribute__((visibility("hidden"))) int xhip_paged_attention_rows(
    const char *const *q_rows, char *const *o_rows, const void *key_cache,
    const void *value_cache, const int *block_tables, const int *seq_lens, int num_seqs,
    int num_heads, int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
    int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream) {
    const RowPtrs rows{q_rows, o_rows};
    return run(nullptr, nullptr, key_cache, value_cache, block_tables, seq_lens, num_seqs,
               num_heads, head_size, num_kv_heads, scale, max_num_blocks_per_seq, block_size,
               elem_bytes(kv_dtype), kv_block_stride, kv_head_stride, stream, kv_dtype, 0,
               nullptr, nullptr, nullptr, &rows);
}

__attribute__((visibility("hidden"))) int xhip_paged_attention_fold_new(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_table, const int *seq_len, float *state_rows, float *state_lse,
    const void *new_k, const void *new_v, int *new_table_entry, int *new_len_entry, int new_slot,
    int new_page, int new_len, int num_heads, int head_size, int num_kv_heads, float scale,
    int max_num_blocks_per_seq, int block_size, int kv_block_stride, int kv_head_stride,
    int kv_dtype, nxt_stream_t stream) {
    if (!state_rows || !state_lse || new_slot < 0 || new_page < 0 || new_len < 1)
        return set_status(NXT_ATTN_E_INVALID, "bad new-token fold arguments");
    const PartialOut po{state_rows, state_lse, 0, 0};
    const NewTokenFold nt{new_k, new_v, new_table_entry, new_len_entry, new_slot, new_page,
                          new_len};
    return run(out, query, key_cache, value_cache, block_table, seq_len, 1, num_heads, head_size,
               num_kv_heads, scale, max_num_blocks_per_seq, block_size, elem_bytes(kv_dtype),
               kv_block_stride, kv_head_stride, stream, kv_dtype, 0, &po, nullptr, nullptr,
               nullptr, &nt);
}

__attribute__((visibility("hidden"))) int xhip_paged_attention_cascade_rows(
    const char *const *q_rows, char *const *o_rows, const void *key_cache,
    const void *value_cache, const int *block_tables, const int *seq_lens,
    const int *prefix_group, const int *prefix_blocks, int max_groups, int num_seqs,
    int num_heads, int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
    int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream) {
    const RowPtrs rows{q_rows, o_rows};
    return cascade_entry(nullptr, nullptr, &rows, key_cache, value_cache, block_tables, seq_lens,
                         prefix_group, prefix_blocks, max_groups, num_seqs, num_heads, head_size,
                         num_kv_heads, scale, max_num_blocks_per_seq, block_size,
                         kv_block_stride, kv_head_stride, kv_dtype, stream);
}

__attribute__((visibility("default"))) int nxt_paged_prefix_groups(
    const int *block_tables, const int *seq_lens, int num_seqs, int max_num_blocks_per_seq,
    int block_size, int *prefix_group, int *prefix_blocks, int *num_groups, nxt_stream_t stream) {
    if (num_seqs < 0 || num_seqs > xhip::kCascadeMaxSeqs)
        return set_status(NXT_ATTN_E_UNSUPPORTED, "prefix detection handles 0..%d sequences",
                          xhip::kCascadeMaxSeqs);
    if (max_num_blocks_per_seq <= 0 || !is_pow2(block_size) || block_size > 1024 ||
        (long long)max_num_blocks_per_seq * block_size > (1LL << 28))
        return set_status(NXT_ATTN_E_INVALID, "bad table shape (%d blocks of %d)",
                          max_num_blocks_per_seq, block_size);
    if (!block_tables || !seq_lens || !prefix_group || !prefix_blocks || !num_groups)
        return set_status(NXT_ATTN_E_INVALID, "NULL pointer");
    const hipError_t e = xhip::launch_prefix_detect(block_tables, seq_lens, num_seqs,
                                                    max_num_blocks_per_seq, block_size,
                                                    prefix_group, prefix_blocks, num_groups,
                                                    (hipStream_t)stream);
    if (e != hipSuccess)
        return set_status(NXT_ATTN_E_HIP, "prefix detection launch: %s", hipGetErrorString(e));
    return ok();
}

__attribute__((visibility("default"))) int nxt_attn_last_status(void) { return t_status; }

__attribute__((visibility("default"))) const char *nxt_attn_last_error(void) { return t_message; }

#if XHIP_WG_TRACE
// Measurement build only (libxllm_hip_backend_trace.so): the calling thread's
// next calls stamp per-workgroup timestamps into `buffer` (device memory of
// xhip::kWgTraceBufferWords 64-bit words, layout in wg_trace.h); NULL stops.
__attribute__((visibility("default"))) void xhip_set_wg_trace(void *buffer) {
    t_wg_trace = (unsigned long long *)buffer;
}
__attribute__((visibility("default"))) unsigned long long xhip_wg_trace_words() {
    return xhip::kWgTraceBufferWords;
}
#endif

__attribute__((visibility("default"))) void nxt_attn_set_trace_events(void *start_event,
                                                                    void *partition_done_event) {
    t_trace_start = (hipEvent_t)start_event;
    t_trace_partition = (hipEvent_t)partition_done_event;
}

__attribute__((visibility("default"))) int nxt_attn_release_workspaces(void) {
    return g_ws.release_all() == WsCache::kOk ? NXT_ATTN_OK : NXT_ATTN_E_HIP;
}

const void *xhip_set_workspace_owner(const void *owner) {
    const void *prev = t_ws_owner;
    t_ws_owner = owner;
    return prev;
}

int xhip_release_owner_workspaces(const void *owner) {
    return g_ws.release_owner(owner) == WsCache::kOk ? 0 : -1;
}

int xhip_release_stream_workspaces(int device, void *stream) {
    return g_ws.release_stream(device, stream) == WsCache::kOk ? 0 : -1;
}

__attribute__((visibility("default"))) const char *nxt_attn_version(void) {
    return "xllm-hip-attn 0.1.0 gfx950";
}

}  // extern "C"
