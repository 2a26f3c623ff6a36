// Per-workgroup timeline of the decode kernels, for the instrumented
// measurement build only (compiled with XHIP_WG_TRACE=1 into
// libxllm_hip_backend_trace.so; the product library compiles every stamp
// below to nothing).  Timestamps are s_memrealtime, the device's constant
// 100 MHz clock, comparable across CUs and XCDs.
//
// Layout of the buffer DecodeParams::wg_trace points at (unsigned 64-bit
// words), filled by one traced call:
//   partition launch, record b (physical workgroup b), 16 words at 16 * b:
//     [0] entry  [1] prologue done (split-unit scan / plan)  [2] exit
//     [3] logical workgroup | role << 32 (cascade: 1 prefix body, 2 suffix)
//     [4 + 3w] wavefront w's first tile issued  [5 + 3w] its last tile done
//     [6 + 3w] tiles | pieces << 32
//   merge launch, record b at kWgTraceMergeBase + 2 * b:
//     [0] entry  [1] exit
#pragma once

namespace xhip {

constexpr int kWgTraceWords = 16;
constexpr unsigned long long kWgTraceMaxGroups = 4096;
constexpr unsigned long long kWgTraceMergeBase = kWgTraceMaxGroups * kWgTraceWords;
constexpr unsigned long long kWgTraceMergeMax = 65536;
constexpr unsigned long long kWgTraceBufferWords = kWgTraceMergeBase + 2 * kWgTraceMergeMax;

}  // namespace xhip

#if defined(XHIP_WG_TRACE) && XHIP_WG_TRACE
#define XHIP_TRACING 1
// word `idx` of partition record blockIdx.x (one lane writes)
#define XHIP_WG_STAMP(p, idx)                                                                  \
    do {                                                                                       \
        if ((p).wg_trace && threadIdx.x == 0 && blockIdx.x < ::xhip::kWgTraceMaxGroups)        \
            (p).wg_trace[blockIdx.x * ::xhip::kWgTraceWords + (idx)] =                         \
                __builtin_amdgcn_s_memrealtime();                                              \
    } while (0)
#define XHIP_WG_PUT(p, idx, value)                                                             \
    do {                                                                                       \
        if ((p).wg_trace && threadIdx.x == 0 && blockIdx.x < ::xhip::kWgTraceMaxGroups)        \
            (p).wg_trace[blockIdx.x * ::xhip::kWgTraceWords + (idx)] =                         \
                (unsigned long long)(value);                                                   \
    } while (0)
// word `idx` of wavefront `wave`'s part of the record (lane 0 of the wavefront)
#define XHIP_WAVE_STAMP(p, wave, idx)                                                          \
    do {                                                                                       \
        if ((p).wg_trace && (threadIdx.x & 63) == 0 && blockIdx.x < ::xhip::kWgTraceMaxGroups) \
            (p).wg_trace[blockIdx.x * ::xhip::kWgTraceWords + 4 + 3 * (wave) + (idx)] =        \
                __builtin_amdgcn_s_memrealtime();                                              \
    } while (0)
#define XHIP_WAVE_PUT(p, wave, idx, value)                                                     \
    do {                                                                                       \
        if ((p).wg_trace && (threadIdx.x & 63) == 0 && blockIdx.x < ::xhip::kWgTraceMaxGroups) \
            (p).wg_trace[blockIdx.x * ::xhip::kWgTraceWords + 4 + 3 * (wave) + (idx)] =        \
                (unsigned long long)(value);                                                   \
    } while (0)
#define XHIP_MERGE_STAMP(p, idx)                                                               \
    do {                                                                                       \
        const unsigned long long b_ = (unsigned long long)blockIdx.x +                         \
                                      (unsigned long long)blockIdx.y * gridDim.x;              \
        if ((p).wg_trace && threadIdx.x == 0 && b_ < ::xhip::kWgTraceMergeMax)                 \
            (p).wg_trace[::xhip::kWgTraceMergeBase + 2 * b_ + (idx)] =                         \
                __builtin_amdgcn_s_memrealtime();                                              \
    } while (0)
// entry now and exit when the scope ends (every return path of a merge)
#define XHIP_MERGE_SCOPE(p)                                                                    \
    XHIP_MERGE_STAMP(p, 0);                                                                    \
    struct XhipMergeExit_ {                                                                    \
        const ::xhip::DecodeParams &p_;                                                        \
        __device__ ~XhipMergeExit_() { XHIP_MERGE_STAMP(p_, 1); }                              \
    } xhip_merge_exit_{p}
#else
#define XHIP_TRACING 0
#define XHIP_MERGE_SCOPE(p) do { } while (0)
#define XHIP_WG_STAMP(p, idx) do { } while (0)
#define XHIP_WG_PUT(p, idx, value) do { } while (0)
#define XHIP_WAVE_STAMP(p, wave, idx) do { } while (0)
#define XHIP_WAVE_PUT(p, wave, idx, value) do { } while (0)
#define XHIP_MERGE_STAMP(p, idx) do { } while (0)
#endif
