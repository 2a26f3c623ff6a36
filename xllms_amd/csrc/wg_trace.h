// Per-workgroup timeline of the decode kernels, for the instrumented
// measurement build only (compiled with XHIP_WG_TRACE=1 into
// libxllm_hip_backend_trace.so; the product library compiles every stamp
// below to nothing).  Timestamps are s_memrealtime, the device's constant
// 100 MHz clock, comparable across CUs and XCDs.  A stamp goes to LDS (a
// global store before a workgroup barrier would make the barrier wait for
// the store to reach memory, ~1-2 us, and distort the timeline); the
// workgroup's record is copied to DecodeParams::wg_trace when it exits.
//
// Layout of the buffer DecodeParams::wg_trace points at (unsigned 64-bit
// words), filled by one traced call:
//   partition launch, record b (physical workgroup b), 24 words at 24 * b:
//     [0] entry  [1] prologue done (split-unit scan / plan)  [2] exit
//     [3] logical workgroup | role << 32 (cascade: 1 prefix body, 2 suffix)
//     MFMA kernels, wavefront w: [4 + 3w] first tile issued  [5 + 3w] last
//     tile done  [6 + 3w] tiles | pieces << 32
//     segment kernel: [7] first tile issued [8] last tile done (wavefront 0)
//     [16..23] kernel-specific phase stamps (cascade plan: [16] caller arrays
//     loaded, [17] members and suffix units, [18] groups laid out)
//   merge launch, record b at kWgTraceMergeBase + 2 * b:
//     [0] entry  [1] exit
#pragma once

namespace xhip {

constexpr int kWgTraceWords = 24;
constexpr unsigned long long kWgTraceMaxGroups = 4096;
constexpr unsigned long long kWgTraceMergeBase = kWgTraceMaxGroups * kWgTraceWords;
constexpr unsigned long long kWgTraceMergeMax = 65536;
constexpr unsigned long long kWgTraceBufferWords = kWgTraceMergeBase + 2 * kWgTraceMergeMax;

}  // namespace xhip

#if defined(XHIP_WG_TRACE) && XHIP_WG_TRACE
#define XHIP_TRACING 1
#ifdef __HIPCC__
namespace xhip {
// The workgroup's record, in LDS until it exits.
__device__ __forceinline__ unsigned long long *wg_trace_lds() {
    __shared__ unsigned long long rec[kWgTraceWords];
    return rec;
}
}  // namespace xhip
#endif
// at kernel entry: the record cleared, the entry stamped
#define XHIP_WG_BEGIN(p)                                                                       \
    do {                                                                                       \
        if ((p).wg_trace && threadIdx.x == 0) {                                                \
            unsigned long long *r_ = ::xhip::wg_trace_lds();                                   \
            for (int i_ = 1; i_ < ::xhip::kWgTraceWords; i_++) r_[i_] = 0;                     \
            r_[0] = __builtin_amdgcn_s_memrealtime();                                          \
        }                                                                                      \
    } while (0)
// word `idx` of this workgroup's record (one lane writes)
#define XHIP_WG_STAMP(p, idx)                                                                  \
    do {                                                                                       \
        if ((p).wg_trace && threadIdx.x == 0)                                                  \
            ::xhip::wg_trace_lds()[(idx)] = __builtin_amdgcn_s_memrealtime();                  \
    } while (0)
#define XHIP_WG_PUT(p, idx, value)                                                             \
    do {                                                                                       \
        if ((p).wg_trace && threadIdx.x == 0)                                                  \
            ::xhip::wg_trace_lds()[(idx)] = (unsigned long long)(value);                       \
    } while (0)
// word `idx` of wavefront `wave`'s part of the record (lane 0 of the wavefront)
#define XHIP_WAVE_STAMP(p, wave, idx)                                                          \
    do {                                                                                       \
        if ((p).wg_trace && (threadIdx.x & 63) == 0)                                           \
            ::xhip::wg_trace_lds()[4 + 3 * (wave) + (idx)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define XHIP_WAVE_PUT(p, wave, idx, value)                                                     \
    do {                                                                                       \
        if ((p).wg_trace && (threadIdx.x & 63) == 0)                                           \
            ::xhip::wg_trace_lds()[4 + 3 * (wave) + (idx)] = (unsigned long long)(value);      \
    } while (0)
// the exit stamp, after every wavefront is done, and the record to memory
#define XHIP_WG_FLUSH(p)                                                                       \
    do {                                                                                       \
        __syncthreads();                                                                       \
        if ((p).wg_trace && threadIdx.x == 0 && blockIdx.x < ::xhip::kWgTraceMaxGroups) {      \
            unsigned long long *r_ = ::xhip::wg_trace_lds();                                   \
            r_[2] = __builtin_amdgcn_s_memrealtime();                                          \
            for (int i_ = 0; i_ < ::xhip::kWgTraceWords; i_++)                                 \
                (p).wg_trace[blockIdx.x * ::xhip::kWgTraceWords + i_] = r_[i_];                \
        }                                                                                      \
    } while (0)
// merge workgroups: entry now, exit (and the record) when the scope ends,
// on every return path
#define XHIP_MERGE_SCOPE(p)                                                                    \
    const unsigned long long xhip_merge_t0_ = __builtin_amdgcn_s_memrealtime();                \
    struct XhipMergeExit_ {                                                                    \
        const ::xhip::DecodeParams &p_;                                                        \
        unsigned long long t0_;                                                                \
        __device__ ~XhipMergeExit_() {                                                         \
            const unsigned long long b_ = (unsigned long long)blockIdx.x +                     \
                                          (unsigned long long)blockIdx.y * gridDim.x;          \
            if (p_.wg_trace && threadIdx.x == 0 && b_ < ::xhip::kWgTraceMergeMax) {            \
                p_.wg_trace[::xhip::kWgTraceMergeBase + 2 * b_] = t0_;                         \
                p_.wg_trace[::xhip::kWgTraceMergeBase + 2 * b_ + 1] =                          \
                    __builtin_amdgcn_s_memrealtime();                                          \
            }                                                                                  \
        }                                                                                      \
    } xhip_merge_exit_{p, xhip_merge_t0_}
#else
#define XHIP_TRACING 0
#define XHIP_WG_BEGIN(p) do { } while (0)
#define XHIP_WG_STAMP(p, idx) do { } while (0)
#define XHIP_WG_PUT(p, idx, value) do { } while (0)
#define XHIP_WAVE_STAMP(p, wave, idx) do { } while (0)
#define XHIP_WAVE_PUT(p, wave, idx, value) do { } while (0)
#define XHIP_WG_FLUSH(p) do { } while (0)
#define XHIP_MERGE_SCOPE(p) do { } while (0)
#endif
