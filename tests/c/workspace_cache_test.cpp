// CPU stress test of the workspace cache (xllms_amd/csrc/workspace_cache.h)
// with a mock device that models queues of in-flight work.
//
// Each call takes a lease, "enqueues" a use of its buffer on its queue (the
// queue is the stream handle, or (handle, thread) for the per-thread handle)
// and gives the lease back; the use stays pending on the queue until that
// queue or the whole device is synchronised.  The mock fails the test when
//   - a buffer is freed while a use of it is still pending (a device
//     use-after-free),
//   - a buffer gets a use on one queue while a use on another queue is
//     pending (two queues racing on one workspace),
//   - two host threads hold one buffer at the same time (interleaved
//     enqueues on one queue),
//   - a lease is smaller than requested, or its buffer is not live.
// Threads share a stream handle, use the per-thread handle, grow their
// workspaces with random sizes, and release by owner and by stream
// concurrently with the calls.  Then, single-threaded:
//   - graph capture: a capturing call that would need to grow is refused; a
//     capturing call pins its buffer, which then survives growth, the
//     owner- and stream-scoped releases and eviction, until release_all;
//   - calls on 200 streams leave at most kMaxEntries entries (the least
//     recently used are evicted, never while their buffer has pending work);
//   - the per-thread handle's entries are gone once their threads exited.
//
//   g++ -std=c++17 -O2 -pthread -I xllms_amd/csrc tests/c/workspace_cache_test.cpp
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <map>
#include <mutex>
#include <random>
#include <set>
#include <thread>
#include <vector>

#include "workspace_cache.h"

namespace {

void *const kPerThread = (void *)2;

struct Buffer {
    size_t bytes;
    bool live;
    std::atomic<int> holder{-1};  // host thread holding a lease on it
};

std::mutex g_mu;
std::set<Buffer *> g_all;
// queue -> pending uses (buffers) in enqueue order
thread_local bool t_capturing = false;
// A queue: the handle, and for the per-thread handle the thread.
using Queue = std::pair<void *, std::thread::id>;

Queue queue_of(void *stream) {
    return {stream, stream == kPerThread ? std::this_thread::get_id() : std::thread::id()};
}

// queue -> pending uses (buffers) in enqueue order
std::map<Queue, std::vector<Buffer *>> g_queues;
std::atomic<int> g_fail{0};
thread_local int t_index = -1;

void fail(const char *what) {
    if (g_fail.fetch_add(1) < 10) fprintf(stderr, "FAIL: %s\n", what);
}

struct MockDev {
    static int sync_stream(int, void *stream) {
        std::lock_guard<std::mutex> g(g_mu);
        g_queues[queue_of(stream)].clear();
        return 0;
    }
    static int sync_device(int) {
        std::lock_guard<std::mutex> g(g_mu);
        for (auto &q : g_queues) q.second.clear();
        return 0;
    }
    static int alloc(int, void **ptr, size_t bytes) {
        Buffer *b = new Buffer();
        b->bytes = bytes;
        b->live = true;
        std::lock_guard<std::mutex> g(g_mu);
        g_all.insert(b);
        *ptr = b;
        return 0;
    }
    static int release(int, void *ptr) {
        Buffer *b = (Buffer *)ptr;
        std::lock_guard<std::mutex> g(g_mu);
        if (!b->live) fail("double free");
        for (auto &q : g_queues)
            for (Buffer *u : q.second)
                if (u == b) fail("buffer freed while a use of it is pending on a queue");
        b->live = false;  // kept allocated so later misuse is still detected
        return 0;
    }
    static bool per_thread(void *stream) { return stream == kPerThread; }
    static bool capturing(void *) { return t_capturing; }
};

using Cache = xhip::WorkspaceCache<MockDev>;
Cache g_cache;

// One operator call: take the workspace, check it, enqueue a use, let go.
void call(void *stream, int kind, size_t bytes, const void *owner) {
    Cache::Lease lease;
    if (g_cache.acquire(0, stream, kind, bytes, owner, &lease) != Cache::kOk) {
        fail("acquire failed");
        return;
    }
    Buffer *b = (Buffer *)lease.ptr();
    if (!b || lease.bytes() < bytes) {
        fail("lease smaller than requested");
        return;
    }
    int expect = -1;
    if (!b->holder.compare_exchange_strong(expect, t_index))
        fail("two host threads hold one workspace at once");
    {
        std::lock_guard<std::mutex> g(g_mu);
        if (!b->live) fail("lease on a freed buffer");
        const auto mine = queue_of(stream);
        for (auto &q : g_queues) {
            if (q.first == mine) continue;
            for (Buffer *u : q.second)
                if (u == b) fail("workspace in flight on another queue");
        }
        auto &q = g_queues[mine];
        q.push_back(b);
        if (q.size() > 64) q.erase(q.begin());  // the oldest work completes
    }
    std::this_thread::yield();
    b->holder.store(-1);
}

}  // namespace

int main() {
    void *const shared = (void *)0x1000;
    std::vector<std::thread> threads;
    const int kCalls = 20000;
    int owners[2];
    for (int t = 0; t < 8; t++) {
        threads.emplace_back([&, t] {
            t_index = t;
            std::mt19937 rng(1234 + t);
            for (int i = 0; i < kCalls; i++) {
                const size_t bytes = 256 + (rng() % 64) * 4096;  // growth at random
                if (t < 3) {
                    call(shared, xhip::kWsSplitK, bytes, nullptr);
                } else if (t < 6) {
                    call(kPerThread, xhip::kWsSplitK, bytes, nullptr);
                } else {
                    // a "plugin": its calls carry an owner tag; the cascade
                    // holds its own workspace across two split-K calls
                    const void *owner = &owners[t - 6];
                    if (rng() % 4 == 0) {
                        Cache::Lease outer;
                        if (g_cache.acquire(0, shared, xhip::kWsCascade, bytes, owner, &outer) !=
                            Cache::kOk)
                            fail("cascade acquire");
                        call(shared, xhip::kWsSplitK, bytes, owner);
                        call(shared, xhip::kWsSplitK, bytes / 2, owner);
                    } else {
                        call(shared, xhip::kWsSplitK, bytes, owner);
                    }
                    if (i % 500 == 499) {
                        if (g_cache.release_owner(owner) != Cache::kOk) fail("release_owner");
                    }
                    if (t == 7 && i % 1500 == 1499) g_cache.release_stream(0, kPerThread);
                }
            }
        });
    }
    for (auto &th : threads) th.join();
    // the per-thread handle's entries went with their threads; the shared
    // handle keeps a split-K and a cascade entry
    if (g_cache.entries() != 2) {
        fprintf(stderr, "entries %zu, expected 2\n", g_cache.entries());
        fail("entry count after the threads exited");
    }

    // graph capture
    void *const cs = (void *)0x2000;
    {
        t_capturing = true;
        Cache::Lease l0;
        if (g_cache.acquire(0, cs, xhip::kWsSplitK, 4096, nullptr, &l0) != Cache::kCaptureGrow)
            fail("a capturing call that needs a new workspace was not refused");
        t_capturing = false;
    }
    Buffer *b1 = nullptr, *b2 = nullptr;
    call(cs, xhip::kWsSplitK, 8192, nullptr);  // the warm-up call creates it
    {
        t_capturing = true;
        Cache::Lease l1;
        if (g_cache.acquire(0, cs, xhip::kWsSplitK, 4096, nullptr, &l1) != Cache::kOk)
            fail("capturing call refused");
        b1 = (Buffer *)l1.ptr();
        t_capturing = false;
    }
    call(cs, xhip::kWsSplitK, 1 << 20, nullptr);  // grows: the graph's buffer stays
    {
        Cache::Lease l2;
        (void)g_cache.acquire(0, cs, xhip::kWsSplitK, 16, nullptr, &l2);
        b2 = (Buffer *)l2.ptr();
    }
    if (!b1 || !b2 || b1 == b2) fail("growth of a pinned workspace did not allocate a new buffer");
    if (g_cache.release_owner(nullptr) != Cache::kOk) fail("release_owner");
    g_cache.release_stream(0, cs);
    {
        std::lock_guard<std::mutex> g(g_mu);
        if (!b1->live || !b2->live) fail("a buffer a captured graph holds was freed");
    }
    if (g_cache.kept_for_graphs() != 2) fail("pinned buffers not kept for the graphs");

    // bound on the entries
    for (int i = 0; i < 200; i++) call((void *)(uintptr_t)(0x10000 + 16 * i), xhip::kWsSplitK, 512, nullptr);
    if (g_cache.entries() > Cache::kMaxEntries) {
        fprintf(stderr, "entries %zu > %zu\n", g_cache.entries(), Cache::kMaxEntries);
        fail("entry list unbounded");
    }

    if (g_cache.release_all() != Cache::kOk) fail("release all");
    for (Buffer *b : g_all)
        if (b->live) fail("a buffer is still live after releasing everything");
    if (g_cache.entries() != 0 || g_cache.kept_for_graphs() != 0)
        fail("entries or kept buffers left after release_all");
    printf("%s: %zu buffers allocated, %d failures\n", g_fail ? "FAILED" : "PASSED",
           g_all.size(), g_fail.load());
    return g_fail ? 1 : 0;
}
