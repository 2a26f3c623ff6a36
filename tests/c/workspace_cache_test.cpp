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
// concurrently with the calls.
//
//   g++ -std=c++17 -O2 -pthread -I xllms_amd/csrc tests/c/workspace_cache_test.cpp
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
std::map<std::pair<void *, std::thread::id>, std::vector<Buffer *>> g_queues;
std::atomic<int> g_fail{0};
thread_local int t_index = -1;

void fail(const char *what) {
    if (g_fail.fetch_add(1) < 10) fprintf(stderr, "FAIL: %s\n", what);
}

std::pair<void *, std::thread::id> queue_of(void *stream) {
    return {stream, stream == kPerThread ? std::this_thread::get_id() : std::thread::id()};
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
    // per-thread handle: one entry per thread that used it, per kind
    if (g_cache.release_owner(nullptr, true) != Cache::kOk) fail("release all");
    for (Buffer *b : g_all)
        if (b->live) fail("a buffer is still live after releasing everything");
    const size_t entries = g_cache.entries();
    // shared handle: split-K + cascade; per-thread handle: one split-K per thread 3-5
    if (entries != 5) {
        fprintf(stderr, "entries %zu, expected 5\n", entries);
        fail("entry count");
    }
    printf("%s: %zu buffers allocated, %d failures\n", g_fail ? "FAILED" : "PASSED",
           g_all.size(), g_fail.load());
    return g_fail ? 1 : 0;
}
