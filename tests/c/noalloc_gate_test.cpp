// CPU test of the ordering of allocation-free calls (xllms_amd/csrc/noalloc_gate.h)
// with a mock device whose queues and events carry vector clocks.
//
// Each call goes through the gate and "launches" one use of the device's
// scratch on its queue (a stream handle, or (handle, thread) for the
// per-thread handle).  A queue's clock advances with every use; recording
// an event copies the queue's clock into it, and a queue that waits for an
// event takes the larger of the two clocks in every component.  A use
// happens after another exactly when its clock has caught up with that
// use's own component, so the mock fails the test when a use of the scratch
// is not ordered after the last use on every other queue: two calls whose
// kernels could overlap on the device.  Host threads call on a shared
// handle, on their own handles, on the per-thread handle and on the null
// stream at random; some calls are made while "capturing" (they go to a
// graph and are not ordered: the test only checks they neither wait nor
// record).  Built with -DPLANT_NO_WAIT the mock ignores waits, and the test
// must report overlapping uses (the checker sees the race it guards).
//
//   g++ -std=c++17 -O2 -pthread -I xllms_amd/csrc tests/c/noalloc_gate_test.cpp
#include <stdint.h>
#include <stdio.h>

#include <atomic>
#include <map>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

#include "noalloc_gate.h"

namespace {

void *const kPerThread = (void *)2;
constexpr int kQueues = 64;

struct Clock {
    unsigned v[kQueues] = {};
    void join(const Clock &o) {
        for (int i = 0; i < kQueues; i++) v[i] = v[i] > o.v[i] ? v[i] : o.v[i];
    }
};

std::mutex g_mu;
std::map<std::pair<void *, std::thread::id>, int> g_qid;  // queue -> index
Clock g_qclock[kQueues];                                    // clock of each queue's last use
Clock g_last_use[kQueues];                                  // last scratch use per queue
bool g_used[kQueues] = {};
std::atomic<int> g_fail{0}, g_events{0}, g_waits{0}, g_capture_ops{0};
thread_local bool t_capturing = false;

void fail(const char *what) {
    if (g_fail.fetch_add(1) < 10) fprintf(stderr, "FAIL: %s\n", what);
}

int queue_of(void *stream) {  // g_mu held
    const auto key = std::make_pair(stream, stream == kPerThread ? std::this_thread::get_id()
                                                                 : std::thread::id());
    auto it = g_qid.find(key);
    if (it != g_qid.end()) return it->second;
    const int q = (int)g_qid.size();
    if (q >= kQueues) {
        fail("too many queues");
        return 0;
    }
    g_qid[key] = q;
    return q;
}

struct Event {
    Clock clock;
};

struct MockDev {
    static int create_event(void **ev) {
        *ev = new Event();
        g_events++;
        return 0;
    }
    static int record(void *ev, void *stream) {
        if (t_capturing) g_capture_ops++;
        std::lock_guard<std::mutex> g(g_mu);
        ((Event *)ev)->clock = g_qclock[queue_of(stream)];
        return 0;
    }
    static int wait(void *stream, void *ev) {
        if (t_capturing) g_capture_ops++;
        g_waits++;
#ifndef PLANT_NO_WAIT
        std::lock_guard<std::mutex> g(g_mu);
        g_qclock[queue_of(stream)].join(((Event *)ev)->clock);
#else
        (void)stream;
        (void)ev;
#endif
        return 0;
    }
    static bool capturing(void *) { return t_capturing; }
    static bool per_thread(void *stream) { return stream == kPerThread; }
};

using Gate = xhip::NoAllocGate<MockDev, 4>;
Gate g_gate;

// The kernels of one call: a use of device 0's scratch on the stream's queue.
void launch(void *stream) {
    std::lock_guard<std::mutex> g(g_mu);
    const int q = queue_of(stream);
    if (t_capturing) return;  // recorded into a graph, run later
    Clock &c = g_qclock[q];
    c.v[q]++;
    for (int r = 0; r < kQueues; r++) {
        if (r == q || !g_used[r]) continue;
        if (c.v[r] < g_last_use[r].v[r]) fail("a no-alloc call may overlap another queue's");
    }
    g_last_use[q] = c;
    g_used[q] = true;
}

void call(void *stream) {
    Gate::Pass pass;
    if (g_gate.enter(0, stream, &pass) != Gate::kOk) {
        fail("enter");
        return;
    }
    launch(stream);
    std::this_thread::yield();
    if (pass.done() != Gate::kOk) fail("done");
}

}  // namespace

int main() {
    void *const shared = (void *)0x1000;
    std::vector<std::thread> threads;
    for (int t = 0; t < 8; t++) {
        threads.emplace_back([t, shared] {
            std::mt19937 rng(77 + t);
            void *const own = (void *)(uintptr_t)(0x2000 + 16 * t);
            for (int i = 0; i < 20000; i++) {
                switch (rng() % 5) {
                case 0: call(shared); break;
                case 1: call(own); break;
                case 2: call(kPerThread); break;
                case 3: call(nullptr); break;
                default:
                    // a capture: it must neither wait nor record (counted
                    // in g_capture_ops, checked after the threads)
                    t_capturing = true;
                    call(own);
                    t_capturing = false;
                    break;
                }
            }
        });
    }
    for (auto &th : threads) th.join();
    if (g_capture_ops.load() != 0) fail("a capturing call waited or recorded");
    if (!g_gate.captured(0)) fail("the capture was not noted");
    if (g_events.load() != 1) fail("more than one event for the device");
    printf("%s: %d waits, %d failures\n", g_fail ? "FAILED" : "PASSED", g_waits.load(),
           g_fail.load());
    return g_fail ? 1 : 0;
}
