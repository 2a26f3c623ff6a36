// Library-owned device workspaces of the paged-decode entry points (split-K
// partials, cascade plan), one per (device, stream queue, kind).
//
// Threading contract.  Calls are host-synchronous enqueues: a call takes its
// workspace, enqueues every launch that uses it, and gives it back.  The
// entry's lock is held over that whole span (a Lease), so
//   - two host threads on one stream handle enqueue their launches one call
//     after the other, never interleaved: kernels on one queue run in
//     enqueue order, so each call's partition kernel and merge see only its
//     own partials;
//   - growing a workspace (wait for its queue, free, allocate) cannot free a
//     buffer that another thread has taken but not yet enqueued on.
// hipStreamPerThread is one handle for a different queue in every host
// thread: its workspaces are keyed by thread as well, so threads never share
// one across queues.  Every other handle names one queue per device.
// Release (owner-scoped, per stream, or all) waits for the whole device under
// the entry's lock before it frees, so it never frees a buffer that an
// enqueued kernel still uses; a later call on that key allocates again.
//
// Entries are never erased (a few dozen bytes per stream ever used), so a
// Lease or a thread blocked on an entry's lock never sees it disappear.
#pragma once

#include <stddef.h>

#include <memory>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

namespace xhip {

enum WsKind : int { kWsSplitK = 0, kWsCascade = 1 };

// Dev supplies the device calls (HIP in the library, a mock in the CPU unit
// test), each returning 0 on success:
//   static int sync_stream(int device, void *stream);   // all work enqueued on it so far
//   static int sync_device(int device);
//   static int alloc(int device, void **ptr, size_t bytes);
//   static int release(int device, void *ptr);
//   static bool per_thread(void *stream);               // hipStreamPerThread
template <class Dev> class WorkspaceCache {
  public:
    enum Status : int { kOk = 0, kSyncFailed = 1, kNoMemory = 2 };

    struct Entry {
        int device;
        void *stream;
        std::thread::id thread;  // only for per-thread handles
        int kind;
        const void *owner;       // who allocated the current buffer
        std::mutex mu;
        void *ptr = nullptr;
        size_t bytes = 0;
    };

    // A workspace taken for one call: `ptr` of at least the requested bytes,
    // locked until the Lease is destroyed (after the call's launches are
    // enqueued).
    class Lease {
      public:
        Lease() = default;
        Lease(Lease &&) = default;
        Lease &operator=(Lease &&) = default;
        void *ptr() const { return entry_ ? entry_->ptr : nullptr; }
        size_t bytes() const { return entry_ ? entry_->bytes : 0; }

      private:
        friend class WorkspaceCache;
        Entry *entry_ = nullptr;
        std::unique_lock<std::mutex> lock_;
    };

    // Takes (device, stream, kind)'s workspace with at least `bytes`,
    // growing it if needed; `owner` is recorded when a buffer is allocated.
    int acquire(int device, void *stream, int kind, size_t bytes, const void *owner, Lease *out) {
        Entry *e = find_or_add(device, stream, kind);
        std::unique_lock<std::mutex> lk(e->mu);
        if (e->bytes < bytes) {
            if (e->ptr) {
                // every earlier call on this entry enqueued on this queue
                if (Dev::sync_stream(device, stream) != 0) return kSyncFailed;
                (void)Dev::release(device, e->ptr);
                e->ptr = nullptr;
                e->bytes = 0;
            }
            void *p = nullptr;
            if (Dev::alloc(device, &p, bytes) != 0) return kNoMemory;
            e->ptr = p;
            e->bytes = bytes;
            e->owner = owner;
        }
        out->entry_ = e;
        out->lock_ = std::move(lk);
        return kOk;
    }

    // Frees the buffers allocated by `owner` (every buffer when owner is
    // null and `all` is set).  Returns kOk or kSyncFailed.
    int release_owner(const void *owner, bool all = false) {
        return release_if([&](const Entry &e) { return all || e.owner == owner; });
    }

    // Frees every workspace of one stream handle on one device (all kinds,
    // all threads): for a caller about to destroy that stream.
    int release_stream(int device, void *stream) {
        return release_if([&](const Entry &e) { return e.device == device && e.stream == stream; });
    }

    // Number of entries (tests).
    size_t entries() {
        std::lock_guard<std::mutex> g(mu_);
        return list_.size();
    }

  private:
    Entry *find_or_add(int device, void *stream, int kind) {
        const std::thread::id tid =
            Dev::per_thread(stream) ? std::this_thread::get_id() : std::thread::id();
        std::lock_guard<std::mutex> g(mu_);
        for (auto &p : list_)
            if (p->device == device && p->stream == stream && p->kind == kind && p->thread == tid)
                return p.get();
        list_.emplace_back(new Entry());
        Entry *e = list_.back().get();
        e->device = device;
        e->stream = stream;
        e->thread = tid;
        e->kind = kind;
        e->owner = nullptr;
        return e;
    }

    template <class Pred> int release_if(Pred &&pred) {
        std::vector<Entry *> snap;
        {
            std::lock_guard<std::mutex> g(mu_);
            for (auto &p : list_) snap.push_back(p.get());
        }
        int rc = kOk;
        for (Entry *e : snap) {
            std::lock_guard<std::mutex> lk(e->mu);
            if (!e->ptr || !pred(*e)) continue;
            // the device, not the stream: the handle may already be destroyed
            if (Dev::sync_device(e->device) != 0) {
                rc = kSyncFailed;
                continue;
            }
            (void)Dev::release(e->device, e->ptr);
            e->ptr = nullptr;
            e->bytes = 0;
            e->owner = nullptr;
        }
        return rc;
    }

    std::mutex mu_;
    std::vector<std::unique_ptr<Entry>> list_;
};

}  // namespace xhip
