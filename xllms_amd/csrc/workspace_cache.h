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
// one across queues, and they are freed when that thread exits.  Every other
// handle names one queue per device.  (Not covered: a stream destroyed with
// calls still pending whose handle a new stream takes at once; the new
// stream's first call does not wait for the old queue.  The HIP runtime
// torch loads has no stream identity to key on.  The model instance
// releases its stream's entries before destroying it.)
//
// Graph capture.  A call made while its stream is capturing puts the
// workspace's address into the captured kernels.  Such an entry is pinned:
// its buffers are never freed by growth, by the owner- or stream-scoped
// releases or by eviction, only by release_all (the caller's statement that
// no graph that used them will be replayed again).  A pinned entry grows by
// allocating a new buffer and keeping the old one.  A capturing call that
// would need a larger workspace is refused (kCaptureGrow): growing needs a
// queue wait and an allocation, neither of which belongs in a capture; one
// call of the shape before the capture creates the workspace.
//
// Bound.  At most kMaxEntries entries are kept: beyond that the least
// recently used entry that no thread holds is released (after waiting for
// the device) and erased, so a process that creates and destroys streams
// keeps a bounded list.  Releases by stream and thread erase their entries;
// releases by owner free buffers and keep the entries.
// Release waits for the whole device under the entry's lock before it
// frees, so it never frees a buffer that an enqueued kernel still uses.
#pragma once

#include <stddef.h>
#include <stdint.h>

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
//   static bool capturing(void *stream);                // in a graph capture
template <class Dev> class WorkspaceCache {
  public:
    enum Status : int { kOk = 0, kSyncFailed = 1, kNoMemory = 2, kCaptureGrow = 3 };
    static constexpr size_t kMaxEntries = 64;

    struct Entry {
        int device;
        void *stream;
        std::thread::id thread;  // only for per-thread handles
        int kind;
        const void *owner;       // who allocated the current buffer
        std::mutex mu;
        void *ptr = nullptr;
        size_t bytes = 0;
        bool pinned = false;          // a captured graph holds its address
        bool dead = false;            // erased from the list: look the key up again
        std::vector<void *> retired;  // pinned buffers outgrown (kept for the graphs)
        uint64_t last_use = 0;        // LRU tick (under the cache's list lock)
    };

    // A workspace taken for one call: `ptr` of at least the requested bytes,
    // locked until the Lease is destroyed (after the call's launches are
    // enqueued).  The Lease keeps its entry alive even if it is erased.
    class Lease {
      public:
        Lease() = default;
        Lease(Lease &&) = default;
        Lease &operator=(Lease &&) = default;
        ~Lease() {
            if (lock_.owns_lock()) lock_.unlock();
        }
        void *ptr() const { return entry_ ? entry_->ptr : nullptr; }
        size_t bytes() const { return entry_ ? entry_->bytes : 0; }

      private:
        friend class WorkspaceCache;
        std::shared_ptr<Entry> entry_;
        std::unique_lock<std::mutex> lock_;
    };

    ~WorkspaceCache() = default;

    // Takes (device, stream, kind)'s workspace with at least `bytes`,
    // growing it if needed; `owner` is recorded when a buffer is allocated.
    int acquire(int device, void *stream, int kind, size_t bytes, const void *owner, Lease *out) {
        const bool cap = Dev::capturing(stream);
        std::shared_ptr<Entry> e;
        std::unique_lock<std::mutex> lk;
        for (;;) {
            // (an entry erased between the lookup and the lock is dead: a
            // buffer allocated into it would be freed by nobody)
            e = find_or_add(device, stream, kind);
            lk = std::unique_lock<std::mutex>(e->mu);
            if (!e->dead) break;
            lk.unlock();
        }
        if (e->bytes < bytes) {
            if (cap) return kCaptureGrow;
            if (e->ptr) {
                if (e->pinned) {
                    // a graph still holds the old address: keep it
                    e->retired.push_back(e->ptr);
                } else {
                    // every earlier call on this entry enqueued on this queue
                    if (Dev::sync_stream(device, stream) != 0) return kSyncFailed;
                    (void)Dev::release(device, e->ptr);
                }
                e->ptr = nullptr;
                e->bytes = 0;
            }
            void *p = nullptr;
            if (Dev::alloc(device, &p, bytes) != 0) return kNoMemory;
            e->ptr = p;
            e->bytes = bytes;
            e->owner = owner;
        }
        if (cap) e->pinned = true;
        out->entry_ = std::move(e);
        out->lock_ = std::move(lk);
        return kOk;
    }

    // Frees the buffers allocated by `owner`, keeping the entries (pinned
    // buffers are kept for their graphs).  Returns kOk or kSyncFailed.
    int release_owner(const void *owner) {
        return release_if([&](const Entry &e) { return e.owner == owner; }, false, false);
    }

    // Frees every buffer, pinned and retired ones included, and erases every
    // entry: the caller states that no graph that used them runs again.
    int release_all() {
        int rc = release_if([](const Entry &) { return true; }, true, true);
        std::vector<std::pair<int, void *>> kept;
        {
            std::lock_guard<std::mutex> g(mu_);
            kept.swap(kept_);
        }
        for (auto &k : kept) {
            if (Dev::sync_device(k.first) != 0) {
                rc = kSyncFailed;
                std::lock_guard<std::mutex> g(mu_);
                kept_.push_back(k);
                continue;
            }
            (void)Dev::release(k.first, k.second);
        }
        return rc;
    }

    // Frees and erases every workspace of one stream handle on one device
    // (all kinds, all threads): for a caller about to destroy that stream.
    int release_stream(int device, void *stream) {
        return release_if([&](const Entry &e) { return e.device == device && e.stream == stream; },
                          true, false);
    }

    // Frees and erases the per-thread-handle workspaces of host thread `tid`
    // (called when that thread exits).
    int release_thread(std::thread::id tid) {
        return release_if(
            [&](const Entry &e) { return Dev::per_thread(e.stream) && e.thread == tid; }, true,
            false);
    }

    // Number of entries, and of buffers held only for captured graphs (tests).
    size_t entries() {
        std::lock_guard<std::mutex> g(mu_);
        return list_.size();
    }
    size_t kept_for_graphs() {
        std::lock_guard<std::mutex> g(mu_);
        size_t n = kept_.size();
        for (auto &p : list_) n += p->retired.size();
        return n;
    }

  private:
    std::shared_ptr<Entry> find_or_add(int device, void *stream, int kind) {
        const bool pt = Dev::per_thread(stream);
        const std::thread::id tid = pt ? std::this_thread::get_id() : std::thread::id();
        std::shared_ptr<Entry> victim;
        std::shared_ptr<Entry> found;
        {
            std::lock_guard<std::mutex> g(mu_);
            ++tick_;
            for (auto &p : list_)
                if (p->device == device && p->stream == stream && p->kind == kind &&
                    p->thread == tid) {
                    p->last_use = tick_;
                    found = p;
                    break;
                }
            if (!found) {
                found = std::make_shared<Entry>();
                found->device = device;
                found->stream = stream;
                found->thread = tid;
                found->kind = kind;
                found->owner = nullptr;
                found->last_use = tick_;
                list_.push_back(found);
                if (list_.size() > kMaxEntries) victim = take_lru_locked(found.get());
            }
        }
        if (pt) register_thread_exit();
        if (victim) evict(victim);
        return found;
    }

    // Removes the least recently used entry that no thread holds (other than
    // `keep`) from the list; the caller frees it.  List lock held.
    std::shared_ptr<Entry> take_lru_locked(const Entry *keep) {
        size_t best = list_.size();
        for (size_t i = 0; i < list_.size(); i++) {
            Entry *p = list_[i].get();
            if (p == keep || list_[i].use_count() > 1) continue;  // held by a Lease
            if (best == list_.size() || p->last_use < list_[best]->last_use) best = i;
        }
        if (best == list_.size()) return nullptr;
        std::shared_ptr<Entry> v = list_[best];
        list_.erase(list_.begin() + (long)best);
        return v;
    }

    // Frees an entry taken off the list (pinned buffers are kept).
    void evict(const std::shared_ptr<Entry> &e) {
        std::lock_guard<std::mutex> lk(e->mu);
        e->dead = true;
        free_entry(*e, false);
    }

    // Frees e's buffers after waiting for its device; pinned ones (and the
    // retired ones) go to kept_ unless `all`.  Entry lock held.
    int free_entry(Entry &e, bool all) {
        if (!e.ptr && e.retired.empty()) return kOk;
        if (e.pinned && !all) {
            std::lock_guard<std::mutex> g(mu_);
            if (e.ptr) kept_.push_back({e.device, e.ptr});
            for (void *r : e.retired) kept_.push_back({e.device, r});
        } else {
            // the device, not the stream: the handle may already be destroyed
            if (Dev::sync_device(e.device) != 0) return kSyncFailed;
            if (e.ptr) (void)Dev::release(e.device, e.ptr);
            for (void *r : e.retired) (void)Dev::release(e.device, r);
        }
        e.retired.clear();
        e.ptr = nullptr;
        e.bytes = 0;
        e.owner = nullptr;
        e.pinned = false;
        return kOk;
    }

    template <class Pred> int release_if(Pred &&pred, bool erase, bool all) {
        std::vector<std::shared_ptr<Entry>> snap;
        {
            std::lock_guard<std::mutex> g(mu_);
            snap = list_;
        }
        int rc = kOk;
        for (auto &sp : snap) {
            Entry *e = sp.get();
            bool match;
            {
                std::lock_guard<std::mutex> lk(e->mu);
                match = pred(*e);
                if (match && free_entry(*e, all) != kOk) {
                    rc = kSyncFailed;
                    continue;
                }
                if (match && erase) e->dead = true;
            }
            if (match && erase) {
                std::lock_guard<std::mutex> g(mu_);
                for (size_t i = 0; i < list_.size(); i++)
                    if (list_[i].get() == e) {
                        list_.erase(list_.begin() + (long)i);
                        break;
                    }
            }
        }
        return rc;
    }

    // The per-thread handle's workspaces of this thread are freed when the
    // thread exits.
    void register_thread_exit() {
        struct Guard {
            WorkspaceCache *cache = nullptr;
            ~Guard() {
                if (cache) (void)cache->release_thread(std::this_thread::get_id());
            }
        };
        thread_local Guard guard;
        guard.cache = this;
    }

    std::mutex mu_;
    std::vector<std::shared_ptr<Entry>> list_;
    std::vector<std::pair<int, void *>> kept_;  // (device, buffer) held for captured graphs
    uint64_t tick_ = 0;
};

}  // namespace xhip
