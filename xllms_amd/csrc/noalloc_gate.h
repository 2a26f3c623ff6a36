// Ordering of the allocation-free entry point's calls on one device
// (nxt_paged_attention_noalloc).  Every such call on a device uses the same
// fixed scratch array, so two calls whose kernels overlap on the GPU would
// corrupt each other's split-K partials.  The gate makes the device run them
// one after another, without blocking the host:
//   - a call holds the device's gate lock while it enqueues its launches, so
//     host threads enqueue whole calls one after the other;
//   - it first makes its stream wait for the device's last no-alloc call
//     (an event recorded after that call's launches) unless that call went
//     to the same queue (same handle, and for hipStreamPerThread the same
//     thread): stream order already covers it;
//   - after its launches it records that event on its own stream.
// The event is created by the first eager call on a device (set-up, like
// the scratch address lookup); later calls allocate nothing.
//
// A call on a stream that is being captured goes into the caller's graph,
// where an ordering against eager calls or other graphs cannot be
// expressed: it neither waits nor records, and marks the device as having
// captured no-alloc work.  Replays of graphs holding no-alloc calls must be
// ordered by the caller (replayed on one stream, or waited for) against one
// another and against eager no-alloc calls on that device.
#pragma once

#include <mutex>
#include <thread>

namespace xhip {

// Dev supplies, each returning 0 on success:
//   static int create_event(void **ev);
//   static int record(void *ev, void *stream);
//   static int wait(void *stream, void *ev);        // the stream waits for ev
//   static bool capturing(void *stream);
//   static bool per_thread(void *stream);
template <class Dev, int kMaxDevices = 64> class NoAllocGate {
  public:
    enum Status : int { kOk = 0, kBadDevice = 1, kEventFailed = 2 };

    struct DeviceState {
        std::mutex mu;
        void *event = nullptr;      // recorded after the last eager call
        void *last_stream = nullptr;
        std::thread::id last_thread;
        bool used = false;          // an eager call has recorded the event
        bool captured = false;      // some capture holds no-alloc work
    };

    // Holds a device's gate while one call enqueues its launches.
    class Pass {
      public:
        Pass() = default;
        Pass(Pass &&) = default;
        Pass &operator=(Pass &&) = default;
        // Call after the launches are enqueued (whatever their status).
        int done() {
            if (!d_) return kOk;
            int rc = kOk;
            if (!capturing_) {
                if (Dev::record(d_->event, stream_) != 0) rc = kEventFailed;
                else {
                    d_->used = true;
                    d_->last_stream = stream_;
                    d_->last_thread = std::this_thread::get_id();
                }
            }
            lock_.unlock();
            d_ = nullptr;
            return rc;
        }
        ~Pass() {
            if (d_) (void)done();
        }

      private:
        friend class NoAllocGate;
        DeviceState *d_ = nullptr;
        void *stream_ = nullptr;
        bool capturing_ = false;
        std::unique_lock<std::mutex> lock_;
    };

    // Orders a call on (device, stream) after the device's previous one.
    int enter(int device, void *stream, Pass *pass) {
        if (device < 0 || device >= kMaxDevices) return kBadDevice;
        DeviceState &d = dev_[device];
        std::unique_lock<std::mutex> lk(d.mu);
        const bool cap = Dev::capturing(stream);
        if (cap) {
            d.captured = true;
        } else {
            if (!d.event && Dev::create_event(&d.event) != 0) {
                d.event = nullptr;
                return kEventFailed;
            }
            const bool same_queue =
                d.last_stream == stream &&
                (!Dev::per_thread(stream) || d.last_thread == std::this_thread::get_id());
            if (d.used && !same_queue && Dev::wait(stream, d.event) != 0) return kEventFailed;
        }
        pass->d_ = &d;
        pass->stream_ = stream;
        pass->capturing_ = cap;
        pass->lock_ = std::move(lk);
        return kOk;
    }

    // Whether a capture on `device` has taken no-alloc work (tests, docs).
    bool captured(int device) {
        if (device < 0 || device >= kMaxDevices) return false;
        std::lock_guard<std::mutex> g(dev_[device].mu);
        return dev_[device].captured;
    }

  private:
    DeviceState dev_[kMaxDevices];
};

}  // namespace xhip
