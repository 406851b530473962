// The host flavour's device: host threads imitating HIP streams and events, so the engine and
// everything above it can be tested without a GPU, with controls that expose ordering bugs as
// corrupted data (reference native/host_device.h:1-269 has the same role).
//
// Semantics the engine relies on, kept exactly:
//   - a stream is a FIFO of commands run in order by one worker thread;
//   - recording an event replaces its pending record: record() bumps a generation counter at
//     enqueue time and the command, when it runs, marks that generation complete;
//   - a wait or query captures the generation current when it is issued, so it ignores
//     records enqueued later.
// Controls: set_paused holds every stream still, set_copy_delay_us slows each copy,
// set_pin_limit makes pinned allocations fail past a byte total, and call() runs a caller
// "kernel" whose nonzero return is a device failure from then on.
#ifndef LAYOVER_AMD_HOST_DEVICE_H
#define LAYOVER_AMD_HOST_DEVICE_H

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <condition_variable>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>

#include "layover_transfer.h"

namespace lt {

class HostDevice {
   public:
    struct StreamState {
        std::deque<std::function<void()>> pending;
        std::thread worker;
        bool running = false;
        bool closing = false;
    };
    struct EventState {
        uint64_t issued = 0;
        uint64_t reached = 0;
    };
    using Stream = StreamState*;
    using Event = EventState*;

    static const char* flavor() { return "host"; }
    static Stream stream_from_handle(void* handle) { return static_cast<Stream>(handle); }

    explicit HostDevice(int) {}
    ~HostDevice() { caller_stream_.reset(); }

    void activate() {
        std::lock_guard<std::mutex> hold(lock_);
        if (!failure_.empty()) throw std::runtime_error(failure_);
    }

    void check_pool(const void*) {}
    void prepare_teardown() { set_paused(false); }

    void* device_alloc(uint64_t bytes) {
        void* pointer = nullptr;
        if (posix_memalign(&pointer, 4096, bytes ? bytes : 1) != 0) throw std::runtime_error("posix_memalign failed");
        return pointer;
    }
    void device_free(void* pointer) { free(pointer); }

    // Null when out of memory (or past the test limit); the engine survives that.
    void* host_alloc(uint64_t bytes) {
        if (bytes > pin_limit_ || pinned_total_ > pin_limit_ - bytes) return nullptr;
        void* pointer = nullptr;
        if (posix_memalign(&pointer, 4096, bytes) != 0) return nullptr;
        pinned_[pointer] = bytes;
        pinned_total_ += bytes;
        return pointer;
    }

    void host_free(void* pointer) {
        auto entry = pinned_.find(pointer);
        if (entry != pinned_.end()) {
            pinned_total_ -= entry->second;
            pinned_.erase(entry);
        }
        free(pointer);
    }

    void set_pin_limit(uint64_t bytes) { pin_limit_ = bytes; }

    Stream stream_create() {
        Stream stream = new StreamState();
        stream->worker = std::thread([this, stream] { serve(stream); });
        return stream;
    }

    void stream_sync(Stream stream) {
        std::unique_lock<std::mutex> hold(lock_);
        changed_.wait(hold, [&] { return stream->pending.empty() && !stream->running; });
    }

    void stream_destroy(Stream stream) {
        {
            std::lock_guard<std::mutex> hold(lock_);
            stream->closing = true;
            changed_.notify_all();
        }
        stream->worker.join();
        delete stream;
    }

    Event event_create() { return new EventState(); }
    void event_destroy(Event event) { delete event; }

    void event_record(Event event, Stream stream) {
        uint64_t generation;
        {
            std::lock_guard<std::mutex> hold(lock_);
            generation = ++event->issued;
        }
        enqueue(stream, [this, event, generation] {
            std::lock_guard<std::mutex> hold(lock_);
            event->reached = std::max(event->reached, generation);
            changed_.notify_all();
        });
    }

    void stream_wait(Stream stream, Event event) {
        uint64_t target;
        {
            std::lock_guard<std::mutex> hold(lock_);
            target = event->issued;
        }
        enqueue(stream, [this, event, target] {
            std::unique_lock<std::mutex> hold(lock_);
            changed_.wait(hold, [&] { return event->reached >= target; });
        });
    }

    bool event_query(Event event) {
        std::lock_guard<std::mutex> hold(lock_);
        if (!failure_.empty()) throw std::runtime_error(failure_);
        return event->reached >= event->issued;
    }

    void event_sync(Event event) {
        std::unique_lock<std::mutex> hold(lock_);
        const uint64_t target = event->issued;
        changed_.wait(hold, [&] { return event->reached >= target || !failure_.empty(); });
        if (!failure_.empty()) throw std::runtime_error(failure_);
    }

    void memcpy_to_host(Stream stream, void* dst, const void* src, uint64_t bytes) { copy(stream, dst, src, bytes); }
    void memcpy_to_device(Stream stream, void* dst, const void* src, uint64_t bytes) { copy(stream, dst, src, bytes); }

    // One thread, block after block in id order: the host flavour's "kernels".
    void launch_gather(Stream stream, const uint8_t* pool, const uint32_t* ids, uint8_t* staging, uint64_t block_bytes,
                       uint32_t blocks) {
        enqueue(stream, [=] {
            for (uint32_t i = 0; i < blocks; ++i)
                memcpy(staging + uint64_t(i) * block_bytes, pool + uint64_t(ids[i]) * block_bytes, block_bytes);
        });
    }

    void launch_scatter(Stream stream, uint8_t* pool, const uint32_t* ids, const uint8_t* staging, uint64_t block_bytes,
                        uint32_t blocks) {
        enqueue(stream, [=] {
            for (uint32_t i = 0; i < blocks; ++i)
                memcpy(pool + uint64_t(ids[i]) * block_bytes, staging + uint64_t(i) * block_bytes, block_bytes);
        });
    }

    void call(Stream stream, lt_host_kernel kernel, void* context) {
        enqueue(stream, [this, kernel, context] {
            if (kernel(context) != 0) {
                std::lock_guard<std::mutex> hold(lock_);
                failure_ = "a host kernel failed";
                changed_.notify_all();
            }
        });
    }

    // A stream for caller kernels, owned by the device and drained before it goes away.
    Stream caller_stream() {
        if (!caller_stream_) caller_stream_.reset(new OwnedStream{this, stream_create()});
        return caller_stream_->stream;
    }

    void set_paused(bool paused) {
        std::lock_guard<std::mutex> hold(lock_);
        paused_ = paused;
        changed_.notify_all();
    }

    void set_copy_delay_us(uint32_t delay_us) {
        std::lock_guard<std::mutex> hold(lock_);
        copy_delay_us_ = delay_us;
    }

   private:
    struct OwnedStream {
        HostDevice* device;
        Stream stream;
        ~OwnedStream() {
            device->stream_sync(stream);
            device->stream_destroy(stream);
        }
    };

    void copy(Stream stream, void* dst, const void* src, uint64_t bytes) {
        enqueue(stream, [this, dst, src, bytes] {
            uint32_t delay;
            {
                std::lock_guard<std::mutex> hold(lock_);
                delay = copy_delay_us_;
            }
            if (delay) std::this_thread::sleep_for(std::chrono::microseconds(delay));
            memcpy(dst, src, bytes);
        });
    }

    void enqueue(Stream stream, std::function<void()> command) {
        std::lock_guard<std::mutex> hold(lock_);
        stream->pending.push_back(std::move(command));
        changed_.notify_all();
    }

    void serve(Stream stream) {
        std::unique_lock<std::mutex> hold(lock_);
        for (;;) {
            changed_.wait(hold, [&] { return stream->closing || (!stream->pending.empty() && !paused_); });
            // Closing while paused drops what is queued, so a paused teardown cannot hang.
            if (stream->closing && (stream->pending.empty() || paused_)) return;
            std::function<void()> command = std::move(stream->pending.front());
            stream->pending.pop_front();
            stream->running = true;
            hold.unlock();
            command();
            hold.lock();
            stream->running = false;
            changed_.notify_all();
        }
    }

    std::mutex lock_;
    std::condition_variable changed_;
    bool paused_ = false;
    uint32_t copy_delay_us_ = 0;
    std::string failure_;
    std::map<void*, uint64_t> pinned_;
    uint64_t pinned_total_ = 0;
    uint64_t pin_limit_ = UINT64_MAX;
    std::unique_ptr<OwnedStream> caller_stream_;
};

}  // namespace lt

#endif  // LAYOVER_AMD_HOST_DEVICE_H
