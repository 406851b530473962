// The host flavour's device back end: HIP's stream and event model played by host threads, so
// the swap engine and everything above it runs and is tested without a GPU (the reference's
// native/host_device.h has the same role).
//
// Model:
//   Lane  one stream: a worker thread draining its own queue of operations in order.
//   Mark  one event: `issued` counts records enqueued, `passed` the highest record a lane has
//         run. A record enqueues "passed = max(passed, n)" for its own number n, so a later
//         record supersedes an earlier one; a wait or query compares against the `issued`
//         value of the moment it is made, so it never sees records enqueued after it.
//   Board one mutex and condition variable on which marks passing, the pause switch and a
//         failed host kernel are announced; lanes block on it for waits and for the pause.
// Test controls: a pause holding every lane before its next operation, a delay before each
// copy, a cap on pinned bytes, and host "kernels" whose nonzero return is a device failure.
#ifndef LAYOVER_AMD_HOST_STREAMS_H
#define LAYOVER_AMD_HOST_STREAMS_H

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>

#include "layover_transfer.h"

namespace lt {

class HostDevice {
   public:
    struct Mark {
        std::atomic<uint64_t> issued{0};
        std::atomic<uint64_t> passed{0};
    };

    class Lane {
       public:
        explicit Lane(HostDevice* owner) : owner_(owner), worker_([this] { drain(); }) {}

        ~Lane() {
            {
                std::lock_guard<std::mutex> hold(mutex_);
                stop_ = true;
            }
            wake_.notify_all();
            worker_.join();
        }

        void push(std::function<void()> op) {
            {
                std::lock_guard<std::mutex> hold(mutex_);
                ops_.push_back(std::move(op));
                ++outstanding_;
            }
            wake_.notify_all();
        }

        void settle() {
            std::unique_lock<std::mutex> hold(mutex_);
            wake_.wait(hold, [&] { return outstanding_ == 0; });
        }

       private:
        void drain() {
            for (;;) {
                std::function<void()> op;
                {
                    std::unique_lock<std::mutex> hold(mutex_);
                    wake_.wait(hold, [&] { return stop_ || !ops_.empty(); });
                    if (ops_.empty()) return;
                    op = std::move(ops_.front());
                    ops_.pop_front();
                }
                owner_->pass_gate();
                op();
                {
                    std::lock_guard<std::mutex> hold(mutex_);
                    --outstanding_;
                }
                wake_.notify_all();
            }
        }

        HostDevice* owner_;
        std::mutex mutex_;
        std::condition_variable wake_;
        std::deque<std::function<void()>> ops_;
        uint64_t outstanding_ = 0;
        bool stop_ = false;
        std::thread worker_;  // last: starts once the members above exist
    };

    using Stream = Lane*;
    using Event = Mark*;

    static const char* flavor() { return "host"; }
    static Stream stream_from_handle(void* handle) { return static_cast<Stream>(handle); }

    explicit HostDevice(int) {}

    ~HostDevice() {
        if (spare_) spare_->settle();
        spare_.reset();
    }

    HostDevice(const HostDevice&) = delete;
    HostDevice& operator=(const HostDevice&) = delete;

    // Each engine call starts here; a failed host kernel fails every call after it.
    void activate() { raise_failure(); }

    void check_pool(const void*) {}

    // Teardown must not hang on lanes a test left paused.
    void prepare_teardown() { set_paused(false); }

    void* device_alloc(uint64_t bytes) {
        void* pointer = nullptr;
        if (posix_memalign(&pointer, 4096, bytes == 0 ? 1 : bytes) != 0) throw std::runtime_error("device_alloc: out of memory");
        return pointer;
    }
    void device_free(void* pointer) { free(pointer); }

    // Null when the request would pass the pin cap or memory runs out: the engine survives it.
    void* host_alloc(uint64_t bytes) {
        if (pinned_bytes_ > pin_cap_ || bytes > pin_cap_ - pinned_bytes_) return nullptr;
        void* pointer = nullptr;
        if (posix_memalign(&pointer, 4096, bytes) != 0) return nullptr;
        pinned_.emplace(pointer, bytes);
        pinned_bytes_ += bytes;
        return pointer;
    }

    void host_free(void* pointer) {
        const auto found = pinned_.find(pointer);
        if (found != pinned_.end()) {
            pinned_bytes_ -= found->second;
            pinned_.erase(found);
        }
        free(pointer);
    }

    Stream stream_create() { return new Lane(this); }
    void stream_sync(Stream stream) { stream->settle(); }
    void stream_destroy(Stream stream) { delete stream; }

    Event event_create() { return new Mark(); }
    void event_destroy(Event event) { delete event; }

    void event_record(Event event, Stream stream) {
        const uint64_t number = event->issued.fetch_add(1) + 1;
        stream->push([this, event, number] {
            std::lock_guard<std::mutex> hold(board_);
            if (event->passed.load() < number) event->passed.store(number);
            board_changed_.notify_all();
        });
    }

    void stream_wait(Stream stream, Event event) {
        const uint64_t target = event->issued.load();
        stream->push([this, event, target] {
            std::unique_lock<std::mutex> hold(board_);
            board_changed_.wait(hold, [&] { return event->passed.load() >= target; });
        });
    }

    bool event_query(Event event) {
        raise_failure();
        return event->passed.load() >= event->issued.load();
    }

    void event_sync(Event event) {
        const uint64_t target = event->issued.load();
        std::unique_lock<std::mutex> hold(board_);
        board_changed_.wait(hold, [&] { return event->passed.load() >= target || !failure_.empty(); });
        if (!failure_.empty()) throw std::runtime_error(failure_);
    }

    void memcpy_to_host(Stream stream, void* dst, const void* src, uint64_t bytes) { push_copy(stream, dst, src, bytes); }
    void memcpy_to_device(Stream stream, void* dst, const void* src, uint64_t bytes) { push_copy(stream, dst, src, bytes); }

    // Host copies have no per-launch size limit.
    bool launch_fits(uint64_t, uint64_t) const { return true; }

    // Block copies in the order of ids: block i of the staging buffer is pool block ids[i].
    void launch_gather(Stream stream, const uint8_t* pool, const uint32_t* ids, uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        stream->push([=] {
            for (uint32_t i = 0; i < blocks; ++i) memcpy(staging + uint64_t(i) * block_bytes, pool + uint64_t(ids[i]) * block_bytes, block_bytes);
        });
    }

    void launch_scatter(Stream stream, uint8_t* pool, const uint32_t* ids, const uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        stream->push([=] {
            for (uint32_t i = 0; i < blocks; ++i) memcpy(pool + uint64_t(ids[i]) * block_bytes, staging + uint64_t(i) * block_bytes, block_bytes);
        });
    }

    // ---- the host-only controls of include/layover_transfer.h ----

    // One extra lane for the caller's own "kernels", made on first request and kept until the
    // device goes away.
    Stream caller_lane() {
        if (!spare_) spare_.reset(new Lane(this));
        return spare_.get();
    }

    void run_host_kernel(Stream stream, lt_host_kernel kernel, void* context) {
        stream->push([this, kernel, context] {
            if (kernel(context) == 0) return;
            std::lock_guard<std::mutex> hold(board_);
            failure_ = "a host kernel failed";
            board_changed_.notify_all();
        });
    }

    void set_paused(bool paused) {
        std::lock_guard<std::mutex> hold(board_);
        paused_ = paused;
        board_changed_.notify_all();
    }

    void set_copy_delay_us(uint32_t delay_us) { copy_delay_us_.store(delay_us); }
    void set_pin_limit(uint64_t bytes) { pin_cap_ = bytes; }

   private:
    void pass_gate() {
        std::unique_lock<std::mutex> hold(board_);
        board_changed_.wait(hold, [&] { return !paused_; });
    }

    void raise_failure() {
        std::lock_guard<std::mutex> hold(board_);
        if (!failure_.empty()) throw std::runtime_error(failure_);
    }

    void push_copy(Stream stream, void* dst, const void* src, uint64_t bytes) {
        stream->push([this, dst, src, bytes] {
            const uint32_t delay = copy_delay_us_.load();
            if (delay != 0) std::this_thread::sleep_for(std::chrono::microseconds(delay));
            memcpy(dst, src, bytes);
        });
    }

    std::mutex board_;
    std::condition_variable board_changed_;
    bool paused_ = false;
    std::string failure_;
    std::atomic<uint32_t> copy_delay_us_{0};

    std::unordered_map<void*, uint64_t> pinned_;
    uint64_t pinned_bytes_ = 0;
    uint64_t pin_cap_ = UINT64_MAX;
    std::unique_ptr<Lane> spare_;
};

}  // namespace lt

#endif  // LAYOVER_AMD_HOST_STREAMS_H
