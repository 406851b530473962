// The transfer engine behind include/layover_transfer.h, written once against a small device
// interface (`Dev`) so the host flavour (host threads) and the HIP flavour run the same
// segmenting, slot events, id ring and pinned cache.
//
// Behaviour follows the reference engine (native/transfer_core.h:57-567); the structure is
// this library's own: the pinned cache, the id ring and the transfer list are separate
// classes, and the C exports live in transfer_exports.h.
//
// Pipeline of one staged transfer, per segment on slot s (transfer_core.h:5-10, :179-225):
//   out: compute waits s.released -> gather into s -> record s.filled
//        copy    waits s.filled   -> DMA s to host -> record s.released
//   in:  copy    waits s.released -> DMA host to s -> record s.filled
//        compute waits s.filled   -> scatter from s -> record s.released
// Everything is enqueued at once. A stream is FIFO and a wait captures the event's latest
// record, so every dependency points backwards in enqueue order and the pipeline cannot
// deadlock. Two slots let segment i+1's kernel overlap segment i's DMA.
#ifndef LAYOVER_AMD_TRANSFER_ENGINE_H
#define LAYOVER_AMD_TRANSFER_ENGINE_H

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <deque>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "layover_transfer.h"

namespace lt {

// Misuse: std::invalid_argument -> LT_ERR_INVALID, engine unchanged.
// Host memory exhausted: OutOfHostMemory -> LT_ERR_NOMEM, engine usable.
// Anything else is a device failure -> LT_ERR_DEVICE, and the engine refuses further work.
struct OutOfHostMemory : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline thread_local std::string last_error;

// Segments are capped at this many blocks. HIP has no 65,535 grid-y limit, but the reference
// derives its segment count from it (native/pack.h:26-28, transfer_core.h:356-358) and its
// tests count kernels and copies per transfer, so the same cap keeps the counts identical.
constexpr uint32_t kSegmentBlockCap = 65535;

inline bool aligned8(const void* pointer, uint64_t bytes) {
    return (reinterpret_cast<uintptr_t>(pointer) & 7) == 0 && (bytes & 7) == 0;
}

// Pinned buffers are rounded up to one of four classes per doubling, at least 1 MiB, so a
// freed buffer serves the next request of similar size while wasting at most a quarter
// (transfer_core.h:45-55): above 1 MiB, the class step is a quarter of the largest power of
// two strictly below the request.
inline uint64_t pinned_class(uint64_t bytes) {
    constexpr uint64_t kFloor = uint64_t(1) << 20;
    if (bytes <= kFloor) return kFloor;
    uint64_t below = kFloor;  // grows to the largest power of two strictly below `bytes`
    while (below * 2 < bytes) below <<= 1;
    const uint64_t step = below / 4;
    return (bytes + step - 1) / step * step;
}

// Pinned host memory handed out by lt_host_alloc and cached after lt_host_free, up to a
// byte limit, evicting what was returned longest ago (transfer_core.h:133-177, :522-534).
template <class Dev>
class PinnedCache {
   public:
    PinnedCache(Dev& dev, uint64_t limit, lt_stats& stats) : dev_(dev), limit_(limit), stats_(stats) {}

    void* take(uint64_t bytes) {
        if (bytes == 0 || bytes > (uint64_t(1) << 62)) throw std::invalid_argument("cannot allocate that many bytes");
        const uint64_t size = pinned_class(bytes);
        void* pointer = reuse(size);
        if (pointer == nullptr) {
            pointer = pin(size);
            // The cached buffers are the only host memory this engine can give back.
            if (pointer == nullptr && cached_bytes_ > 0) {
                while (cached_bytes_ > 0) evict_oldest();
                pointer = pin(size);
            }
            if (pointer == nullptr) {
                stats_.host_pin_failures++;
                throw OutOfHostMemory("cannot pin " + std::to_string(size) + " bytes of host memory");
            }
            held_ += size;
        }
        live_[pointer] = size;
        stats_.host_bytes_live += size;
        return pointer;
    }

    void give_back(void* pointer) {
        auto entry = live_.find(pointer);
        if (entry == live_.end()) throw std::invalid_argument("not a live host buffer of this engine");
        const uint64_t size = entry->second;
        live_.erase(entry);
        stats_.host_bytes_live -= size;
        if (size > limit_) {
            dev_.host_free(pointer);
            held_ -= size;
            return;
        }
        while (cached_bytes_ + size > limit_) evict_oldest();
        idle_[size].push_back({pointer, ++clock_});
        cached_bytes_ += size;
    }

    uint64_t held() const { return held_; }

    // Frees every buffer, live or cached. Reports failures through `note`.
    template <class Note>
    void release_all(Note&& note) {
        for (auto& entry : live_) note([&] { dev_.host_free(entry.first); });
        live_.clear();
        for (auto& bucket : idle_)
            for (const Idle& idle : bucket.second) note([&] { dev_.host_free(idle.pointer); });
        idle_.clear();
        cached_bytes_ = held_ = 0;
    }

   private:
    struct Idle {
        void* pointer;
        uint64_t returned_at;
    };

    void* reuse(uint64_t size) {
        auto bucket = idle_.find(size);
        if (bucket == idle_.end()) return nullptr;
        // The most recently returned buffer of the class: its pages are the warmest.
        void* pointer = bucket->second.back().pointer;
        bucket->second.pop_back();
        if (bucket->second.empty()) idle_.erase(bucket);
        cached_bytes_ -= size;
        return pointer;
    }

    // Pinning runs on the calling thread and stalls it; the stats make every stall visible.
    void* pin(uint64_t size) {
        const auto start = std::chrono::steady_clock::now();
        void* pointer = dev_.host_alloc(size);
        const uint64_t ns = uint64_t(
            std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - start).count());
        stats_.host_pins++;
        stats_.host_pin_ns += ns;
        stats_.host_pin_max_ns = std::max(stats_.host_pin_max_ns, ns);
        if (pointer != nullptr) stats_.host_pin_bytes += size;
        return pointer;
    }

    void evict_oldest() {
        auto victim = idle_.end();
        for (auto bucket = idle_.begin(); bucket != idle_.end(); ++bucket) {
            if (victim == idle_.end() || bucket->second.front().returned_at < victim->second.front().returned_at)
                victim = bucket;
        }
        const uint64_t size = victim->first;
        void* pointer = victim->second.front().pointer;
        victim->second.pop_front();
        if (victim->second.empty()) idle_.erase(victim);
        cached_bytes_ -= size;
        held_ -= size;
        dev_.host_free(pointer);
    }

    Dev& dev_;
    uint64_t limit_;
    lt_stats& stats_;
    std::map<void*, uint64_t> live_;
    std::map<uint64_t, std::deque<Idle>> idle_;  // per class, oldest first; never empty
    uint64_t clock_ = 0;
    uint64_t cached_bytes_ = 0;
    uint64_t held_ = 0;
};

// Positions in a ring of `capacity` block ids. A reservation is contiguous (it skips the
// tail end of the ring when it would not fit there) and is held until its transfer has
// finished; space comes back in reservation order (transfer_core.h:406-455).
class IdRing {
   public:
    explicit IdRing(uint64_t capacity) : capacity_(capacity) {}

    // Offset of a reservation of `count` ids, or -1 when the ring is too full right now.
    int64_t try_reserve(uint64_t count, uint64_t* end) {
        if (head_ == tail_) head_ = tail_ = 0;  // empty: start over, so a full-size run fits
        const uint64_t offset = head_ % capacity_;
        const uint64_t skip = offset + count > capacity_ ? capacity_ - offset : 0;
        if (head_ + skip + count - tail_ > capacity_) return -1;
        head_ += skip;
        const uint64_t start = head_ % capacity_;
        head_ += count;
        *end = head_;
        return int64_t(start);
    }

    void reclaim_to(uint64_t end) { tail_ = end; }

   private:
    uint64_t capacity_;
    uint64_t head_ = 0;
    uint64_t tail_ = 0;
};

template <class Dev>
class Engine {
    using Stream = typename Dev::Stream;
    using Event = typename Dev::Event;

    struct Slot {
        void* staging = nullptr;
        Event filled{};
        Event released{};
    };

   public:
    struct Transfer {
        Event done{};
        uint64_t ring_end = 0;
        bool holds_ring = false;
        bool finished = false;
        bool released = false;
    };

    Engine(int device, uint64_t staging_bytes, uint32_t num_staging, uint32_t ids_capacity, uint64_t host_cache_bytes)
        : dev_(device),
          staging_bytes_(staging_bytes),
          ids_capacity_(ids_capacity),
          ring_(ids_capacity == 0 ? 1 : ids_capacity),
          host_(dev_, host_cache_bytes, stats_) {
        if (staging_bytes == 0 || num_staging == 0 || ids_capacity == 0)
            throw std::invalid_argument("staging_bytes, num_staging and ids_capacity must be positive");
        try {
            compute_ = dev_.stream_create();
            have_compute_ = true;
            copy_ = dev_.stream_create();
            have_copy_ = true;
            own_.resize(num_staging);
            ext_.resize(num_staging);
            for (auto* slots : {&own_, &ext_})
                for (Slot& slot : *slots) {
                    slot.filled = make_event();
                    slot.released = make_event();
                }
            ids_host_ = static_cast<uint32_t*>(dev_.host_alloc(uint64_t(ids_capacity) * 4));
            if (ids_host_ == nullptr) throw std::runtime_error("cannot pin the block-id ring");
            ids_device_ = static_cast<uint32_t*>(dev_.device_alloc(uint64_t(ids_capacity) * 4));
        } catch (...) {
            teardown();
            throw;
        }
    }

    ~Engine() { teardown(); }

    Dev& device() { return dev_; }
    void mark_failed() { failed_ = true; }

    void prepare_staging() {
        for (Slot& slot : own_)
            if (slot.staging == nullptr) slot.staging = dev_.device_alloc(staging_bytes_);
    }

    std::string shutdown() {
        teardown();
        return teardown_error_;
    }

    lt_stats stats() const {
        lt_stats out = stats_;
        out.host_bytes_held = host_.held();
        return out;
    }

    void* host_alloc(uint64_t bytes) {
        require_healthy();
        return host_.take(bytes);
    }

    void host_free(void* pointer) {
        require_healthy();
        host_.give_back(pointer);
    }

    Transfer* out_gather(const uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, uint8_t* host) {
        check_staged(pool, block_bytes, ids, count, host);
        prepare_staging();
        uint64_t ring_end = 0;
        const uint32_t* device_ids = upload_ids(ids, count, &ring_end);
        Transfer* transfer = begin(ring_end);
        for_each_segment(block_bytes, count, [&](uint64_t first, uint32_t blocks, Slot& slot) {
            const uint64_t bytes = uint64_t(blocks) * block_bytes;
            wait(compute_, slot.released);
            dev_.launch_gather(compute_, pool, device_ids + first, static_cast<uint8_t*>(slot.staging), block_bytes, blocks);
            stats_.kernels++;
            dev_.event_record(slot.filled, compute_);
            wait(copy_, slot.filled);
            dev_.memcpy_to_host(copy_, host + first * block_bytes, slot.staging, bytes);
            copied(bytes, true);
            dev_.event_record(slot.released, copy_);
        });
        dev_.event_record(transfer->done, copy_);
        return transfer;
    }

    Transfer* in_scatter(uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const uint8_t* host) {
        check_staged(pool, block_bytes, ids, count, host);
        prepare_staging();
        uint64_t ring_end = 0;
        const uint32_t* device_ids = upload_ids(ids, count, &ring_end);
        Transfer* transfer = begin(ring_end);
        for_each_segment(block_bytes, count, [&](uint64_t first, uint32_t blocks, Slot& slot) {
            const uint64_t bytes = uint64_t(blocks) * block_bytes;
            wait(copy_, slot.released);
            dev_.memcpy_to_device(copy_, slot.staging, host + first * block_bytes, bytes);
            copied(bytes, false);
            dev_.event_record(slot.filled, copy_);
            wait(compute_, slot.filled);
            dev_.launch_scatter(compute_, pool, device_ids + first, static_cast<const uint8_t*>(slot.staging), block_bytes, blocks);
            stats_.kernels++;
            dev_.event_record(slot.released, compute_);
        });
        dev_.event_record(transfer->done, compute_);
        return transfer;
    }

    Transfer* out_per_block(const uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, uint8_t* host) {
        check_blocks(pool, block_bytes, ids, count, host);
        Transfer* transfer = begin(0);
        for (uint32_t i = 0; i < count; ++i) {
            dev_.memcpy_to_host(copy_, host + uint64_t(i) * block_bytes, pool + uint64_t(ids[i]) * block_bytes, block_bytes);
            copied(block_bytes, true);
        }
        dev_.event_record(transfer->done, copy_);
        return transfer;
    }

    Transfer* in_per_block(uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const uint8_t* host) {
        check_blocks(pool, block_bytes, ids, count, host);
        Transfer* transfer = begin(0);
        for (uint32_t i = 0; i < count; ++i) {
            dev_.memcpy_to_device(copy_, pool + uint64_t(ids[i]) * block_bytes, host + uint64_t(i) * block_bytes, block_bytes);
            copied(block_bytes, false);
        }
        dev_.event_record(transfer->done, copy_);
        return transfer;
    }

    void ext_wait(void* stream, uint32_t slot, int which) {
        require_healthy();
        wait(caller(stream), ext_event(slot, which));
    }

    void ext_record(void* stream, uint32_t slot, int which) {
        require_healthy();
        dev_.event_record(ext_event(slot, which), caller(stream));
    }

    void ext_copy_out(const void* staging, uint8_t* host, uint64_t bytes, uint32_t slot) {
        require_healthy();
        Event filled = ext_event(slot, LT_SLOT_FILLED);
        Event released = ext_event(slot, LT_SLOT_RELEASED);
        check_ext(staging, host, bytes);
        wait(copy_, filled);
        dev_.memcpy_to_host(copy_, host, staging, bytes);
        copied(bytes, true);
        dev_.event_record(released, copy_);
    }

    void ext_copy_in(void* staging, const uint8_t* host, uint64_t bytes, uint32_t slot) {
        require_healthy();
        Event filled = ext_event(slot, LT_SLOT_FILLED);
        Event released = ext_event(slot, LT_SLOT_RELEASED);
        check_ext(staging, host, bytes);
        wait(copy_, released);
        dev_.memcpy_to_device(copy_, staging, host, bytes);
        copied(bytes, false);
        dev_.event_record(filled, copy_);
    }

    Transfer* ext_finish(void* stream) {
        require_healthy();
        Stream on = stream == nullptr ? copy_ : caller(stream);
        Transfer* transfer = begin(0);
        dev_.event_record(transfer->done, on);
        return transfer;
    }

    bool poll(Transfer* transfer) {
        require_live(transfer);
        if (!transfer->finished && dev_.event_query(transfer->done)) transfer->finished = true;
        if (transfer->finished) settle();
        return transfer->finished;
    }

    void wait_for(Transfer* transfer) {
        require_live(transfer);
        if (!transfer->finished) {
            dev_.event_sync(transfer->done);
            transfer->finished = true;
        }
        settle();
    }

    void release(Transfer* transfer) {
        require_live(transfer);
        if (!poll(transfer)) throw std::invalid_argument("transfer is still in flight");
        transfer->released = true;
        settle();
    }

   private:
    Event make_event() {
        Event event = dev_.event_create();
        events_.push_back(event);
        return event;
    }

    void require_healthy() const {
        if (failed_) throw std::runtime_error("engine refused work after an earlier device failure");
    }

    void check_blocks(const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const void* host) {
        require_healthy();
        if (pool == nullptr || host == nullptr || block_bytes == 0 || (ids == nullptr && count != 0))
            throw std::invalid_argument("null pool, host or ids, or zero block_bytes");
        dev_.check_pool(pool);
    }

    void check_staged(const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const void* host) {
        check_blocks(pool, block_bytes, ids, count, host);
        if (!aligned8(pool, block_bytes) || !aligned8(host, block_bytes))
            throw std::invalid_argument("pool and host must be 8-byte aligned and block_bytes a multiple of 8");
        if (block_bytes > staging_bytes_) throw std::invalid_argument("one block is larger than a staging buffer");
        if (count > ids_capacity_) throw std::invalid_argument("transfer has more blocks than ids_capacity");
    }

    static void check_ext(const void* staging, const void* host, uint64_t bytes) {
        if (staging == nullptr || host == nullptr || bytes == 0)
            throw std::invalid_argument("null staging or host, or zero bytes");
    }

    // A null stream would be the legacy default stream, which synchronizes with everything
    // and would silently serialize the copy stream against the caller's work.
    static Stream caller(void* stream) {
        if (stream == nullptr) throw std::invalid_argument("null stream");
        return Dev::stream_from_handle(stream);
    }

    Event ext_event(uint32_t slot, int which) {
        if (slot >= ext_.size() || (which != LT_SLOT_FILLED && which != LT_SLOT_RELEASED))
            throw std::invalid_argument("bad slot or event");
        return which == LT_SLOT_FILLED ? ext_[slot].filled : ext_[slot].released;
    }

    template <class Body>
    void for_each_segment(uint64_t block_bytes, uint32_t count, Body&& body) {
        const uint32_t per_segment = uint32_t(std::min<uint64_t>(staging_bytes_ / block_bytes, kSegmentBlockCap));
        for (uint64_t first = 0; first < count; first += per_segment) {
            const uint32_t blocks = uint32_t(std::min<uint64_t>(per_segment, count - first));
            Slot& slot = own_[next_slot_];
            next_slot_ = (next_slot_ + 1) % uint32_t(own_.size());
            body(first, blocks, slot);
        }
    }

    void wait(Stream stream, Event event) {
        dev_.stream_wait(stream, event);
        stats_.stream_waits++;
    }

    void copied(uint64_t bytes, bool to_host) {
        stats_.memcpys++;
        (to_host ? stats_.bytes_to_host : stats_.bytes_to_device) += bytes;
    }

    // The caller records the completion right after this, with nothing in between that
    // inspects transfers: an event never recorded would read as complete.
    Transfer* begin(uint64_t ring_end) {
        auto transfer = std::make_unique<Transfer>();
        transfer->done = dev_.event_create();
        transfer->ring_end = ring_end;
        transfer->holds_ring = ring_end != 0;
        Transfer* raw = transfer.get();
        transfers_.push_back(std::move(transfer));
        stats_.transfers++;
        return raw;
    }

    // Copies the ids into the pinned ring and uploads them on the compute stream, ahead of the
    // kernels that read them. A pageable source would make the async copy synchronous.
    const uint32_t* upload_ids(const uint32_t* ids, uint32_t count, uint64_t* ring_end) {
        if (count == 0) return nullptr;
        int64_t offset;
        while ((offset = ring_.try_reserve(count, ring_end)) < 0) wait_for_oldest_ring_holder();
        memcpy(ids_host_ + offset, ids, uint64_t(count) * 4);
        dev_.memcpy_to_device(compute_, ids_device_ + offset, ids_host_ + offset, uint64_t(count) * 4);
        stats_.ids_uploads++;
        return ids_device_ + offset;
    }

    void wait_for_oldest_ring_holder() {
        for (const auto& transfer : transfers_) {
            if (transfer->holds_ring) {
                wait_for(transfer.get());
                return;
            }
        }
        throw std::logic_error("id ring is full with nothing in flight");
    }

    // Marks transfers finished in order, returns their ring space in reservation order and
    // drops those that are finished and released from the front of the list.
    void settle() {
        for (const auto& transfer : transfers_) {
            if (!transfer->finished) {
                if (!dev_.event_query(transfer->done)) break;
                transfer->finished = true;
            }
            if (transfer->holds_ring) {
                ring_.reclaim_to(transfer->ring_end);
                transfer->holds_ring = false;
            }
        }
        while (!transfers_.empty() && transfers_.front()->finished && transfers_.front()->released) {
            dev_.event_destroy(transfers_.front()->done);
            transfers_.pop_front();
        }
    }

    void require_live(Transfer* transfer) const {
        for (const auto& known : transfers_)
            if (known.get() == transfer && !known->released) return;
        throw std::invalid_argument("not a live transfer of this engine");
    }

    template <class Fn>
    void quietly(Fn&& fn) {
        try {
            fn();
        } catch (const std::exception& error) {
            if (teardown_error_.empty()) teardown_error_ = error.what();
        }
    }

    // Waits for every transfer (some end on caller streams this engine cannot synchronize),
    // then its own streams, and only then frees memory.
    void teardown() {
        if (torn_down_) return;
        torn_down_ = true;
        dev_.prepare_teardown();
        for (const auto& transfer : transfers_)
            if (!transfer->finished) quietly([&] { dev_.event_sync(transfer->done); });
        if (have_compute_) quietly([&] { dev_.stream_sync(compute_); });
        if (have_copy_) quietly([&] { dev_.stream_sync(copy_); });
        for (const auto& transfer : transfers_) quietly([&] { dev_.event_destroy(transfer->done); });
        transfers_.clear();
        for (Event event : events_) quietly([&] { dev_.event_destroy(event); });
        events_.clear();
        for (Slot& slot : own_)
            if (slot.staging != nullptr) quietly([&] { dev_.device_free(slot.staging); });
        own_.clear();
        ext_.clear();
        if (ids_device_ != nullptr) quietly([&] { dev_.device_free(ids_device_); });
        if (ids_host_ != nullptr) quietly([&] { dev_.host_free(ids_host_); });
        host_.release_all([&](auto&& fn) { quietly(fn); });
        if (have_copy_) quietly([&] { dev_.stream_destroy(copy_); });
        if (have_compute_) quietly([&] { dev_.stream_destroy(compute_); });
    }

    Dev dev_;
    uint64_t staging_bytes_;
    uint32_t ids_capacity_;
    lt_stats stats_{};
    IdRing ring_;
    PinnedCache<Dev> host_;

    Stream compute_{};
    Stream copy_{};
    bool have_compute_ = false;
    bool have_copy_ = false;
    std::vector<Slot> own_;
    std::vector<Slot> ext_;
    std::vector<Event> events_;
    uint32_t next_slot_ = 0;
    uint32_t* ids_host_ = nullptr;
    uint32_t* ids_device_ = nullptr;
    std::deque<std::unique_ptr<Transfer>> transfers_;

    bool failed_ = false;
    bool torn_down_ = false;
    std::string teardown_error_;
};

}  // namespace lt

#endif  // LAYOVER_AMD_TRANSFER_ENGINE_H
