// The swap engine behind include/layover_transfer.h: one template over a device back end
// (`Dev`), instantiated by the HIP flavour (transfer_hip.hip) and by the host flavour
// (transfer_host.cc, host threads standing in for streams), and the C exports over it.
//
// Behaviour is the reference engine's (native/transfer_core.h:57-567, :581-732): the same
// segments, slot events, block-id upload, pinned cache policy, counters and error codes.
// The organisation is this file's own:
//
//   Fault       every error carries its LT_ERR_* code; the export wrapper maps it.
//   HostCache   pinned buffers: one list of idle buffers in the order they came back.
//   IdArena     the block-id ring as a FIFO of live spans over one pinned array and its
//               device mirror, each span owned by the ticket of the transfer that uses it.
//   SwapEngine  streams, staging slots and tickets; one `staged` loop serves both
//               directions, each segment being a fill step on one stream and a drain step
//               on the other, with the slot's two events between them.
//
// A staged segment on slot s:
//   to host:   compute  wait s.released, gather into s, record s.filled
//              copy     wait s.filled,   copy s to host, record s.released
//   to device: copy     wait s.released, copy host to s, record s.filled
//              compute  wait s.filled,   scatter from s, record s.released
// All of a transfer is enqueued before the call returns. Streams run in order and a wait
// binds to the event's latest record, so each wait points at work enqueued earlier: the
// graph has no cycle. With two slots, segment i+1's fill overlaps segment i's drain.
//
// The compute stream is created on first use: the FP8 path launches its own kernels on the
// caller's stream and only uses the copy stream, and on MI355X every stream a process
// creates takes one of a few hardware queues.
#ifndef LAYOVER_AMD_SWAP_ENGINE_H
#define LAYOVER_AMD_SWAP_ENGINE_H

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <deque>
#include <exception>
#include <list>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "layover_transfer.h"

namespace lt {

// An error with the code the C ABI reports for it. LT_ERR_INVALID: nothing changed.
// LT_ERR_NOMEM: pinning failed, nothing was enqueued. LT_ERR_DEVICE: the engine is unusable
// from then on. Device back ends may throw any std::exception for a device failure.
struct Fault : std::runtime_error {
    int code;
    Fault(int status, const std::string& text) : std::runtime_error(text), code(status) {}
};

[[noreturn]] inline void misuse(const std::string& text) { throw Fault(LT_ERR_INVALID, text); }

inline thread_local std::string last_error;

// The reference cuts segments at 65,535 blocks, its CUDA grid-y limit (pack.h:26-28,
// transfer_core.h:356-358). HIP grids have no such limit, but the kernel and copy counts its
// tests assert follow from the cap, so it is kept.
constexpr uint64_t kMaxSegmentBlocks = 65535;

inline bool eight_byte_words(const void* pointer, uint64_t block_bytes) {
    return ((reinterpret_cast<uintptr_t>(pointer) | block_bytes) & 7) == 0;
}

// Pinned sizes: at or below 1 MiB, 1 MiB; above it, rounded up to a multiple of a quarter of
// the largest power of two below the request (transfer_core.h:45-55), so a reused buffer
// wastes at most a quarter of itself.
inline uint64_t pinned_size(uint64_t bytes) {
    const uint64_t mib = uint64_t(1) << 20;
    if (bytes <= mib) return mib;
    const int top = 63 - __builtin_clzll(bytes - 1);  // 2^top < bytes <= 2^(top+1)
    const uint64_t quarter = (uint64_t(1) << top) >> 2;
    return (bytes + quarter - 1) / quarter * quarter;
}

// Pinned host memory for payloads. Handed-out buffers are counted live; returned ones wait in
// `idle_` (oldest first) up to `limit_` bytes for a request of the same size. A request takes
// the most recently returned buffer of its size. Room is made by freeing the oldest idle
// buffers, whatever their size: sizes only grow with context, so the oldest are the least
// likely to be asked for again (transfer_core.h:133-177, :522-534).
template <class Dev>
class HostCache {
   public:
    HostCache(Dev& dev, uint64_t limit, lt_stats& stats) : dev_(dev), limit_(limit), stats_(stats) {}

    void* acquire(uint64_t bytes) {
        if (bytes == 0 || bytes > (uint64_t(1) << 62)) misuse("cannot allocate that many bytes");
        const uint64_t size = pinned_size(bytes);
        void* pointer = take_idle(size);
        if (pointer == nullptr) pointer = pin_new(size);
        live_.emplace(pointer, size);
        stats_.host_bytes_live += size;
        return pointer;
    }

    void give_back(void* pointer) {
        const auto found = live_.find(pointer);
        if (found == live_.end()) misuse("not a live host buffer of this engine");
        const uint64_t size = found->second;
        live_.erase(found);
        stats_.host_bytes_live -= size;
        if (size > limit_) {
            unpin(pointer, size);
            return;
        }
        while (idle_bytes_ + size > limit_) drop_oldest();
        idle_.push_back({pointer, size});
        idle_bytes_ += size;
    }

    uint64_t held() const { return held_; }

    template <class Quietly>
    void free_everything(Quietly&& quietly) {
        for (const auto& entry : live_) quietly([&] { dev_.host_free(entry.first); });
        for (const Idle& idle : idle_) quietly([&] { dev_.host_free(idle.pointer); });
        live_.clear();
        idle_.clear();
        idle_bytes_ = held_ = 0;
    }

   private:
    struct Idle {
        void* pointer;
        uint64_t size;
    };

    void* take_idle(uint64_t size) {
        for (auto it = idle_.rbegin(); it != idle_.rend(); ++it) {
            if (it->size != size) continue;
            void* pointer = it->pointer;
            idle_.erase(std::next(it).base());
            idle_bytes_ -= size;
            return pointer;
        }
        return nullptr;
    }

    // A miss pins new memory on the calling thread; if the host is out, the idle buffers
    // are all this engine can give back, and then it tries once more.
    void* pin_new(uint64_t size) {
        void* pointer = timed_pin(size);
        if (pointer == nullptr && !idle_.empty()) {
            while (!idle_.empty()) drop_oldest();
            pointer = timed_pin(size);
        }
        if (pointer == nullptr) {
            stats_.host_pin_failures++;
            throw Fault(LT_ERR_NOMEM, "cannot pin " + std::to_string(size) + " bytes of host memory");
        }
        held_ += size;
        return pointer;
    }

    // Every attempt is counted and timed, failures too: each one stalled its caller.
    void* timed_pin(uint64_t size) {
        const auto began = std::chrono::steady_clock::now();
        void* pointer = dev_.host_alloc(size);
        const uint64_t ns = uint64_t(std::chrono::nanoseconds(std::chrono::steady_clock::now() - began).count());
        stats_.host_pins++;
        stats_.host_pin_ns += ns;
        if (ns > stats_.host_pin_max_ns) stats_.host_pin_max_ns = ns;
        if (pointer != nullptr) stats_.host_pin_bytes += size;
        return pointer;
    }

    void drop_oldest() {
        const Idle oldest = idle_.front();
        idle_.pop_front();
        idle_bytes_ -= oldest.size;
        unpin(oldest.pointer, oldest.size);
    }

    void unpin(void* pointer, uint64_t size) {
        held_ -= size;
        dev_.host_free(pointer);
    }

    Dev& dev_;
    uint64_t limit_;
    lt_stats& stats_;
    std::unordered_map<void*, uint64_t> live_;
    std::list<Idle> idle_;
    uint64_t idle_bytes_ = 0;
    uint64_t held_ = 0;
};

// Where a transfer's block ids live on the device while its kernels may still read them: a
// contiguous span of a ring of `capacity` ids, kept until the transfer has finished. Spans are
// handed out in order and come back in the same order, so the free space is the gap from the
// newest span's end round to the oldest span's start. An empty ring starts again at 0, so a
// request of the full capacity always fits once the ring has drained.
class IdArena {
   public:
    explicit IdArena(uint64_t capacity) : capacity_(capacity) {}

    // The offset of a new span of `count` ids owned by `owner`, or -1 if it does not fit now.
    int64_t claim(uint64_t count, const void* owner) {
        uint64_t at;
        if (spans_.empty()) {
            at = 0;
        } else {
            const uint64_t head = spans_.back().offset + spans_.back().count;
            const uint64_t tail = spans_.front().offset;
            if (head > tail) {  // live ids in [tail, head): room after head, else from 0
                if (capacity_ - head >= count) at = head;
                else if (tail >= count) at = 0;
                else return -1;
            } else {  // wrapped: live ids in [tail, capacity) and [0, head)
                if (tail - head >= count) at = head;
                else return -1;
            }
        }
        spans_.push_back({at, count, owner});
        return int64_t(at);
    }

    bool empty() const { return spans_.empty(); }
    const void* oldest_owner() const { return spans_.front().owner; }
    void pop_oldest() { spans_.pop_front(); }

   private:
    struct Span {
        uint64_t offset;
        uint64_t count;
        const void* owner;
    };
    uint64_t capacity_;
    std::deque<Span> spans_;
};

enum class Direction { ToHost, ToDevice };

template <class Dev>
class SwapEngine {
    using Stream = typename Dev::Stream;
    using Event = typename Dev::Event;

    struct Slot {
        void* staging = nullptr;
        Event filled{};
        Event released{};
    };

   public:
    // What an lt_transfer* points at. It lives until it is both released by the caller and
    // no longer owns an id span.
    struct Ticket {
        Event done{};
        bool finished = false;
        bool released = false;
        bool owns_ids = false;
    };

    SwapEngine(int device, uint64_t staging_bytes, uint32_t num_staging, uint32_t ids_capacity, uint64_t host_cache_bytes)
        : dev_(device),
          staging_bytes_(staging_bytes),
          ids_capacity_(ids_capacity),
          cache_(dev_, host_cache_bytes, stats_),
          arena_(ids_capacity) {
        if (staging_bytes == 0 || num_staging == 0 || ids_capacity == 0)
            misuse("staging_bytes, num_staging and ids_capacity must be positive");
        // A failure part-way leaves only what close() knows how to free.
        try {
            copy_ = dev_.stream_create();
            have_copy_ = true;
            slots_.resize(num_staging);
            caller_slots_.resize(num_staging);
            for (Slot& slot : slots_) make_events(slot);
            for (Slot& slot : caller_slots_) make_events(slot);
            ids_pinned_ = static_cast<uint32_t*>(dev_.host_alloc(uint64_t(ids_capacity) * sizeof(uint32_t)));
            if (ids_pinned_ == nullptr) throw std::runtime_error("cannot pin the block-id ring");
            ids_device_ = static_cast<uint32_t*>(dev_.device_alloc(uint64_t(ids_capacity) * sizeof(uint32_t)));
        } catch (...) {
            close();
            throw;
        }
    }

    ~SwapEngine() { close(); }
    SwapEngine(const SwapEngine&) = delete;
    SwapEngine& operator=(const SwapEngine&) = delete;

    Dev& device() { return dev_; }
    void poison() { broken_ = true; }

    // Waits for every transfer and both streams, then frees everything; returns the first
    // error met on the way (the rest is freed regardless).
    std::string close() {
        if (closed_) return close_error_;
        closed_ = true;
        dev_.prepare_teardown();
        // Some transfers end on caller streams, which only their events can wait for.
        for (auto& entry : tickets_)
            if (!entry.second->finished) quietly([&] { dev_.event_sync(entry.second->done); });
        if (have_compute_) quietly([&] { dev_.stream_sync(compute_); });
        if (have_copy_) quietly([&] { dev_.stream_sync(copy_); });
        for (auto& entry : tickets_) quietly([&] { dev_.event_destroy(entry.second->done); });
        tickets_.clear();
        for (Event event : events_) quietly([&] { dev_.event_destroy(event); });
        events_.clear();
        for (Slot& slot : slots_)
            if (slot.staging != nullptr) quietly([&] { dev_.device_free(slot.staging); });
        slots_.clear();
        caller_slots_.clear();
        if (ids_device_ != nullptr) quietly([&] { dev_.device_free(ids_device_); });
        if (ids_pinned_ != nullptr) quietly([&] { dev_.host_free(ids_pinned_); });
        cache_.free_everything([&](auto&& step) { quietly(step); });
        if (have_copy_) quietly([&] { dev_.stream_destroy(copy_); });
        if (have_compute_) quietly([&] { dev_.stream_destroy(compute_); });
        return close_error_;
    }

    lt_stats stats() const {
        lt_stats snapshot = stats_;
        snapshot.host_bytes_held = cache_.held();
        return snapshot;
    }

    void prepare_staging() {
        healthy();
        compute();
        for (Slot& slot : slots_)
            if (slot.staging == nullptr) slot.staging = dev_.device_alloc(staging_bytes_);
    }

    void* host_alloc(uint64_t bytes) {
        healthy();
        return cache_.acquire(bytes);
    }

    void host_free(void* pointer) {
        healthy();
        cache_.give_back(pointer);
    }

    // Staged transfers: count blocks of block_bytes, in the order of ids, between the pool and
    // one contiguous host buffer.
    Ticket* staged(Direction direction, uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, uint8_t* host) {
        check_blocks(pool, block_bytes, ids, count, host);
        if (!eight_byte_words(pool, block_bytes) || !eight_byte_words(host, block_bytes))
            misuse("pool and host must be 8-byte aligned and block_bytes a multiple of 8");
        if (block_bytes > staging_bytes_) misuse("one block is larger than a staging buffer");
        if (count > ids_capacity_) misuse("transfer has more blocks than ids_capacity");
        const uint64_t per_segment = std::min<uint64_t>(staging_bytes_ / block_bytes, kMaxSegmentBlocks);
        if (!dev_.launch_fits(block_bytes, per_segment)) misuse("a staging buffer of these blocks is too many chunks for one kernel launch");
        prepare_staging();
        Ticket* ticket = new_ticket();
        const uint32_t* device_ids = nullptr;
        if (count) {
            // A transfer whose ids never reached the device was never started: its ticket goes
            // (it was not handed out), so it neither lingers nor counts as a transfer.
            try {
                device_ids = upload_ids(ids, count, ticket);
            } catch (...) {
                if (!ticket->owns_ids) drop_ticket(ticket);
                throw;
            }
        }
        const bool out = direction == Direction::ToHost;
        Stream fill_on = out ? compute_ : copy_;
        Stream drain_on = out ? copy_ : compute_;
        for (uint64_t first = 0; first < count; first += per_segment) {
            const uint32_t blocks = uint32_t(std::min<uint64_t>(per_segment, count - first));
            const uint64_t bytes = uint64_t(blocks) * block_bytes;
            uint8_t* staging = static_cast<uint8_t*>(slots_[turn_].staging);
            uint8_t* segment_host = host + first * block_bytes;
            Slot& slot = slots_[turn_];
            turn_ = (turn_ + 1) % uint32_t(slots_.size());

            wait(fill_on, slot.released);
            if (out) launch_gather(pool, device_ids + first, staging, block_bytes, blocks);
            else to_device(staging, segment_host, bytes);
            dev_.event_record(slot.filled, fill_on);

            wait(drain_on, slot.filled);
            if (out) to_host(segment_host, staging, bytes);
            else launch_scatter(pool, device_ids + first, staging, block_bytes, blocks);
            dev_.event_record(slot.released, drain_on);
        }
        dev_.event_record(ticket->done, drain_on);
        return ticket;
    }

    // One copy per block on the copy stream, no staging: the reference's measured baseline.
    Ticket* per_block(Direction direction, uint8_t* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, uint8_t* host) {
        check_blocks(pool, block_bytes, ids, count, host);
        Ticket* ticket = new_ticket();
        for (uint32_t i = 0; i < count; ++i) {
            uint8_t* block = pool + uint64_t(ids[i]) * block_bytes;
            uint8_t* record = host + uint64_t(i) * block_bytes;
            if (direction == Direction::ToHost) to_host(record, block, block_bytes);
            else to_device(block, record, block_bytes);
        }
        dev_.event_record(ticket->done, copy_);
        return ticket;
    }

    // Caller-owned staging (the FP8 path): the caller's kernels and the engine's copies meet
    // at the caller slots' events.
    void caller_wait(void* stream, uint32_t slot, int which) {
        healthy();
        wait(caller_stream(stream), caller_event(slot, which));
    }

    void caller_record(void* stream, uint32_t slot, int which) {
        healthy();
        dev_.event_record(caller_event(slot, which), caller_stream(stream));
    }

    void caller_copy(Direction direction, void* staging, uint8_t* host, uint64_t bytes, uint32_t slot) {
        healthy();
        Event filled = caller_event(slot, LT_SLOT_FILLED);
        Event released = caller_event(slot, LT_SLOT_RELEASED);
        if (staging == nullptr || host == nullptr || bytes == 0) misuse("null staging or host, or zero bytes");
        if (direction == Direction::ToHost) {
            wait(copy_, filled);
            to_host(host, staging, bytes);
            dev_.event_record(released, copy_);
        } else {
            wait(copy_, released);
            to_device(staging, host, bytes);
            dev_.event_record(filled, copy_);
        }
    }

    Ticket* caller_finish(void* stream) {
        healthy();
        Stream on = stream == nullptr ? copy_ : caller_stream(stream);
        Ticket* ticket = new_ticket();
        dev_.event_record(ticket->done, on);
        return ticket;
    }

    bool poll(Ticket* ticket) {
        live(ticket);
        if (!ticket->finished) ticket->finished = dev_.event_query(ticket->done);
        if (ticket->finished) collect();
        return ticket->finished;
    }

    void wait_for(Ticket* ticket) {
        live(ticket);
        if (!ticket->finished) {
            dev_.event_sync(ticket->done);
            ticket->finished = true;
        }
        collect();
    }

    void release(Ticket* ticket) {
        live(ticket);
        if (!poll(ticket)) misuse("transfer is still in flight");
        ticket->released = true;
        collect();
    }

   private:
    void make_events(Slot& slot) {
        slot.filled = dev_.event_create();
        events_.push_back(slot.filled);
        slot.released = dev_.event_create();
        events_.push_back(slot.released);
    }

    Stream compute() {
        if (!have_compute_) {
            compute_ = dev_.stream_create();
            have_compute_ = true;
        }
        return compute_;
    }

    void healthy() const {
        if (broken_) throw std::runtime_error("engine refused work after an earlier device failure");
    }

    void check_blocks(const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const void* host) {
        healthy();
        if (pool == nullptr || host == nullptr || block_bytes == 0 || (count != 0 && ids == nullptr))
            misuse("null pool, host or ids, or zero block_bytes");
        dev_.check_pool(pool);
    }

    // A null handle is the legacy default stream, which synchronizes with every other stream
    // and would silently serialize the copy stream behind the caller's work.
    static Stream caller_stream(void* stream) {
        if (stream == nullptr) misuse("null stream");
        return Dev::stream_from_handle(stream);
    }

    Event caller_event(uint32_t slot, int which) {
        if (slot >= caller_slots_.size() || (which != LT_SLOT_FILLED && which != LT_SLOT_RELEASED)) misuse("bad slot or event");
        return which == LT_SLOT_FILLED ? caller_slots_[slot].filled : caller_slots_[slot].released;
    }

    void wait(Stream stream, Event event) {
        dev_.stream_wait(stream, event);
        stats_.stream_waits++;
    }

    void to_host(void* dst, const void* src, uint64_t bytes) {
        dev_.memcpy_to_host(copy_, dst, src, bytes);
        stats_.memcpys++;
        stats_.bytes_to_host += bytes;
    }

    void to_device(void* dst, const void* src, uint64_t bytes) {
        dev_.memcpy_to_device(copy_, dst, src, bytes);
        stats_.memcpys++;
        stats_.bytes_to_device += bytes;
    }

    void launch_gather(const uint8_t* pool, const uint32_t* ids, uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        dev_.launch_gather(compute_, pool, ids, staging, block_bytes, blocks);
        stats_.kernels++;
    }

    void launch_scatter(uint8_t* pool, const uint32_t* ids, const uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        dev_.launch_scatter(compute_, pool, ids, staging, block_bytes, blocks);
        stats_.kernels++;
    }

    // The new ticket's event is recorded by the caller before anything looks at tickets
    // again: an event that was never recorded reads as complete.
    Ticket* new_ticket() {
        auto ticket = std::make_unique<Ticket>();
        ticket->done = dev_.event_create();
        Ticket* raw = ticket.get();
        tickets_.emplace(raw, std::move(ticket));
        stats_.transfers++;
        return raw;
    }

    void drop_ticket(Ticket* ticket) {
        quietly([&] { dev_.event_destroy(ticket->done); });
        tickets_.erase(ticket);
        stats_.transfers--;
    }

    void live(Ticket* ticket) const {
        const auto found = tickets_.find(ticket);
        if (found == tickets_.end() || found->second->released) misuse("not a live transfer of this engine");
    }

    // Copies the ids into the pinned ring and uploads them on the compute stream ahead of the
    // kernels that read them. From pinned memory the upload stays asynchronous; a pageable
    // source would synchronize the stream first. When the ring is full, the oldest transfer
    // holding ids is waited for: only a very large backlog gets there.
    const uint32_t* upload_ids(const uint32_t* ids, uint32_t count, Ticket* owner) {
        int64_t at;
        while ((at = arena_.claim(count, owner)) < 0) {
            if (arena_.empty()) throw std::logic_error("id ring is full with nothing in flight");
            wait_for(const_cast<Ticket*>(static_cast<const Ticket*>(arena_.oldest_owner())));
        }
        owner->owns_ids = true;
        memcpy(ids_pinned_ + at, ids, uint64_t(count) * sizeof(uint32_t));
        dev_.memcpy_to_device(compute_, ids_device_ + at, ids_pinned_ + at, uint64_t(count) * sizeof(uint32_t));
        stats_.ids_uploads++;
        return ids_device_ + at;
    }

    // Returns id spans of finished transfers, oldest first (a span waits for every older one),
    // then frees tickets that are released and hold no span.
    void collect() {
        while (!arena_.empty()) {
            Ticket* oldest = const_cast<Ticket*>(static_cast<const Ticket*>(arena_.oldest_owner()));
            if (!oldest->finished && !(oldest->finished = dev_.event_query(oldest->done))) break;
            oldest->owns_ids = false;
            arena_.pop_oldest();
        }
        for (auto it = tickets_.begin(); it != tickets_.end();) {
            if (it->second->released && !it->second->owns_ids) {
                dev_.event_destroy(it->second->done);
                it = tickets_.erase(it);
            } else {
                ++it;
            }
        }
    }

    template <class Step>
    void quietly(Step&& step) {
        try {
            step();
        } catch (const std::exception& error) {
            if (close_error_.empty()) close_error_ = error.what();
        }
    }

    Dev dev_;
    uint64_t staging_bytes_;
    uint32_t ids_capacity_;
    lt_stats stats_{};
    HostCache<Dev> cache_;
    IdArena arena_;

    Stream copy_{};
    Stream compute_{};
    bool have_copy_ = false;
    bool have_compute_ = false;
    std::vector<Slot> slots_;
    std::vector<Slot> caller_slots_;
    std::vector<Event> events_;
    uint32_t turn_ = 0;
    uint32_t* ids_pinned_ = nullptr;
    uint32_t* ids_device_ = nullptr;
    std::unordered_map<Ticket*, std::unique_ptr<Ticket>> tickets_;

    bool broken_ = false;
    bool closed_ = false;
    std::string close_error_;
};

}  // namespace lt

// ---- C exports ---------------------------------------------------------------------------
// Include this header once per flavour, after defining `Device`.

struct lt_engine {
    lt::SwapEngine<Device> core;
    lt_engine(int device, uint64_t staging, uint32_t slots, uint32_t ids, uint64_t cache) : core(device, staging, slots, ids, cache) {}
};

#define LT_EXPORT extern "C" __attribute__((visibility("default")))

namespace lt {

using EngineTicket = SwapEngine<Device>::Ticket;

// The status of the exception being handled, its text kept in last_error: a Fault carries its
// own code; a device back end's refusal of an argument (std::invalid_argument: a foreign pool,
// a device index that does not exist) is LT_ERR_INVALID; anything else is LT_ERR_DEVICE.
// Called only from inside a catch block.
inline int status_of_current_exception() {
    try {
        throw;
    } catch (const Fault& fault) {
        last_error = fault.what();
        return fault.code;
    } catch (const std::invalid_argument& refusal) {
        last_error = refusal.what();
        return LT_ERR_INVALID;
    } catch (const std::exception& failure) {
        last_error = failure.what();
        return LT_ERR_DEVICE;
    } catch (...) {
        last_error = "unknown failure";
        return LT_ERR_DEVICE;
    }
}

// Runs one call on an engine (its device made current first) and returns its status. After a
// device failure the engine refuses all further work: one can leave half a transfer enqueued.
template <class Call>
int on_engine(lt_engine* engine, Call&& call) {
    if (engine == nullptr) {
        last_error = "null engine";
        return LT_ERR_INVALID;
    }
    try {
        engine->core.device().activate();
        call(engine->core);
        return LT_OK;
    } catch (...) {
        const int status = status_of_current_exception();
        if (status == LT_ERR_DEVICE) engine->core.poison();
        return status;
    }
}

inline int refused(const char* text) {
    last_error = text;
    return LT_ERR_INVALID;
}

inline lt_transfer* handle_of(EngineTicket* ticket) { return reinterpret_cast<lt_transfer*>(ticket); }
inline EngineTicket* ticket_of(lt_transfer* handle) { return reinterpret_cast<EngineTicket*>(handle); }

template <class Start>
int start_transfer(lt_engine* engine, lt_transfer** out, Start&& start) {
    if (out == nullptr) return refused("null out pointer");
    return on_engine(engine, [&](SwapEngine<Device>& core) { *out = handle_of(start(core)); });
}

}  // namespace lt

LT_EXPORT int lt_abi_version(void) { return LT_ABI_VERSION; }
LT_EXPORT const char* lt_flavor(void) { return Device::flavor(); }
LT_EXPORT const char* lt_last_error(void) { return lt::last_error.c_str(); }

LT_EXPORT int lt_create(int device, uint64_t staging_bytes, uint32_t num_staging, uint32_t ids_capacity, uint64_t host_cache_bytes,
                        lt_engine** out) {
    if (out == nullptr) return lt::refused("null out pointer");
    try {
        *out = new lt_engine(device, staging_bytes, num_staging, ids_capacity, host_cache_bytes);
        return LT_OK;
    } catch (...) {
        return lt::status_of_current_exception();
    }
}

// Always frees the engine. Teardown goes on past a failure (the device cannot be made
// current, a stream cannot be drained); the first failure is the one reported.
LT_EXPORT int lt_destroy(lt_engine* engine) {
    if (engine == nullptr) return LT_OK;
    std::unique_ptr<lt_engine> owned(engine);
    std::vector<std::string> failures;
    try {
        owned->core.device().activate();
    } catch (const std::exception& failure) {
        failures.emplace_back(failure.what());
    }
    if (std::string closing = owned->core.close(); !closing.empty()) failures.push_back(std::move(closing));
    owned.reset();
    if (failures.empty()) return LT_OK;
    lt::last_error = failures.front();
    return LT_ERR_DEVICE;
}

LT_EXPORT int lt_prepare_staging(lt_engine* engine) {
    return lt::on_engine(engine, [](auto& core) { core.prepare_staging(); });
}

LT_EXPORT int lt_get_stats(lt_engine* engine, lt_stats* out) {
    if (engine == nullptr || out == nullptr) return lt::refused("null engine or out pointer");
    *out = engine->core.stats();
    return LT_OK;
}

LT_EXPORT int lt_host_alloc(lt_engine* engine, uint64_t bytes, void** out) {
    if (out == nullptr) return lt::refused("null out pointer");
    return lt::on_engine(engine, [&](auto& core) { *out = core.host_alloc(bytes); });
}

LT_EXPORT int lt_host_free(lt_engine* engine, void* pointer) {
    return lt::on_engine(engine, [&](auto& core) { core.host_free(pointer); });
}

LT_EXPORT int lt_out_gather(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, void* host,
                            lt_transfer** out) {
    return lt::start_transfer(engine, out, [&](auto& core) {
        return core.staged(lt::Direction::ToHost, static_cast<uint8_t*>(const_cast<void*>(pool)), block_bytes, ids, count,
                           static_cast<uint8_t*>(host));
    });
}

LT_EXPORT int lt_in_scatter(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const void* host,
                            lt_transfer** out) {
    return lt::start_transfer(engine, out, [&](auto& core) {
        return core.staged(lt::Direction::ToDevice, static_cast<uint8_t*>(pool), block_bytes, ids, count,
                           static_cast<uint8_t*>(const_cast<void*>(host)));
    });
}

LT_EXPORT int lt_out_per_block(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, void* host,
                               lt_transfer** out) {
    return lt::start_transfer(engine, out, [&](auto& core) {
        return core.per_block(lt::Direction::ToHost, static_cast<uint8_t*>(const_cast<void*>(pool)), block_bytes, ids, count,
                              static_cast<uint8_t*>(host));
    });
}

LT_EXPORT int lt_in_per_block(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count, const void* host,
                              lt_transfer** out) {
    return lt::start_transfer(engine, out, [&](auto& core) {
        return core.per_block(lt::Direction::ToDevice, static_cast<uint8_t*>(pool), block_bytes, ids, count,
                              static_cast<uint8_t*>(const_cast<void*>(host)));
    });
}

LT_EXPORT int lt_ext_wait(lt_engine* engine, void* stream, uint32_t slot, int which) {
    return lt::on_engine(engine, [&](auto& core) { core.caller_wait(stream, slot, which); });
}

LT_EXPORT int lt_ext_record(lt_engine* engine, void* stream, uint32_t slot, int which) {
    return lt::on_engine(engine, [&](auto& core) { core.caller_record(stream, slot, which); });
}

LT_EXPORT int lt_ext_copy_out(lt_engine* engine, const void* staging, void* host, uint64_t bytes, uint32_t slot) {
    return lt::on_engine(engine, [&](auto& core) {
        core.caller_copy(lt::Direction::ToHost, const_cast<void*>(staging), static_cast<uint8_t*>(host), bytes, slot);
    });
}

LT_EXPORT int lt_ext_copy_in(lt_engine* engine, void* staging, const void* host, uint64_t bytes, uint32_t slot) {
    return lt::on_engine(engine, [&](auto& core) {
        core.caller_copy(lt::Direction::ToDevice, staging, static_cast<uint8_t*>(const_cast<void*>(host)), bytes, slot);
    });
}

LT_EXPORT int lt_ext_finish(lt_engine* engine, void* stream, lt_transfer** out) {
    return lt::start_transfer(engine, out, [&](auto& core) { return core.caller_finish(stream); });
}

LT_EXPORT int lt_poll(lt_engine* engine, lt_transfer* transfer, int* done) {
    if (done == nullptr) return lt::refused("null done pointer");
    return lt::on_engine(engine, [&](auto& core) { *done = core.poll(lt::ticket_of(transfer)) ? 1 : 0; });
}

LT_EXPORT int lt_wait(lt_engine* engine, lt_transfer* transfer) {
    return lt::on_engine(engine, [&](auto& core) { core.wait_for(lt::ticket_of(transfer)); });
}

LT_EXPORT int lt_release(lt_engine* engine, lt_transfer* transfer) {
    return lt::on_engine(engine, [&](auto& core) { core.release(lt::ticket_of(transfer)); });
}

#endif  // LAYOVER_AMD_SWAP_ENGINE_H
