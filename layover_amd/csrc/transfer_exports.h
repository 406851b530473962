// The C exports of include/layover_transfer.h over Engine<Device>. Include once per flavour,
// after defining `Device`. Error mapping follows the reference (transfer_core.h:581-603):
// std::invalid_argument -> LT_ERR_INVALID, OutOfHostMemory -> LT_ERR_NOMEM, anything else ->
// LT_ERR_DEVICE, which also marks the engine failed for good.
#ifndef LAYOVER_AMD_TRANSFER_EXPORTS_H
#define LAYOVER_AMD_TRANSFER_EXPORTS_H

#include "transfer_engine.h"

struct lt_engine {
    lt::Engine<Device> impl;
    lt_engine(int device, uint64_t staging, uint32_t slots, uint32_t ids, uint64_t cache)
        : impl(device, staging, slots, ids, cache) {}
};

#define LT_EXPORT extern "C" __attribute__((visibility("default")))

namespace lt {

using EngineTransfer = Engine<Device>::Transfer;

inline EngineTransfer* unwrap(lt_transfer* transfer) { return reinterpret_cast<EngineTransfer*>(transfer); }
inline lt_transfer* wrap(EngineTransfer* transfer) { return reinterpret_cast<lt_transfer*>(transfer); }

template <class Fn>
int guarded(lt_engine* engine, Fn&& fn) {
    if (engine == nullptr) {
        last_error = "null engine";
        return LT_ERR_INVALID;
    }
    try {
        engine->impl.device().activate();
        fn();
        return LT_OK;
    } catch (const std::invalid_argument& error) {
        last_error = error.what();
        return LT_ERR_INVALID;
    } catch (const OutOfHostMemory& error) {
        last_error = error.what();
        return LT_ERR_NOMEM;
    } catch (const std::exception& error) {
        last_error = error.what();
        engine->impl.mark_failed();
        return LT_ERR_DEVICE;
    }
}

inline int refuse_null(const void* out, const char* what) {
    last_error = std::string("null ") + what;
    return out == nullptr ? LT_ERR_INVALID : LT_OK;
}

}  // namespace lt

LT_EXPORT int lt_abi_version(void) { return LT_ABI_VERSION; }
LT_EXPORT const char* lt_flavor(void) { return Device::flavor(); }
LT_EXPORT const char* lt_last_error(void) { return lt::last_error.c_str(); }

LT_EXPORT int lt_create(int device, uint64_t staging_bytes, uint32_t num_staging, uint32_t ids_capacity,
                        uint64_t host_cache_bytes, lt_engine** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    try {
        *out = new lt_engine(device, staging_bytes, num_staging, ids_capacity, host_cache_bytes);
        return LT_OK;
    } catch (const std::invalid_argument& error) {
        lt::last_error = error.what();
        return LT_ERR_INVALID;
    } catch (const std::exception& error) {
        lt::last_error = error.what();
        return LT_ERR_DEVICE;
    }
}

LT_EXPORT int lt_destroy(lt_engine* engine) {
    if (engine == nullptr) return LT_OK;
    std::string problem;
    try {
        engine->impl.device().activate();
    } catch (const std::exception& error) {
        problem = error.what();
    }
    const std::string shutdown = engine->impl.shutdown();
    delete engine;
    if (problem.empty()) problem = shutdown;
    if (problem.empty()) return LT_OK;
    lt::last_error = problem;
    return LT_ERR_DEVICE;
}

LT_EXPORT int lt_prepare_staging(lt_engine* engine) {
    return lt::guarded(engine, [&] { engine->impl.prepare_staging(); });
}

LT_EXPORT int lt_get_stats(lt_engine* engine, lt_stats* out) {
    if (engine == nullptr || out == nullptr) return lt::refuse_null(nullptr, "engine or out pointer");
    *out = engine->impl.stats();
    return LT_OK;
}

LT_EXPORT int lt_host_alloc(lt_engine* engine, uint64_t bytes, void** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] { *out = engine->impl.host_alloc(bytes); });
}

LT_EXPORT int lt_host_free(lt_engine* engine, void* pointer) {
    return lt::guarded(engine, [&] { engine->impl.host_free(pointer); });
}

LT_EXPORT int lt_out_gather(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count,
                            void* host, lt_transfer** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] {
        *out = lt::wrap(engine->impl.out_gather(static_cast<const uint8_t*>(pool), block_bytes, ids, count, static_cast<uint8_t*>(host)));
    });
}

LT_EXPORT int lt_in_scatter(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count,
                            const void* host, lt_transfer** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] {
        *out = lt::wrap(engine->impl.in_scatter(static_cast<uint8_t*>(pool), block_bytes, ids, count, static_cast<const uint8_t*>(host)));
    });
}

LT_EXPORT int lt_out_per_block(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count,
                               void* host, lt_transfer** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] {
        *out = lt::wrap(engine->impl.out_per_block(static_cast<const uint8_t*>(pool), block_bytes, ids, count, static_cast<uint8_t*>(host)));
    });
}

LT_EXPORT int lt_in_per_block(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids, uint32_t count,
                              const void* host, lt_transfer** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] {
        *out = lt::wrap(engine->impl.in_per_block(static_cast<uint8_t*>(pool), block_bytes, ids, count, static_cast<const uint8_t*>(host)));
    });
}

LT_EXPORT int lt_ext_wait(lt_engine* engine, void* stream, uint32_t slot, int which) {
    return lt::guarded(engine, [&] { engine->impl.ext_wait(stream, slot, which); });
}

LT_EXPORT int lt_ext_record(lt_engine* engine, void* stream, uint32_t slot, int which) {
    return lt::guarded(engine, [&] { engine->impl.ext_record(stream, slot, which); });
}

LT_EXPORT int lt_ext_copy_out(lt_engine* engine, const void* staging, void* host, uint64_t bytes, uint32_t slot) {
    return lt::guarded(engine, [&] { engine->impl.ext_copy_out(staging, static_cast<uint8_t*>(host), bytes, slot); });
}

LT_EXPORT int lt_ext_copy_in(lt_engine* engine, void* staging, const void* host, uint64_t bytes, uint32_t slot) {
    return lt::guarded(engine, [&] { engine->impl.ext_copy_in(staging, static_cast<const uint8_t*>(host), bytes, slot); });
}

LT_EXPORT int lt_ext_finish(lt_engine* engine, void* stream, lt_transfer** out) {
    if (out == nullptr) return lt::refuse_null(out, "out pointer");
    return lt::guarded(engine, [&] { *out = lt::wrap(engine->impl.ext_finish(stream)); });
}

LT_EXPORT int lt_poll(lt_engine* engine, lt_transfer* transfer, int* done) {
    if (done == nullptr) return lt::refuse_null(done, "done pointer");
    return lt::guarded(engine, [&] { *done = engine->impl.poll(lt::unwrap(transfer)) ? 1 : 0; });
}

LT_EXPORT int lt_wait(lt_engine* engine, lt_transfer* transfer) {
    return lt::guarded(engine, [&] { engine->impl.wait_for(lt::unwrap(transfer)); });
}

LT_EXPORT int lt_release(lt_engine* engine, lt_transfer* transfer) {
    return lt::guarded(engine, [&] { engine->impl.release(lt::unwrap(transfer)); });
}

#endif  // LAYOVER_AMD_TRANSFER_EXPORTS_H
