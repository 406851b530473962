/*
 * layover_transfer.h: C ABI of the KV block transfer library, version 2.
 *
 * Drop-in for the reference's native/layover_transfer.h (ABI 2): the same 26 entry points,
 * the same argument meaning, error codes, slot-event numbering and ownership rules, so the
 * reference's ctypes binding (layover/kv/native.py:54-78) binds this library unchanged apart
 * from the flavour name. Flavours of this library:
 *   "host"  host threads stand in for device streams (tests, CPU baseline)
 *   "hip"   MI355X (gfx950): HIP streams and events, hipMemcpyAsync to and from pinned
 *           memory and hand-written gather and scatter kernels; replaces the reference's
 *           native/transfer_cuda.cu.
 *
 * Contract (reference native/layover_transfer.h:1-5, native/transfer_core.h:581-603):
 *   - one engine is driven by one thread; calls are not thread-safe;
 *   - every stream operation of a call is enqueued before the call returns;
 *   - LT_ERR_INVALID leaves the engine unchanged, LT_ERR_DEVICE is sticky (every later call
 *     fails), LT_ERR_NOMEM (lt_host_alloc only) leaves the engine usable;
 *   - the caller owns `pool` (device memory of the engine's device) and host buffers from
 *     lt_host_alloc until lt_host_free; the engine owns its streams, events, staging,
 *     id ring and pinned cache, all freed by lt_destroy after in-flight work finished.
 */
#ifndef LAYOVER_TRANSFER_H
#define LAYOVER_TRANSFER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LT_ABI_VERSION 2

/* layover_transfer.h:17-23 */
enum {
    LT_OK = 0,
    LT_ERR_INVALID = 1,
    LT_ERR_DEVICE = 2,
    LT_ERR_UNSUPPORTED = 3,
    LT_ERR_NOMEM = 4,
};

/* Per-slot events of caller-owned staging (layover_transfer.h:26). */
enum { LT_SLOT_FILLED = 0, LT_SLOT_RELEASED = 1 };

typedef struct lt_engine lt_engine;
typedef struct lt_transfer lt_transfer;

/* Counters, field for field as layover_transfer.h:31-46 (native.py:31-47 reads them). */
typedef struct {
    uint64_t kernels;           /* gather/scatter launches */
    uint64_t memcpys;           /* KV copies on the copy stream */
    uint64_t ids_uploads;       /* block-id uploads ahead of kernels */
    uint64_t stream_waits;
    uint64_t bytes_to_host;
    uint64_t bytes_to_device;
    uint64_t transfers;
    uint64_t host_bytes_live;   /* pinned bytes handed out and not yet returned */
    uint64_t host_bytes_held;   /* pinned bytes owned, cached ones included */
    uint64_t host_pins;         /* pin attempts the cache could not serve */
    uint64_t host_pin_bytes;
    uint64_t host_pin_ns;
    uint64_t host_pin_max_ns;
    uint64_t host_pin_failures; /* lt_host_alloc calls that ended in LT_ERR_NOMEM */
} lt_stats;

/* layover_transfer.h:48-51 */
int lt_abi_version(void);
const char* lt_flavor(void); /* "host" or "hip" */
const char* lt_last_error(void);

/* layover_transfer.h:53-63 */
int lt_create(int device, uint64_t staging_bytes, uint32_t num_staging, uint32_t ids_capacity,
              uint64_t host_cache_bytes, lt_engine** out);
int lt_destroy(lt_engine* engine);
int lt_prepare_staging(lt_engine* engine);
int lt_get_stats(lt_engine* engine, lt_stats* out);

/* layover_transfer.h:65-69: pinned host memory, cached by size class. */
int lt_host_alloc(lt_engine* engine, uint64_t bytes, void** out);
int lt_host_free(lt_engine* engine, void* pointer);

/* layover_transfer.h:71-76: gather `count` blocks of `block_bytes` in the order of `ids`
 * through staging to `host`, and the reverse. pool and host 8-byte aligned, block_bytes a
 * multiple of 8 and at most one staging buffer, count at most ids_capacity. */
int lt_out_gather(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids,
                  uint32_t count, void* host, lt_transfer** out);
int lt_in_scatter(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids,
                  uint32_t count, const void* host, lt_transfer** out);

/* layover_transfer.h:78-82: one copy per block, no staging; kept as the measured baseline. */
int lt_out_per_block(lt_engine* engine, const void* pool, uint64_t block_bytes, const uint32_t* ids,
                     uint32_t count, void* host, lt_transfer** out);
int lt_in_per_block(lt_engine* engine, void* pool, uint64_t block_bytes, const uint32_t* ids,
                    uint32_t count, const void* host, lt_transfer** out);

/* layover_transfer.h:84-96: caller-owned staging ordered against the copy stream.
 *   out: ext_wait(s, slot, RELEASED); kernel on s; ext_record(s, slot, FILLED);
 *        ext_copy_out(slot, ...); finally ext_finish(NULL)
 *   in:  ext_copy_in(slot, ...); ext_wait(s, slot, FILLED); kernel on s;
 *        ext_record(s, slot, RELEASED); finally ext_finish(s)
 * `stream` is a hipStream_t (a torch.cuda.Stream's cuda_stream) and is never null. */
int lt_ext_wait(lt_engine* engine, void* stream, uint32_t slot, int which);
int lt_ext_record(lt_engine* engine, void* stream, uint32_t slot, int which);
int lt_ext_copy_out(lt_engine* engine, const void* staging, void* host, uint64_t bytes, uint32_t slot);
int lt_ext_copy_in(lt_engine* engine, void* staging, const void* host, uint64_t bytes, uint32_t slot);
int lt_ext_finish(lt_engine* engine, void* stream, lt_transfer** out);

/* layover_transfer.h:98-102 */
int lt_poll(lt_engine* engine, lt_transfer* transfer, int* done);
int lt_wait(lt_engine* engine, lt_transfer* transfer);
int lt_release(lt_engine* engine, lt_transfer* transfer);

/* layover_transfer.h:104-112: host flavour only (others return LT_ERR_UNSUPPORTED). */
typedef int (*lt_host_kernel)(void* context);
int lt_host_stream(lt_engine* engine, void** out);
int lt_host_call(lt_engine* engine, void* stream, lt_host_kernel kernel, void* context);
int lt_host_set_paused(lt_engine* engine, int paused);
int lt_host_set_copy_delay_us(lt_engine* engine, uint32_t delay_us);
int lt_host_set_pin_limit(lt_engine* engine, uint64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* LAYOVER_TRANSFER_H */
