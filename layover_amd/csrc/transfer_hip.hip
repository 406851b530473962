// The HIP flavour of include/layover_transfer.h for MI355X (gfx950). Replaces the reference's
// native/transfer_cuda.cu: the swap engine (swap_engine.h) over HIP streams, events, copies to
// and from pinned memory, and the gather and scatter kernels of block_copy.h.
//
// Both directions of a copy are hipMemcpyAsync between device memory and pinned host memory.
// Copies to the device run on an SDMA engine; copies to the host run as the runtime's blit
// kernel, which measured faster on MI355X than handing them to an SDMA engine through the HSA
// runtime (a 2,048-block FP8 swap-out beside decode: 43.4 ms against 45.1 ms).
//
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <stdexcept>
#include <string>

#include "block_copy.h"
#include "layover_transfer.h"

namespace lt {

class HipDevice {
   public:
    using Stream = hipStream_t;
    using Event = hipEvent_t;

    static const char* flavor() { return "hip"; }
    static Stream stream_from_handle(void* handle) { return static_cast<Stream>(handle); }

    explicit HipDevice(int device) : device_(device) {
        int count = 0;
        check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        if (device < 0 || device >= count)
            throw std::invalid_argument("device " + std::to_string(device) + " does not exist (" + std::to_string(count) + " visible)");
        activate();
    }

    HipDevice(const HipDevice&) = delete;
    HipDevice& operator=(const HipDevice&) = delete;

    // The scheduler may call from any thread; the current device is per thread.
    void activate() { check(hipSetDevice(device_), "hipSetDevice"); }

    void prepare_teardown() {}

    // A kernel given host memory or another device's memory as the pool would fault the GPU.
    void check_pool(const void* pool) {
        hipPointerAttribute_t attributes{};
        const hipError_t status = hipPointerGetAttributes(&attributes, pool);
        if (status != hipSuccess) (void)hipGetLastError();  // unknown to HIP: plain host memory
        if (status != hipSuccess || attributes.type != hipMemoryTypeDevice || attributes.device != device_) {
            throw std::invalid_argument("pool is not memory of HIP device " + std::to_string(device_) +
                                        ": it is host memory, another device's, or unknown to this HIP runtime");
        }
    }

    void* device_alloc(uint64_t bytes) {
        void* pointer = nullptr;
        check(hipMalloc(&pointer, bytes), "hipMalloc");
        return pointer;
    }
    void device_free(void* pointer) { check(hipFree(pointer), "hipFree"); }

    // Null when the host is out of memory, which the engine survives.
    void* host_alloc(uint64_t bytes) {
        void* pointer = nullptr;
        const hipError_t status = hipHostMalloc(&pointer, bytes, hipHostMallocDefault);
        if (status == hipErrorOutOfMemory || status == hipErrorMemoryAllocation) {
            (void)hipGetLastError();
            return nullptr;
        }
        check(status, "hipHostMalloc");
        return pointer;
    }
    void host_free(void* pointer) { check(hipHostFree(pointer), "hipHostFree"); }

    // Non-blocking, default priority: torch's null stream must not serialize against the copy
    // stream, or decode would wait for every transfer in flight.
    Stream stream_create() {
        Stream stream = nullptr;
        check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        return stream;
    }
    void stream_sync(Stream stream) { check(hipStreamSynchronize(stream), "hipStreamSynchronize"); }
    void stream_destroy(Stream stream) { check(hipStreamDestroy(stream), "hipStreamDestroy"); }

    Event event_create() {
        Event event = nullptr;
        check(hipEventCreateWithFlags(&event, hipEventDisableTiming), "hipEventCreateWithFlags");
        return event;
    }
    void event_destroy(Event event) { check(hipEventDestroy(event), "hipEventDestroy"); }
    void event_record(Event event, Stream stream) { check(hipEventRecord(event, stream), "hipEventRecord"); }
    void stream_wait(Stream stream, Event event) { check(hipStreamWaitEvent(stream, event, 0), "hipStreamWaitEvent"); }

    bool event_query(Event event) {
        const hipError_t status = hipEventQuery(event);
        if (status == hipErrorNotReady) return false;
        check(status, "hipEventQuery");
        return true;
    }
    void event_sync(Event event) {
        check(hipEventSynchronize(event), "hipEventSynchronize");
    }

    void memcpy_to_host(Stream stream, void* dst, const void* src, uint64_t bytes) {
        check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(device to host)");
    }
    void memcpy_to_device(Stream stream, void* dst, const void* src, uint64_t bytes) {
        check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(host to device)");
    }

    bool launch_fits(uint64_t block_bytes, uint64_t blocks) const { return blockcopy::launch_fits(block_bytes, blocks); }

    void launch_gather(Stream stream, const uint8_t* pool, const uint32_t* ids, uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        check(blockcopy::launch_gather(stream, pool, ids, staging, block_bytes, blocks), "launch gather_blocks");
    }

    void launch_scatter(Stream stream, uint8_t* pool, const uint32_t* ids, const uint8_t* staging, uint64_t block_bytes, uint32_t blocks) {
        check(blockcopy::launch_scatter(stream, pool, ids, staging, block_bytes, blocks), "launch scatter_blocks");
    }

   private:
    static void check(hipError_t status, const char* call) {
        if (status != hipSuccess) throw std::runtime_error(std::string(call) + ": " + hipGetErrorName(status) + ": " + hipGetErrorString(status));
    }

    int device_;
};

}  // namespace lt

using Device = lt::HipDevice;

#include "swap_engine.h"

static int host_only(const char* name) {
    lt::last_error = std::string(name) + " exists only in the host flavour";
    return LT_ERR_UNSUPPORTED;
}

LT_EXPORT int lt_host_stream(lt_engine*, void**) { return host_only("lt_host_stream"); }
LT_EXPORT int lt_host_call(lt_engine*, void*, lt_host_kernel, void*) { return host_only("lt_host_call"); }
LT_EXPORT int lt_host_set_paused(lt_engine*, int) { return host_only("lt_host_set_paused"); }
LT_EXPORT int lt_host_set_copy_delay_us(lt_engine*, uint32_t) { return host_only("lt_host_set_copy_delay_us"); }
LT_EXPORT int lt_host_set_pin_limit(lt_engine*, uint64_t) { return host_only("lt_host_set_pin_limit"); }

