// Host-side pieces shared by the C ABI's translation units (kernels.hip, prefill.hip): the
// error plumbing behind lk_last_error, argument checks, and the pool and device facts both use.
#ifndef LAYOVER_AMD_HOST_COMMON_H
#define LAYOVER_AMD_HOST_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

#include "layover_kernels.h"

namespace lk {

// The calling thread's last error message (lk_last_error), defined in kernels.hip.
extern thread_local std::string last_error;

struct Invalid : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

template <class Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        const hipError_t status = hipGetLastError();
        if (status != hipSuccess) {
            last_error = std::string("kernel launch failed: ") + hipGetErrorName(status) + ": " + hipGetErrorString(status);
            return LK_ERR_DEVICE;
        }
        return LK_OK;
    } catch (const std::invalid_argument& error) {
        last_error = error.what();
        return LK_ERR_INVALID;
    } catch (const std::exception& error) {
        last_error = error.what();
        return LK_ERR_DEVICE;
    }
}

inline bool aligned(const void* pointer, uintptr_t to) { return (reinterpret_cast<uintptr_t>(pointer) % to) == 0; }

inline void require(bool condition, const char* message) {
    if (!condition) throw Invalid(message);
}

// Bytes of one pool block of this shape (all layers, K and V; FP8 records with their shifts).
uint64_t pool_block_bytes(const lk_decode_shape& s);
// CUs of the current device, cached per device; 256 (MI355X) when no device answers.
uint32_t compute_units();

}  // namespace lk

#endif  // LAYOVER_AMD_HOST_COMMON_H
