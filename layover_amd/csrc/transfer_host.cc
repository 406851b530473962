// The host flavour of include/layover_transfer.h: the swap engine over host threads
// (host_streams.h), plus the five controls only this flavour has (layover_transfer.h:104-112
// of the reference). Each control is one method of the host device, reached through the
// engine the handle names.
#include "host_streams.h"

using Device = lt::HostDevice;

#include "swap_engine.h"

namespace {

template <class Control>
int host_control(lt_engine* engine, Control&& control) {
    return lt::on_engine(engine, [&](lt::SwapEngine<Device>& core) { control(core.device()); });
}

}  // namespace

LT_EXPORT int lt_host_stream(lt_engine* engine, void** out) {
    if (out == nullptr) return lt::refused("null out pointer");
    return host_control(engine, [&](Device& device) { *out = device.caller_lane(); });
}

LT_EXPORT int lt_host_call(lt_engine* engine, void* stream, lt_host_kernel kernel, void* context) {
    if (stream == nullptr || kernel == nullptr) return lt::refused("null stream or kernel");
    return host_control(engine, [&](Device& device) { device.run_host_kernel(Device::stream_from_handle(stream), kernel, context); });
}

LT_EXPORT int lt_host_set_paused(lt_engine* engine, int paused) {
    return host_control(engine, [&](Device& device) { device.set_paused(paused != 0); });
}

LT_EXPORT int lt_host_set_copy_delay_us(lt_engine* engine, uint32_t delay_us) {
    return host_control(engine, [&](Device& device) { device.set_copy_delay_us(delay_us); });
}

LT_EXPORT int lt_host_set_pin_limit(lt_engine* engine, uint64_t bytes) {
    return host_control(engine, [&](Device& device) { device.set_pin_limit(bytes); });
}
