// libhmx core: error reporting, ABI version, the device check and the
// per-thread timing events of hmx_time_launches.
#include <string.h>

#include <string>

#include "hmx_internal.hpp"

namespace hmx {

namespace {
thread_local char g_error[1024] = {0};
thread_local LaunchEvents g_events = {nullptr, nullptr};
}

LaunchEvents& launch_events() { return g_events; }

int set_error(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return status;
}

void clear_error() { g_error[0] = 0; }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(HMX_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  return HMX_OK;
}

}  // namespace hmx

extern "C" {

const char* hmx_last_error(void) { return hmx::g_error; }

int hmx_abi_version(void) { return HMX_ABI_VERSION; }

int hmx_time_launches(void* start_event, void* stop_event) {
  hmx::g_events.start = (hipEvent_t)start_event;
  hmx::g_events.stop = (hipEvent_t)stop_event;
  return HMX_OK;
}

int hmx_device_check(int* compute_units) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess)
    return hmx::set_error(HMX_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(err));
  hipDeviceProp_t prop;
  err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess)
    return hmx::set_error(HMX_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(err));
  if (compute_units) *compute_units = prop.multiProcessorCount;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return hmx::set_error(HMX_ERR_UNSUPPORTED,
                          "libhmx is built for gfx950 (MI355X); device %d is %s",
                          device, prop.gcnArchName);
  return HMX_OK;
}

}  // extern "C"
