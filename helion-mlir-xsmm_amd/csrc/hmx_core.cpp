// libhmx core: error reporting, ABI version, the device check and the
// per-thread timing events of hmx_time_launches.
#include <string.h>

#include <atomic>
#include <string>

#include "hmx_internal.hpp"

namespace hmx {

namespace {
thread_local char g_error[1024] = {0};
thread_local LaunchEvents g_events = {nullptr, nullptr};

// Device shapes read so far, by device index: (cus << 16) | xcds, 0 = not yet
// read. Written once per device with the same value from any thread.
constexpr int kMaxDevices = 64;
std::atomic<uint32_t> g_shapes[kMaxDevices];

DeviceShape query_shape(int device) {
  int cus = 0, xcds = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
    return kMi355x;
  if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device) != hipSuccess || xcds <= 0)
    xcds = 1;
  return DeviceShape{cus, xcds};
}
}  // namespace

LaunchEvents& launch_events() { return g_events; }

DeviceShape current_device_shape() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    (void)hipGetLastError();  // no device: not an error of the caller's next call
    return kMi355x;
  }
  if (device < 0 || device >= kMaxDevices) return query_shape(device);
  const uint32_t known = g_shapes[device].load(std::memory_order_relaxed);
  if (known != 0) return DeviceShape{(int)(known >> 16), (int)(known & 0xffff)};
  const DeviceShape d = query_shape(device);
  g_shapes[device].store(((uint32_t)d.cus << 16) | (uint32_t)(d.xcds & 0xffff), std::memory_order_relaxed);
  return d;
}

int set_error(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return status;
}

void clear_error() { g_error[0] = 0; }

int check_epilogue(const char* what, int code, const hmx_program* program, hmx_program* out) {
  *out = hmx_program{};
  if (!valid_activation(code)) return set_error(HMX_ERR_INVALID, "%s: unknown epilogue %d", what, code);
  if (code != HMX_EPI_PROGRAM) return HMX_OK;
  if (program == nullptr) return set_error(HMX_ERR_INVALID, "%s: epilogue program is null", what);
  if (program->count < 1 || program->count > HMX_PROGRAM_MAX)
    return set_error(HMX_ERR_INVALID, "%s: epilogue program of %d instructions (1..%d)", what, program->count,
                     HMX_PROGRAM_MAX);
  if (program->result < 0 || program->result >= HMX_PROGRAM_REGS)
    return set_error(HMX_ERR_INVALID, "%s: epilogue program result register %d", what, program->result);
  for (int i = 0; i < program->count; ++i) {
    const hmx_instr& in = program->code[i];
    if (in.op >= HMX_OP_COUNT)
      return set_error(HMX_ERR_INVALID, "%s: epilogue program instruction %d: unknown opcode %d", what, i, in.op);
    if (in.dst >= HMX_PROGRAM_REGS || in.a >= HMX_PROGRAM_REGS || in.b >= HMX_PROGRAM_REGS)
      return set_error(HMX_ERR_INVALID, "%s: epilogue program instruction %d: register past %d", what, i,
                       HMX_PROGRAM_REGS - 1);
  }
  *out = *program;
  return HMX_OK;
}

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
