// Host-side plumbing shared by libhmx's translation units: the per-thread
// error message, argument checks and launch-error capture.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "hmx.h"

namespace hmx {

// Records the calling thread's error message and returns `status`.
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// The HIP error of the last launch on this thread, as an hmx status.
int check_launch(const char* what);

// Timing events armed on this thread by hmx_time_launches (null when not).
struct LaunchEvents {
  hipEvent_t start;
  hipEvent_t stop;
};
LaunchEvents& launch_events();

// Enqueues kernel<<<grid, block, 0, stream>>>(args...), each argument
// converted to the kernel's parameter type. While timing events are armed on
// this thread the launch goes through hipExtLaunchKernelGGL instead: the first
// such launch records `start` as it begins and every one records `stop` as it
// ends.
template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                   Args... args) {
  LaunchEvents& ev = launch_events();
  if (ev.start == nullptr && ev.stop == nullptr) {
    kernel<<<grid, block, 0, stream>>>(static_cast<KArgs>(args)...);
    return;
  }
  hipEvent_t start = ev.start;
  ev.start = nullptr;
  hipExtLaunchKernelGGL<KArgs...>(kernel, grid, block, 0, stream, start, ev.stop, 0,
                                  static_cast<KArgs>(args)...);
}

// The shape of a device that launches are planned for: its compute units and
// XCDs (the chiplets workgroups are dealt to in turn, each with its own L2).
struct DeviceShape {
  int cus;
  int xcds;
};
// MI355X: 256 CUs in 8 XCDs. Plans made without a device use it.
constexpr DeviceShape kMi355x = {256, 8};

// The current device's shape, read from the runtime once per device and
// kept (a device's properties do not change while the process runs). With no
// device visible: kMi355x.
DeviceShape current_device_shape();

// Enqueues dst[c, r] = src[r, c] for 16-bit elements, src [rows, cols] with
// row stride ld, dst [cols, rows] contiguous (hmx_pack.hip).
void launch_transpose16(const void* src, void* dst, int64_t rows, int64_t cols, int64_t ld,
                        hipStream_t stream);

inline bool valid_dtype(int dtype) {
  return dtype == HMX_DTYPE_F32 || dtype == HMX_DTYPE_BF16;
}
inline int64_t dtype_bytes(int dtype) { return dtype == HMX_DTYPE_BF16 ? 2 : 4; }
inline bool valid_activation(int code) {
  return code >= HMX_EPI_IDENTITY && code <= HMX_EPI_PROGRAM;
}

// Checks the epilogue (activation code, program) of an entry point `what`
// and copies the program into `out` (zeroed when the code is not
// HMX_EPI_PROGRAM). Returns HMX_OK or the HMX_ERR_INVALID of a bad code or
// program: a null program, a count outside 1..HMX_PROGRAM_MAX, an unknown
// opcode, or a register past HMX_PROGRAM_REGS.
int check_epilogue(const char* what, int code, const hmx_program* program, hmx_program* out);
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace hmx

#define HMX_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::hmx::set_error(HMX_ERR_INVALID, __VA_ARGS__); \
  } while (0)
