// Run-time compiled epilogues. A GEMM whose epilogue is a program (or a named
// activation the precompiled register epilogue does not carry) runs the
// 16x16x32 kernel with that epilogue compiled into its register epilogue:
// the kernel body (hmx_gemm_mi16.hpp) and the headers it needs are embedded
// in the library, a source that defines hmx_jit_epilogue as straight-line
// code is generated from the program, and hipRTC compiles it on first use
// (about half a second). Code objects are cached per device, kernel variant
// and epilogue. The interpreter (ACT_PROG) stays the path when run-time
// compilation is off (HMX_JIT=0) or fails.
//
// The generated code evaluates each instruction with the same formula as the
// interpreter (program_op with a constant opcode), so both give the same
// results.
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "hmx_gemm_common.hpp"
#include "hmx_rows_common.hpp"

// The headers of the run-time sources, embedded NUL-terminated (paths are
// relative to this file's directory, where the Makefile compiles it).
extern "C" const char hmx_jit_src_hmx_h[], hmx_jit_src_device[], hmx_jit_src_common[], hmx_jit_src_lds[],
    hmx_jit_src_mi16[], hmx_jit_src_rows[];
#if !defined(__HIP_DEVICE_COMPILE__)
#define HMX_EMBED(sym, path)                  \
  asm(".section .rodata\n"                    \
      ".p2align 4\n"                          \
      ".global " #sym "\n" #sym ":\n"         \
      ".incbin \"" path "\"\n"                \
      ".byte 0\n"                             \
      ".previous\n");
HMX_EMBED(hmx_jit_src_hmx_h, "../../include/hmx.h")
HMX_EMBED(hmx_jit_src_device, "hmx_device.hpp")
HMX_EMBED(hmx_jit_src_common, "hmx_gemm_common.hpp")
HMX_EMBED(hmx_jit_src_lds, "hmx_gemm_lds.hpp")
HMX_EMBED(hmx_jit_src_mi16, "hmx_gemm_mi16.hpp")
HMX_EMBED(hmx_jit_src_rows, "hmx_rows_common.hpp")
#undef HMX_EMBED
#endif

namespace hmx {
namespace {

struct JitStats {
  int64_t compiled = 0;
  int64_t failed = 0;
  int64_t launches = 0;
};

std::mutex g_jit_lock;
JitStats g_jit_stats;
// Set by JitCompileOff: this thread may not compile or load kernels.
thread_local bool t_compile_off = false;
// Compiled kernels by key; a null function marks a key whose compilation
// failed (it is not tried again).
std::map<std::string, hipFunction_t> g_jit_kernels;
std::string g_jit_last_log;

// A float constant as source text that reads back bit for bit.
std::string float_text(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  char buf[40];
  std::snprintf(buf, sizeof buf, "__uint_as_float(0x%08xu)", bits);
  return buf;
}

// hmx_jit_epilogue(x, extra) for an epilogue: a named activation code (and
// its argument), or the program's instructions in turn over registers r0
// (the value), r1 (the extra operand) and r2..r7 (zero).
std::string epilogue_source(int act, float act_arg, const hmx_program& prog) {
  std::string s = "namespace hmx {\n__device__ float hmx_jit_epilogue(float x, float extra) {\n";
  if (act != HMX_EPI_PROGRAM) {
    s += "  (void)extra;\n  return apply_activation(" + std::to_string(act) + ", x, " + float_text(act_arg) +
         ");\n}\n}  // namespace hmx\n";
    return s;
  }
  s += "  float r0 = x, r1 = extra, r2 = 0.f, r3 = 0.f, r4 = 0.f, r5 = 0.f, r6 = 0.f, r7 = 0.f;\n";
  for (int i = 0; i < prog.count; ++i) {
    const hmx_instr& in = prog.code[i];
    s += "  r" + std::to_string(in.dst) + " = program_op(" + std::to_string(in.op) + ", r" +
         std::to_string(in.a) + ", r" + std::to_string(in.b) + ", " + float_text(in.c0) + ", " +
         float_text(in.c1) + ");\n";
  }
  s += "  (void)r0; (void)r1; (void)r2; (void)r3; (void)r4; (void)r5; (void)r6; (void)r7;\n";
  s += "  return r" + std::to_string(prog.result) + ";\n}\n}  // namespace hmx\n";
  return s;
}

// The epilogue part of a compiled kernel's key.
std::string epilogue_key(int act, float act_arg, const hmx_program& prog) {
  uint32_t bits;
  std::memcpy(&bits, &act_arg, 4);
  std::string k = std::to_string(act) + "|" + std::to_string(bits);
  if (act == HMX_EPI_PROGRAM) {
    k += "|" + std::to_string(prog.count) + "," + std::to_string(prog.result);
    for (int i = 0; i < prog.count; ++i) {
      const hmx_instr& in = prog.code[i];
      uint32_t c0, c1;
      std::memcpy(&c0, &in.c0, 4);
      std::memcpy(&c1, &in.c1, 4);
      k += ";" + std::to_string(in.op) + "," + std::to_string(in.dst) + "," + std::to_string(in.a) + "," +
           std::to_string(in.b) + "," + std::to_string(c0) + "," + std::to_string(c1);
    }
  }
  return k;
}

// Compiles `source` for the current device and loads it; the kernel
// `hmx_jit_kernel`, or null (the log kept in g_jit_last_log). A HIP call that
// fails here leaves no error behind: the call goes on with the prebuilt
// kernels, and their launch check must not see this one's error.
hipFunction_t compile(const std::string& source, int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    (void)hipGetLastError();
    g_jit_last_log = "hipGetDeviceProperties failed";
    return nullptr;
  }
  const char* headers[] = {hmx_jit_src_hmx_h, hmx_jit_src_device, hmx_jit_src_common, hmx_jit_src_lds,
                           hmx_jit_src_mi16, hmx_jit_src_rows};
  const char* names[] = {"hmx.h", "hmx_device.hpp", "hmx_gemm_common.hpp", "hmx_gemm_lds.hpp",
                         "hmx_gemm_mi16.hpp", "hmx_rows_common.hpp"};
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source.c_str(), "hmx_jit.hip", 6, headers, names) != HIPRTC_SUCCESS) {
    g_jit_last_log = "hiprtcCreateProgram failed";
    return nullptr;
  }
  // The library's own flags: no packed f32 instructions, no contraction.
  const std::string arch = std::string("--offload-arch=") + prop.gcnArchName;
  const char* opts[] = {arch.c_str(), "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string log(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, &log[0]);
  hipFunction_t fn = nullptr;
  if (rc == HIPRTC_SUCCESS) {
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hipModule_t module = nullptr;
    // The module stays loaded for the process: its kernel is cached.
    if (hipModuleLoadData(&module, code.data()) == hipSuccess &&
        hipModuleGetFunction(&fn, module, "hmx_jit_kernel") != hipSuccess)
      fn = nullptr;
    if (!fn) {
      (void)hipGetLastError();
      log += "\nloading the code object failed";
    }
  } else {
    log = std::string(hiprtcGetErrorString(rc)) + " (" + arch + ")\n" + log + "\nsource:\n" + source;
  }
  hiprtcDestroyProgram(&prog);
  if (!fn) g_jit_last_log = log;
  return fn;
}

// The compiled kernel for `key` (compiling `source` on first use), or null
// when run-time compilation is off or failed, or the kernel is not compiled
// yet and this thread may not compile (JitCompileOff). Counts a launch when
// found.
hipFunction_t jit_function(const std::string& key, const std::string& source, int device) {
  std::lock_guard<std::mutex> guard(g_jit_lock);
  auto it = g_jit_kernels.find(key);
  if (it == g_jit_kernels.end()) {
    if (t_compile_off) return nullptr;
    hipFunction_t fn = compile(source, device);
    if (fn) ++g_jit_stats.compiled;
    else ++g_jit_stats.failed;
    it = g_jit_kernels.emplace(key, fn).first;
  }
  if (it->second) ++g_jit_stats.launches;
  return it->second;
}

// Enqueues `fn` on `stream` (through hipExtModuleLaunchKernel while timing
// events are armed on this thread, as launch() does for the library's own
// kernels). A launch the runtime refuses is remembered like a failed
// compilation (key `key` is not tried again), leaves no error behind and
// returns HMX_ERR_UNSUPPORTED: the call takes the prebuilt kernels.
int jit_launch(const std::string& key, hipFunction_t fn, dim3 grid, unsigned block, void** params,
               hipStream_t stream, const char* what) {
  LaunchEvents& ev = launch_events();
  hipError_t err;
  if (ev.start == nullptr && ev.stop == nullptr) {
    err = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block, 1, 1, 0, stream, params, nullptr);
  } else {
    // The step's first kernel records the start event: taken only by a
    // launch that happens.
    err = hipExtModuleLaunchKernel(fn, grid.x * block, grid.y, grid.z, block, 1, 1, 0, stream, params, nullptr,
                                   ev.start, ev.stop, 0);
    if (err == hipSuccess) ev.start = nullptr;
  }
  if (err == hipSuccess) return HMX_OK;
  (void)hipGetLastError();
  std::lock_guard<std::mutex> guard(g_jit_lock);
  g_jit_kernels[key] = nullptr;
  ++g_jit_stats.failed;
  g_jit_last_log = std::string(what) + ": run-time compiled kernel launch: " + hipGetErrorString(err);
  return HMX_ERR_UNSUPPORTED;
}

}  // namespace

JitCompileOff::JitCompileOff(bool on_) : was(t_compile_off), on(on_) {
  if (on) t_compile_off = true;
}
JitCompileOff::~JitCompileOff() {
  if (on) t_compile_off = was;
}

bool jit_enabled() {
  const char* e = getenv("HMX_JIT");
  return !(e && e[0] == '0');
}

int launch_mi16_jit(const GemmArgs& g, int lb, bool bf16, bool ragged, int bm, int bn, int nw, int stages,
                    dim3 grid, hipStream_t stream) {
  if (!jit_enabled()) return HMX_ERR_UNSUPPORTED;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return HMX_ERR_UNSUPPORTED;
  const std::string args = std::string(bf16 ? "true" : "false") + ", " + (ragged ? "true" : "false") + ", " +
                           std::to_string(bm) + ", " + std::to_string(bn) + ", " + std::to_string(nw) + ", " +
                           std::to_string(stages);
  const std::string key = std::to_string(device) + "|gemm|" + std::to_string(lb) + "," + args + "|" +
                          epilogue_key(g.act, g.act_arg, g.prog);
  const std::string source = "#include \"hmx_gemm_mi16.hpp\"\n" + epilogue_source(g.act, g.act_arg, g.prog) +
                             "extern \"C\" __global__ __launch_bounds__(" + std::to_string(nw * 64) +
                             ", 1) void hmx_jit_kernel(hmx::GemmArgs g) {\n  hmx::gemm_bf16_mi16_body<" +
                             std::to_string(lb) + ", hmx::ACT_JIT, " + args + ">(g);\n}\n";
  hipFunction_t fn = jit_function(key, source, device);
  if (!fn) return HMX_ERR_UNSUPPORTED;
  GemmArgs copy = g;
  void* params[] = {&copy};
  return jit_launch(key, fn, grid, (unsigned)nw * 64, params, stream, "gemm");
}

int launch_mi16_rounds_jit(const GemmArgs& head, const GemmArgs& rest, int lb, bool bf16, unsigned head_blocks,
                           unsigned rest_blocks, hipStream_t stream) {
  if (!jit_enabled()) return HMX_ERR_UNSUPPORTED;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return HMX_ERR_UNSUPPORTED;
  const std::string tmpl = std::to_string(lb) + ", hmx::ACT_JIT, " + (bf16 ? "true" : "false") + ", false";
  const std::string key = std::to_string(device) + "|gemm_rounds|" + std::to_string(lb) + "," +
                          (bf16 ? "bf16" : "f32") + "|" + epilogue_key(head.act, head.act_arg, head.prog);
  const std::string source =
      "#include \"hmx_gemm_mi16.hpp\"\n" + epilogue_source(head.act, head.act_arg, head.prog) +
      "extern \"C\" __global__ __launch_bounds__(512, 1) void hmx_jit_kernel(hmx::GemmArgs head, "
      "hmx::GemmArgs rest, int head_blocks) {\n"
      "  __shared__ __attribute__((aligned(1024))) uint8_t lds[hmx::mi16_lds_bytes<hmx::ACT_JIT, 256, 256, 8, 2>()];\n"
      "  const int b = (int)blockIdx.x;\n"
      "  if (b < head_blocks) hmx::gemm_bf16_mi16_body<" + tmpl + ", 256, 256, 8, 2>(head, lds, b, false);\n"
      "  else hmx::gemm_bf16_mi16_body<" + tmpl + ", 256, 128, 8, 2>(rest, lds, b - head_blocks, false);\n}\n";
  hipFunction_t fn = jit_function(key, source, device);
  if (!fn) return HMX_ERR_UNSUPPORTED;
  GemmArgs h = head, r = rest;
  int hb = (int)head_blocks;
  void* params[] = {&h, &r, &hb};
  return jit_launch(key, fn, dim3(head_blocks + rest_blocks), 512u, params, stream, "gemm");
}

int launch_group_norm_jit(bool bf16, const void* x, void* y, const GroupNormArgs& a, int64_t rows, int tpr,
                          int gv, int epv, int vpl, bool one, bool extra, unsigned block, int rows_per_block,
                          int cus, hipStream_t stream) {
  if (!jit_enabled()) return HMX_ERR_UNSUPPORTED;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return HMX_ERR_UNSUPPORTED;
  const std::string args = std::string(bf16 ? "uint16_t" : "float") + ", " + std::to_string(epv) + ", " +
                           std::to_string(vpl) + ", " + (one ? "true" : "false") + ", " +
                           (extra ? "true" : "false");
  const std::string key = std::to_string(device) + "|group_norm|" + args + "|" +
                          epilogue_key(a.act, a.act_arg, a.prog);
  const std::string t = bf16 ? "uint16_t" : "float";
  const std::string source =
      "#include \"hmx_rows_common.hpp\"\n" + epilogue_source(a.act, a.act_arg, a.prog) +
      "extern \"C\" __global__ __launch_bounds__(1024) void hmx_jit_kernel(const " + t + "* x, " + t +
      "* y, hmx::GroupNormArgs a, int64_t rows, int tpr, int gv) {\n  hmx::group_norm_rows_body<" + args +
      ", hmx::EPI_JIT>(x, y, a, rows, tpr, gv);\n}\n";
  hipFunction_t fn = jit_function(key, source, device);
  if (!fn) return HMX_ERR_UNSUPPORTED;
  // As many workgroups as the GPU holds at once, each walking rows blockIdx,
  // blockIdx + grid, ... (as the library's own launch of the kernel).
  int per_cu = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, (int)block, 0) != hipSuccess) {
    (void)hipGetLastError();
    per_cu = 1;
  }
  per_cu = std::max(per_cu, 1);
  const int64_t needed = ceil_div(rows, rows_per_block);
  const dim3 grid((unsigned)std::min<int64_t>(needed, (int64_t)per_cu * cus));
  const void* xp = x;
  void* yp = y;
  GroupNormArgs copy = a;
  void* params[] = {&xp, &yp, &copy, &rows, &tpr, &gv};
  return jit_launch(key, fn, grid, block, params, stream, "group_norm");
}

}  // namespace hmx

extern "C" int hmx_jit_info(int64_t* compiled, int64_t* failed, int64_t* launches) {
  std::lock_guard<std::mutex> guard(hmx::g_jit_lock);
  if (compiled) *compiled = hmx::g_jit_stats.compiled;
  if (failed) *failed = hmx::g_jit_stats.failed;
  if (launches) *launches = hmx::g_jit_stats.launches;
  return HMX_OK;
}

extern "C" const char* hmx_jit_last_log(void) {
  // A copy per thread: valid until this thread's next call, whatever other
  // threads' compilations write meanwhile.
  thread_local std::string copy;
  std::lock_guard<std::mutex> guard(hmx::g_jit_lock);
  copy = hmx::g_jit_last_log;
  return copy.c_str();
}
