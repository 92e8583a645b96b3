// Run-time kernels and file-backed buffers: the gfx950 equivalents of the reference's Library (source + macros,
// compiled at run time), Pipeline (one function of a library), Dispatch/Queue launch and Buffer.from_file
// (runtime/src/metal_core.h:37-66, metal_core.mm:70-127; the nanobind surface runtime/src/native.mm:24-58).
//
// MI355X design: hiprtc compiles source for gfx950 into a code object (no GPU needed, so a program can be built on
// a host without one and shipped as bytes); hipModuleLoadData loads it per device; a launch passes the kernel's
// parameters as one packed argument block (the HIP kernarg segment) rather than per-index bindings. File windows
// are read through a bounded pinned staging buffer into device memory (HBM is not host-mapped the way Apple's
// unified memory is, so the reference's no-copy mmap buffer becomes a copy at load time).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "mi_common.h"

namespace {

int rtc_fail(hiprtcResult r, const char* what, const std::string& log = "") {
  // the log's tail carries the first error's line in practice; the error buffer holds 512 bytes
  const std::string tail = log.size() > 380 ? log.substr(log.size() - 380) : log;
  return mi_set_error(MI_E_INVALID, "%s: %s%s%s", what, hiprtcGetErrorString(r), tail.empty() ? "" : "\n",
                      tail.c_str());
}

constexpr size_t kStageBytes = 64ull << 20;   // pinned staging for file windows

}  // namespace

extern "C" {

int mi_library_compile(const char* source, const char* const* macros, int32_t n_macros, int32_t fast_math,
                       void** code, size_t* code_bytes) {
  MI_REQUIRE(source && code && code_bytes, "mi_library_compile: null argument");
  MI_REQUIRE(n_macros >= 0 && (n_macros == 0 || macros), "mi_library_compile: bad macro list");
  *code = nullptr;
  *code_bytes = 0;
  std::vector<std::string> opts = {"--offload-arch=gfx950", "-O3", "-std=c++17",
                                   // no packed-FP32 instructions (the same rule as the library's own kernels)
                                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  if (fast_math) opts.push_back("-ffast-math");
  for (int i = 0; i < n_macros; ++i) {
    MI_REQUIRE(macros[2 * i] && macros[2 * i][0], "mi_library_compile: macro %d has no name", i);
    const char* v = macros[2 * i + 1];
    opts.push_back(std::string("-D") + macros[2 * i] + (v && v[0] ? std::string("=") + v : std::string()));
  }
  std::vector<const char*> argv;
  for (auto& o : opts) argv.push_back(o.c_str());

  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, "library.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return rtc_fail(r, "hiprtcCreateProgram");
  r = hiprtcCompileProgram(prog, (int)argv.size(), argv.data());
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    std::string log;
    if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
      log.resize(n);
      if (hiprtcGetProgramLog(prog, &log[0]) != HIPRTC_SUCCESS) log.clear();
      while (!log.empty() && (log.back() == '\0' || log.back() == '\n')) log.pop_back();
    }
    (void)hiprtcDestroyProgram(&prog);
    return rtc_fail(r, "compile failed", log);
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  void* buf = (r == HIPRTC_SUCCESS && n) ? malloc(n) : nullptr;
  if (buf) r = hiprtcGetCode(prog, static_cast<char*>(buf));
  (void)hiprtcDestroyProgram(&prog);
  if (!buf || r != HIPRTC_SUCCESS) {
    free(buf);
    return rtc_fail(r == HIPRTC_SUCCESS ? HIPRTC_ERROR_INTERNAL_ERROR : r, "hiprtcGetCode");
  }
  *code = buf;
  *code_bytes = n;
  return MI_OK;
}

int mi_code_free(void* code) {
  free(code);
  return MI_OK;
}

int mi_library_load(const void* code, size_t code_bytes, void** library) {
  MI_REQUIRE(code && code_bytes && library, "mi_library_load: null argument");
  hipModule_t m;
  MI_TRY_HIP(hipModuleLoadData(&m, code), "hipModuleLoadData");
  *library = m;
  return MI_OK;
}

int mi_library_release(void* library) {
  if (!library) return MI_OK;
  MI_TRY_HIP(hipModuleUnload(static_cast<hipModule_t>(library)), "hipModuleUnload");
  return MI_OK;
}

int mi_kernel_get(void* library, const char* name, void** kernel) {
  MI_REQUIRE(library && name && kernel, "mi_kernel_get: null argument");
  hipFunction_t f;
  const hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(library), name);
  if (e == hipErrorNotFound || e == hipErrorInvalidSymbol) {
    (void)hipGetLastError();   // the lookup's error is reported here, not to the next HIP caller
    return mi_set_error(MI_E_INVALID, "no kernel named %s", name);
  }
  MI_TRY_HIP(e, "hipModuleGetFunction");
  *kernel = f;
  return MI_OK;
}

int mi_kernel_info(void* kernel, mi_kernel_attrs* out) {
  MI_REQUIRE(kernel && out, "mi_kernel_info: null argument");
  const hipFunction_t f = static_cast<hipFunction_t>(kernel);
  int v = 0;
  memset(out, 0, sizeof(*out));
  MI_TRY_HIP(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f), "hipFuncGetAttribute");
  out->max_threads_per_block = v;
  MI_TRY_HIP(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f), "hipFuncGetAttribute");
  out->static_lds_bytes = v;
  MI_TRY_HIP(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, f), "hipFuncGetAttribute");
  out->registers = v;
  MI_TRY_HIP(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, f), "hipFuncGetAttribute");
  out->scratch_bytes = v;
  out->wave_size = 64;
  return MI_OK;
}

int mi_launch(void* kernel, const void* args, size_t args_bytes, const uint32_t grid[3], const uint32_t block[3],
              uint32_t lds_bytes, void* stream) {
  MI_REQUIRE(kernel && grid && block, "mi_launch: null argument");
  MI_REQUIRE(args_bytes == 0 || args, "mi_launch: %zu argument bytes and no argument block", args_bytes);
  MI_REQUIRE(args_bytes <= 4096, "mi_launch: argument block of %zu bytes exceeds 4096", args_bytes);
  for (int i = 0; i < 3; ++i) MI_REQUIRE(grid[i] >= 1 && block[i] >= 1, "mi_launch: empty grid or workgroup");
  const uint64_t threads = (uint64_t)block[0] * block[1] * block[2];
  MI_REQUIRE(threads <= 1024, "mi_launch: %llu threads per workgroup exceed 1024", (unsigned long long)threads);
  MI_REQUIRE(lds_bytes <= 160 * 1024, "mi_launch: %u LDS bytes exceed 160 KiB", lds_bytes);
  alignas(16) unsigned char block_args[4096];
  size_t n = args_bytes;
  if (n) memcpy(block_args, args, n);
  void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, block_args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &n,
                   HIP_LAUNCH_PARAM_END};
  MI_TRY_HIP(hipModuleLaunchKernel(static_cast<hipFunction_t>(kernel), grid[0], grid[1], grid[2], block[0], block[1],
                                   block[2], lds_bytes, static_cast<hipStream_t>(stream), nullptr,
                                   n ? extra : nullptr),
             "hipModuleLaunchKernel");
  return MI_OK;
}

int mi_buf_from_file(const char* path, uint64_t offset, size_t bytes, void** ptr) {
  MI_REQUIRE(path && ptr, "mi_buf_from_file: null argument");
  *ptr = nullptr;
  const long page = sysconf(_SC_PAGESIZE);
  MI_REQUIRE(bytes > 0 && offset % page == 0 && bytes % page == 0,
             "mi_buf_from_file: file windows need a page-aligned offset and length (page %ld)", page);
  const int fd = open(path, O_RDONLY);
  MI_REQUIRE(fd >= 0, "mi_buf_from_file: open failed: %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || (uint64_t)st.st_size < offset + bytes) {
    close(fd);
    return mi_set_error(MI_E_INVALID, "mi_buf_from_file: %s holds %lld bytes, the window ends at %llu", path,
                        (long long)st.st_size, (unsigned long long)(offset + bytes));
  }
  void* dev = nullptr;
  void* stage = nullptr;
  hipError_t e = hipMalloc(&dev, bytes);
  if (e == hipSuccess) e = hipHostMalloc(&stage, std::min(bytes, kStageBytes), hipHostMallocDefault);
  int rc = e == hipSuccess ? MI_OK : mi_check_hip(e, "mi_buf_from_file: allocation");
  for (size_t done = 0; rc == MI_OK && done < bytes;) {
    const size_t want = std::min(bytes - done, kStageBytes);
    size_t got = 0;
    while (got < want) {
      const ssize_t r = pread(fd, static_cast<char*>(stage) + got, want - got, (off_t)(offset + done + got));
      if (r <= 0) break;
      got += (size_t)r;
    }
    if (got != want) {
      rc = mi_set_error(MI_E_INVALID, "mi_buf_from_file: short read of %s at %llu", path,
                        (unsigned long long)(offset + done + got));
      break;
    }
    e = hipMemcpy(static_cast<char*>(dev) + done, stage, want, hipMemcpyHostToDevice);
    if (e != hipSuccess) rc = mi_check_hip(e, "mi_buf_from_file: hipMemcpy");
    done += want;
  }
  close(fd);
  if (stage) (void)hipHostFree(stage);
  if (rc != MI_OK) {
    if (dev) (void)hipFree(dev);
    return rc;
  }
  *ptr = dev;
  return MI_OK;
}

}  // extern "C"
