// The runtime half of the C ABI: errors, device info, buffers, streams, events and graph capture — the gfx950
// equivalents of the reference's native Device/Buffer/Queue/Icb classes (runtime/src/metal_core.h:20-116).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "mi_common.h"

namespace {
thread_local char g_err[512] = "";
}

int mi_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int mi_check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return MI_OK;
  (void)hipGetLastError();     // reported here: clear the thread's sticky error so the next caller's check is its own
  return mi_set_error(MI_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

namespace {
struct Scratch { void* ptr; size_t bytes; };
std::mutex g_scratch_mu;
std::map<std::tuple<int, int, hipStream_t>, Scratch> g_scratch;
std::vector<void*> g_retired;   // outgrown buffers: kept until the process ends (captured graphs may point at them)
}  // namespace

int mi_library_scratch(int kind, size_t bytes, hipStream_t stream, void** out) {
  int dev = 0;
  MI_TRY_HIP(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  Scratch& w = g_scratch[std::make_tuple(kind, dev, stream)];
  if (w.bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    MI_TRY_HIP(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
      return mi_set_error(MI_E_INVALID, "library scratch (kind %d) must grow from %zu to %zu bytes during a graph "
                          "capture: run one eager call of this shape on the stream first, or pass a workspace",
                          kind, w.bytes, bytes);
    const size_t grow = bytes < (64u << 10) ? (64u << 10) : bytes;
    void* p = nullptr;
    MI_TRY_HIP(hipMalloc(&p, grow), "hipMalloc(library scratch)");
    // zeroed on the stream that will use it, so the clear is ordered before that stream's kernels (a plain
    // hipMemset runs on the null stream, which a non-blocking stream does not wait for)
    if (int rc = mi_check_hip(hipMemsetAsync(p, 0, grow, stream), "hipMemsetAsync(library scratch)")) {
      (void)hipFree(p);
      return rc;
    }
    if (w.ptr) g_retired.push_back(w.ptr);
    w = {p, grow};
  }
  *out = w.ptr;
  return MI_OK;
}

extern "C" {

const char* mi_version(void) { return "lithos-mi355 0.1.0 (gfx950)"; }

int mi_last_error(char* buf, size_t n) {
  if (buf && n) {
    strncpy(buf, g_err, n - 1);
    buf[n - 1] = 0;
  }
  return MI_OK;
}

int mi_device_count(int32_t* count) {
  MI_REQUIRE(count, "mi_device_count: null output");
  int c = 0;
  MI_TRY_HIP(hipGetDeviceCount(&c), "hipGetDeviceCount");
  *count = c;
  return MI_OK;
}

int mi_device_info_get(int32_t device, mi_device_info* out) {
  MI_REQUIRE(out, "mi_device_info_get: null output");
  hipDeviceProp_t p;
  MI_TRY_HIP(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
  memset(out, 0, sizeof(*out));
  strncpy(out->name, p.name, sizeof(out->name) - 1);
  strncpy(out->arch, p.gcnArchName, sizeof(out->arch) - 1);
  out->compute_units = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->hbm_bytes = (int64_t)p.totalGlobalMem;
  out->lds_bytes_per_block = (int32_t)p.sharedMemPerBlock;
  out->warp_size = p.warpSize;
  return MI_OK;
}

int mi_set_device(int32_t device) {
  MI_TRY_HIP(hipSetDevice(device), "hipSetDevice");
  return MI_OK;
}

int mi_malloc(void** ptr, size_t bytes) {
  MI_REQUIRE(ptr, "mi_malloc: null output");
  MI_TRY_HIP(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
  return MI_OK;
}

int mi_free(void* ptr) {
  if (!ptr) return MI_OK;
  MI_TRY_HIP(hipFree(ptr), "hipFree");
  return MI_OK;
}

int mi_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  MI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync(h2d)");
  if (!stream) MI_TRY_HIP(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
  return MI_OK;
}

int mi_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  MI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync(d2h)");
  if (!stream) MI_TRY_HIP(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
  return MI_OK;
}

int mi_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  MI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync(d2d)");
  return MI_OK;
}

int mi_memset(void* dst, int32_t byte, size_t bytes, void* stream) {
  MI_TRY_HIP(hipMemsetAsync(dst, byte, bytes, (hipStream_t)stream), "hipMemsetAsync");
  return MI_OK;
}

int mi_stream_create(void** stream) {
  MI_REQUIRE(stream, "mi_stream_create: null output");
  hipStream_t s;
  MI_TRY_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return MI_OK;
}

int mi_stream_destroy(void* stream) {
  if (!stream) return MI_OK;
  MI_TRY_HIP(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
  return MI_OK;
}

int mi_stream_synchronize(void* stream) {
  MI_TRY_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  return MI_OK;
}

int mi_event_create(void** event) {
  MI_REQUIRE(event, "mi_event_create: null output");
  hipEvent_t e;
  MI_TRY_HIP(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return MI_OK;
}

int mi_event_destroy(void* event) {
  if (!event) return MI_OK;
  MI_TRY_HIP(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
  return MI_OK;
}

int mi_event_record(void* event, void* stream) {
  MI_TRY_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
  return MI_OK;
}

int mi_event_synchronize(void* event) {
  MI_TRY_HIP(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
  return MI_OK;
}

int mi_event_elapsed_ms(void* start, void* end, float* ms) {
  MI_REQUIRE(ms, "mi_event_elapsed_ms: null output");
  MI_TRY_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
  return MI_OK;
}

int mi_graph_begin(void* stream) {
  MI_REQUIRE(stream, "mi_graph_begin: capture needs a created stream (not the null stream)");
  MI_TRY_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  return MI_OK;
}

int mi_graph_end(void* stream, void** graph_exec) {
  MI_REQUIRE(graph_exec, "mi_graph_end: null output");
  hipGraph_t g;
  MI_TRY_HIP(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture");
  hipGraphExec_t ex;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  MI_TRY_HIP(e, "hipGraphInstantiate");
  *graph_exec = ex;
  return MI_OK;
}

int mi_graph_launch(void* graph_exec, void* stream) {
  MI_TRY_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream), "hipGraphLaunch");
  return MI_OK;
}

int mi_graph_destroy(void* graph_exec) {
  if (!graph_exec) return MI_OK;
  MI_TRY_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec), "hipGraphExecDestroy");
  return MI_OK;
}

}  // extern "C"
