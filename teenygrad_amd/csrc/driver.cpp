// Device, buffer, stream, event and code-object surface of teeny_hip.
//
// Replaces the CUDA driver crate's device layer (drivers/teeny-cuda/src/device/
// mod.rs:212-490, buffer.rs:37-62, program.rs:327-390) with direct HIP runtime
// calls.  Kernels are compiled ahead of time for gfx950, so there is no PTX
// JIT, no nvrtc and no Triton scratch-pointer convention.
#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <cstdlib>
#include <cstring>

#include "common.hpp"

namespace teeny {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

teeny_status fail(teeny_status code, const std::string &msg) {
  g_last_error = std::string(teeny_status_string(code)) + ": " + msg;
  return code;
}

teeny_status hip_fail(hipError_t err, const char *what) {
  // A failed HIP call also sets the runtime's per-thread last error, which
  // hipGetLastError would report again after the next launch: clear it, the
  // failure is reported here.
  (void)hipGetLastError();
  g_last_error = std::string("hip error ") + std::to_string(static_cast<int>(err)) + " (" +
                 hipGetErrorString(err) + ") in " + what;
  if (err == hipErrorNoDevice || err == hipErrorInvalidDevice) return TEENY_ERR_NO_DEVICE;
  return TEENY_ERR_HIP;
}

static bool sync_after_launch() {
  static const bool on = [] {
    const char *v = std::getenv("TEENY_HIP_SYNC");
    return v != nullptr && v[0] != '\0' && v[0] != '0';
  }();
  return on;
}

teeny_status after_launch(const char *what, hipStream_t stream) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  if (sync_after_launch()) {
    // a stream being captured into a graph records work instead of running it
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream != nullptr && hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return TEENY_OK;
    e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return hip_fail(e, what);
  }
  return TEENY_OK;
}

// Workspace registry: one caller-owned buffer per stream.  The null stream
// is per device, so it is keyed by the current device as well.
static std::mutex g_scratch_mu;
static std::map<std::pair<int, void *>, Scratch> g_scratch;

static std::pair<int, void *> scratch_key(void *stream) {
  int dev = -1;
  if (stream == nullptr && hipGetDevice(&dev) != hipSuccess) dev = 0;
  return {dev, stream};
}

Scratch stream_scratch(hipStream_t stream) {
  const auto key = scratch_key(stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch.find(key);
  return it == g_scratch.end() ? Scratch{} : it->second;
}

static void drop_scratch(void *stream) {
  const auto key = scratch_key(stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  g_scratch.erase(key);
}

int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

const char *teeny_hip_last_error(void) { return g_last_error.c_str(); }

const char *teeny_status_string(teeny_status status) {
  switch (status) {
    case TEENY_OK: return "ok";
    case TEENY_ERR_INVALID_ARGUMENT: return "invalid argument";
    case TEENY_ERR_NULL_POINTER: return "null pointer";
    case TEENY_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype";
    case TEENY_ERR_SHAPE_MISMATCH: return "shape mismatch";
    case TEENY_ERR_MISALIGNED: return "misaligned pointer";
    case TEENY_ERR_INVALID_AXIS: return "invalid axis";
    case TEENY_ERR_INVALID_GROUP_SIZE: return "invalid group size";
    case TEENY_ERR_NO_DEVICE: return "no device";
    case TEENY_ERR_HIP: return "hip error";
    case TEENY_ERR_NOT_FOUND: return "not found";
    case TEENY_ERR_UNSUPPORTED: return "unsupported";
    default: return "unknown status";
  }
}

const char *teeny_hip_version(void) { return "teeny_hip 0.1.0 gfx950"; }

teeny_status teeny_hip_init(void) {
  TEENY_CHECK_HIP(hipInit(0));
  return TEENY_OK;
}

teeny_status teeny_hip_device_count(int32_t *count) {
  TEENY_REQUIRE(count != nullptr, TEENY_ERR_NULL_POINTER, "count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return TEENY_OK;
  }
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  return TEENY_OK;
}

teeny_status teeny_hip_device_open(int32_t ordinal) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(TEENY_ERR_NO_DEVICE, "no HIP device visible");
  TEENY_REQUIRE(ordinal >= 0 && ordinal < n, TEENY_ERR_INVALID_ARGUMENT,
                "device ordinal " + std::to_string(ordinal) + " out of range");
  TEENY_CHECK_HIP(hipSetDevice(ordinal));
  return TEENY_OK;
}

teeny_status teeny_hip_device_info(int32_t ordinal, teeny_device_info *info) {
  TEENY_REQUIRE(info != nullptr, TEENY_ERR_NULL_POINTER, "info");
  hipDeviceProp_t p;
  TEENY_CHECK_HIP(hipGetDeviceProperties(&p, ordinal));
  std::memset(info, 0, sizeof(*info));
  std::strncpy(info->name, p.name, sizeof(info->name) - 1);
  std::strncpy(info->arch, p.gcnArchName, sizeof(info->arch) - 1);
  info->compute_units = p.multiProcessorCount;
  info->wavefront_size = p.warpSize;
  info->clock_khz = p.clockRate;
  info->memory_clock_khz = p.memoryClockRate;
  info->memory_bus_width = p.memoryBusWidth;
  info->l2_cache_bytes = p.l2CacheSize;
  info->total_global_mem = static_cast<int64_t>(p.totalGlobalMem);
  info->shared_mem_per_block = static_cast<int64_t>(p.sharedMemPerBlock);
  return TEENY_OK;
}

teeny_status teeny_hip_device_synchronize(void) {
  TEENY_CHECK_HIP(hipDeviceSynchronize());
  return TEENY_OK;
}

teeny_status teeny_hip_device_close(int32_t ordinal) {
  int cur = 0;
  TEENY_CHECK_HIP(hipGetDevice(&cur));
  if (cur == ordinal) TEENY_CHECK_HIP(hipDeviceSynchronize());
  return TEENY_OK;
}

teeny_status teeny_hip_malloc(void **ptr, size_t bytes) {
  TEENY_REQUIRE(ptr != nullptr, TEENY_ERR_NULL_POINTER, "ptr");
  *ptr = nullptr;
  if (bytes == 0) return TEENY_OK;
  TEENY_CHECK_HIP(hipMalloc(ptr, bytes));
  return TEENY_OK;
}

teeny_status teeny_hip_free(void *ptr) {
  if (ptr == nullptr) return TEENY_OK;
  TEENY_CHECK_HIP(hipFree(ptr));
  return TEENY_OK;
}

static teeny_status copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                         teeny_stream stream, const char *what) {
  if (bytes == 0) return TEENY_OK;
  TEENY_REQUIRE(dst != nullptr && src != nullptr, TEENY_ERR_NULL_POINTER, what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  TEENY_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, kind, s));
  // Host-side buffers are pageable: complete the copy before returning so the
  // caller may reuse or read its host memory immediately.
  if (kind != hipMemcpyDeviceToDevice) TEENY_CHECK_HIP(hipStreamSynchronize(s));
  return TEENY_OK;
}

teeny_status teeny_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, teeny_stream stream) {
  return copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "memcpy_h2d");
}
teeny_status teeny_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, teeny_stream stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "memcpy_d2h");
}
teeny_status teeny_hip_memcpy_d2d(void *dst, const void *src, size_t bytes, teeny_stream stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "memcpy_d2d");
}

teeny_status teeny_hip_memset(void *dst, int32_t value, size_t bytes, teeny_stream stream) {
  if (bytes == 0) return TEENY_OK;
  TEENY_REQUIRE(dst != nullptr, TEENY_ERR_NULL_POINTER, "dst");
  TEENY_CHECK_HIP(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)));
  return TEENY_OK;
}

teeny_status teeny_hip_stream_create(teeny_stream *stream) {
  TEENY_REQUIRE(stream != nullptr, TEENY_ERR_NULL_POINTER, "stream");
  hipStream_t s = nullptr;
  TEENY_CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return TEENY_OK;
}

teeny_status teeny_hip_stream_destroy(teeny_stream stream) {
  if (stream == nullptr) return TEENY_OK;
  drop_scratch(stream);
  TEENY_CHECK_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return TEENY_OK;
}

teeny_status teeny_hip_stream_set_workspace(teeny_stream stream, void *ptr, size_t bytes) {
  if (ptr == nullptr || bytes == 0) {
    drop_scratch(stream);
    return TEENY_OK;
  }
  TEENY_REQUIRE(aligned(ptr, 256), TEENY_ERR_MISALIGNED,
                "stream_set_workspace: workspace must be 256-byte aligned");
  const auto key = scratch_key(stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  g_scratch[key] = Scratch{ptr, bytes};
  return TEENY_OK;
}

teeny_status teeny_hip_stream_sync(teeny_stream stream) {
  TEENY_CHECK_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return TEENY_OK;
}

teeny_status teeny_hip_event_create(teeny_event *event) {
  TEENY_REQUIRE(event != nullptr, TEENY_ERR_NULL_POINTER, "event");
  hipEvent_t e = nullptr;
  TEENY_CHECK_HIP(hipEventCreate(&e));
  *event = e;
  return TEENY_OK;
}

teeny_status teeny_hip_event_destroy(teeny_event event) {
  if (event == nullptr) return TEENY_OK;
  TEENY_CHECK_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return TEENY_OK;
}

teeny_status teeny_hip_event_record(teeny_event event, teeny_stream stream) {
  TEENY_REQUIRE(event != nullptr, TEENY_ERR_NULL_POINTER, "event");
  TEENY_CHECK_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return TEENY_OK;
}

teeny_status teeny_hip_event_sync(teeny_event event) {
  TEENY_REQUIRE(event != nullptr, TEENY_ERR_NULL_POINTER, "event");
  TEENY_CHECK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return TEENY_OK;
}

teeny_status teeny_hip_event_elapsed_ms(float *ms, teeny_event start, teeny_event stop) {
  TEENY_REQUIRE(ms != nullptr && start != nullptr && stop != nullptr, TEENY_ERR_NULL_POINTER,
                "ms/start/stop");
  TEENY_CHECK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                      static_cast<hipEvent_t>(stop)));
  return TEENY_OK;
}

teeny_status teeny_hip_stream_begin_capture(teeny_stream stream) {
  TEENY_REQUIRE(stream != nullptr, TEENY_ERR_INVALID_ARGUMENT,
                "stream_begin_capture: the null stream cannot be captured");
  TEENY_CHECK_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
  return TEENY_OK;
}

teeny_status teeny_hip_stream_end_capture(teeny_stream stream, teeny_graph *graph) {
  TEENY_REQUIRE(stream != nullptr && graph != nullptr, TEENY_ERR_NULL_POINTER, "stream_end_capture: stream/graph");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  TEENY_CHECK_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph = exec;
  return TEENY_OK;
}

teeny_status teeny_hip_graph_launch(teeny_graph graph, teeny_stream stream) {
  TEENY_REQUIRE(graph != nullptr, TEENY_ERR_NULL_POINTER, "graph_launch: graph");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TEENY_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), s));
  if (sync_after_launch()) TEENY_CHECK_HIP(hipStreamSynchronize(s));
  return TEENY_OK;
}

teeny_status teeny_hip_graph_destroy(teeny_graph graph) {
  if (graph == nullptr) return TEENY_OK;
  TEENY_CHECK_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
  return TEENY_OK;
}

teeny_status teeny_hip_module_load(teeny_module *module, const char *path) {
  TEENY_REQUIRE(module != nullptr && path != nullptr, TEENY_ERR_NULL_POINTER, "module/path");
  hipModule_t m = nullptr;
  TEENY_CHECK_HIP(hipModuleLoad(&m, path));
  *module = m;
  return TEENY_OK;
}

teeny_status teeny_hip_module_load_data(teeny_module *module, const void *image) {
  TEENY_REQUIRE(module != nullptr && image != nullptr, TEENY_ERR_NULL_POINTER, "module/image");
  hipModule_t m = nullptr;
  TEENY_CHECK_HIP(hipModuleLoadData(&m, image));
  *module = m;
  return TEENY_OK;
}

teeny_status teeny_hip_module_get_function(teeny_function *function, teeny_module module,
                                           const char *name) {
  TEENY_REQUIRE(function != nullptr && module != nullptr && name != nullptr,
                TEENY_ERR_NULL_POINTER, "function/module/name");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (e == hipErrorNotFound) {
    (void)hipGetLastError();  // clear the runtime's last error (see hip_fail)
    return fail(TEENY_ERR_NOT_FOUND, std::string("kernel ") + name);
  }
  if (e != hipSuccess) return hip_fail(e, "hipModuleGetFunction");
  *function = f;
  return TEENY_OK;
}

teeny_status teeny_hip_module_unload(teeny_module module) {
  if (module == nullptr) return TEENY_OK;
  TEENY_CHECK_HIP(hipModuleUnload(static_cast<hipModule_t>(module)));
  return TEENY_OK;
}

teeny_status teeny_hip_launch(teeny_function function, const uint32_t grid[3],
                              const uint32_t block[3], uint32_t shared_mem_bytes,
                              teeny_stream stream, void **args) {
  TEENY_REQUIRE(function != nullptr && grid != nullptr && block != nullptr,
                TEENY_ERR_NULL_POINTER, "function/grid/block");
  TEENY_REQUIRE(grid[0] && grid[1] && grid[2], TEENY_ERR_INVALID_ARGUMENT, "empty grid");
  const uint64_t threads = static_cast<uint64_t>(block[0]) * block[1] * block[2];
  TEENY_REQUIRE(threads >= 1 && threads <= 1024, TEENY_ERR_INVALID_ARGUMENT,
                "block must have 1..1024 threads");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the launch reports its own status: a stale last error from an earlier,
  // unrelated HIP call must not be attributed to it
  (void)hipGetLastError();
  TEENY_CHECK_HIP(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid[0], grid[1],
                                        grid[2], block[0], block[1], block[2], shared_mem_bytes,
                                        s, args, nullptr));
  return after_launch("teeny_hip_launch", s);
}

}  // extern "C"
