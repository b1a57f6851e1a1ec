// runtime.hip -- device selection, memory, stream ordering and error reporting.
//
// Replaces the Metal bridge's runtime half (engine/metal/metal_backend.h:15-69,
// metal_backend.m:336-368 mtl_alloc/mtl_free).  One global device and stream,
// like the bridge's one device/queue; see madi_q8.h for the contract.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>

#include "common.h"

namespace madi {

namespace {
thread_local char g_err[512] = "";
bool g_init = false;
int g_cu_count = 0;
hipStream_t g_stream = nullptr;
// Orders a newly chosen stream after the work already issued on the old one.
hipEvent_t g_switch = nullptr;
// Split-K workspace: kCounters zeroed arrival counters, then the partial sums.
constexpr size_t kCounters = 16384;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;
// Workspaces outgrown by a larger split shape.  A HIP graph captured before
// the growth still names the old buffer in its kernel arguments, so an
// outgrown buffer stays allocated (and its counters at zero) until
// madi_cleanup; freeing it would let a replay write partial sums into
// memory that may have been handed out again.
constexpr int kMaxRetired = 32;
void *g_retired[kMaxRetired];
int g_nretired = 0;
// Live madi_alloc allocations (base -> bytes), for the deferred
// dequantisation's free and write extents.
std::map<uintptr_t, size_t> g_allocs;

void free_workspace() {
  if (g_ws || g_nretired) (void)hipDeviceSynchronize();
  if (g_ws) (void)hipFree(g_ws);
  for (int i = 0; i < g_nretired; ++i) (void)hipFree(g_retired[i]);
  g_nretired = 0;
  g_ws = nullptr;
  g_ws_bytes = 0;
}
}  // namespace

int workspace(size_t partial_bytes, size_t counters, float **partials, uint32_t **cnt) {
  if (counters > kCounters)
    return fail(MADI_ERR_SHAPE, "split-K workspace: %zu tiles exceed %zu", counters, kCounters);
  const size_t need = kCounters * 4 + partial_bytes;
  if (need > g_ws_bytes) {
    // growing allocates and synchronises, which a stream under graph capture
    // cannot do: the caller makes one such call before capturing
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(MADI_ERR_ARG,
                  "split-K workspace must grow to %zu bytes, which cannot happen during graph "
                  "capture; run this GEMM shape once before capturing", need);
    // the old buffer is retired, not freed (kernels still running and graphs
    // captured earlier may use it); growing at least twofold keeps the
    // number of retired buffers logarithmic in the largest shape
    if (g_ws && g_nretired == kMaxRetired)
      return fail(MADI_ERR_ALLOC, "split-K workspace: %d growths already retired", kMaxRetired);
    const size_t grow = g_ws_bytes * 2 > need ? g_ws_bytes * 2 : need;
    void *fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, grow);
    if (e != hipSuccess)
      return fail(MADI_ERR_ALLOC, "split-K workspace (%zu bytes): %s", grow, hipGetErrorString(e));
    // the counters start at zero; every use returns them to zero
    e = hipMemset(fresh, 0, kCounters * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      (void)hipFree(fresh);
      return fail(MADI_ERR_ALLOC, "split-K workspace: clearing the counters: %s", hipGetErrorString(e));
    }
    if (g_ws) g_retired[g_nretired++] = g_ws;
    g_ws = fresh;
    g_ws_bytes = grow;
  }
  *cnt = static_cast<uint32_t *>(g_ws);
  *partials = reinterpret_cast<float *>(static_cast<uint8_t *>(g_ws) + kCounters * 4);
  return MADI_OK;
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MADI_ERR_DISPATCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MADI_OK;
}

size_t alloc_extent(const void *ptr) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  auto it = g_allocs.upper_bound(p);
  if (it == g_allocs.begin()) return 0;
  --it;
  const uintptr_t end = it->first + it->second;
  return p < end ? end - p : 0;
}

bool initialized() { return g_init; }
int cu_count() { return g_cu_count; }
hipStream_t stream() { return g_stream; }

}  // namespace madi

using namespace madi;

extern "C" int madi_init(void) {
  if (g_init) return MADI_OK;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count < 1)
    return fail(MADI_ERR_INIT, "madi_init: no HIP device (%s)", hipGetErrorString(e));
  e = hipSetDevice(0);
  if (e != hipSuccess) return fail(MADI_ERR_INIT, "madi_init: hipSetDevice: %s", hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, 0);
  if (e != hipSuccess)
    return fail(MADI_ERR_INIT, "madi_init: hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MADI_ERR_INIT, "madi_init: device is %s, this library is built for gfx950",
                prop.gcnArchName);
  g_cu_count = prop.multiProcessorCount;
  g_init = true;
  // A workspace big enough for every split GEMV / projection (and small
  // split GEMMs) from the start, so those never allocate later (e.g. while a
  // caller captures a graph).
  float *partials = nullptr;
  uint32_t *cnt = nullptr;
  if (int rc = workspace(size_t(4) << 20, kCounters, &partials, &cnt)) {
    g_init = false;
    return rc;
  }
  // the allocation-free GEMM's scratch address on this device
  if (int rc = gemm_scratch_init()) {
    g_init = false;
    return rc;
  }
  if (!g_switch) {
    e = hipEventCreateWithFlags(&g_switch, hipEventDisableTiming);
    if (e != hipSuccess) {
      g_switch = nullptr;
      g_init = false;
      return fail(MADI_ERR_INIT, "madi_init: hipEventCreate: %s", hipGetErrorString(e));
    }
  }
  g_err[0] = 0;
  return MADI_OK;
}

extern "C" void madi_cleanup(void) {
  if (!g_init) return;
  (void)deferred_flush_all();
  (void)hipStreamSynchronize(g_stream);
  free_workspace();
  f16gemm_cleanup();
  if (g_switch) (void)hipEventDestroy(g_switch);
  g_switch = nullptr;
  g_stream = nullptr;
  g_init = false;
}

extern "C" void *madi_alloc(size_t size) {
  if (!g_init) {
    fail(MADI_ERR_NOT_INIT, "madi_alloc: madi_init has not succeeded");
    return nullptr;
  }
  if (size == 0) size = 1;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) {
    fail(MADI_ERR_ALLOC, "madi_alloc(%zu): %s", size, hipGetErrorString(e));
    return nullptr;
  }
  g_allocs[reinterpret_cast<uintptr_t>(p)] = size;
  return p;
}

extern "C" void madi_free(void *ptr) {
  if (!ptr || !g_init) return;
  const size_t ext = alloc_extent(ptr);
  // a dequantisation launched from the memory being freed finishes first
  if (deferred_before_free(ptr, ext ? ext : 1) > 0) (void)hipStreamSynchronize(g_stream);
  g_allocs.erase(reinterpret_cast<uintptr_t>(ptr));
  (void)hipFree(ptr);
}

extern "C" int madi_upload(void *dst, const void *src, size_t size) {
  if (!g_init) return fail(MADI_ERR_NOT_INIT, "madi_upload: madi_init has not succeeded");
  if (size == 0) return MADI_OK;
  if (!dst || !src) return fail(MADI_ERR_NULL, "madi_upload: null pointer");
  if (int rc = deferred_before_write(dst, size)) return rc;
  hipError_t e = hipMemcpyAsync(dst, src, size, hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) return fail(MADI_ERR_SYNC, "madi_upload: %s", hipGetErrorString(e));
  return MADI_OK;
}

extern "C" int madi_download(void *dst, const void *src, size_t size) {
  if (!g_init) return fail(MADI_ERR_NOT_INIT, "madi_download: madi_init has not succeeded");
  if (size == 0) return MADI_OK;
  if (!dst || !src) return fail(MADI_ERR_NULL, "madi_download: null pointer");
  if (int rc = deferred_before_read(src, size)) return rc;
  hipError_t e = hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) return fail(MADI_ERR_SYNC, "madi_download: %s", hipGetErrorString(e));
  return MADI_OK;
}

extern "C" int madi_begin_command_buffer(void) {
  if (!g_init) return fail(MADI_ERR_NOT_INIT, "madi_begin_command_buffer: not initialised");
  return MADI_OK;
}

extern "C" int madi_commit_command_buffer(void) {
  if (!g_init) return fail(MADI_ERR_NOT_INIT, "madi_commit_command_buffer: not initialised");
  if (int rc = group_flush()) return rc;
  return check_launch("madi_commit_command_buffer");
}

extern "C" int madi_sync(void) {
  if (!g_init) return fail(MADI_ERR_NOT_INIT, "madi_sync: madi_init has not succeeded");
  if (int rc = group_flush()) return rc;
  hipError_t e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) return fail(MADI_ERR_SYNC, "madi_sync: %s", hipGetErrorString(e));
  return MADI_OK;
}

extern "C" int madi_set_stream(void *s) {
  const hipStream_t ns = reinterpret_cast<hipStream_t>(s);
  if (g_init) {
    // work held for a later launch goes to the stream it was issued on
    if (int rc = group_flush()) return rc;
    // The library's launches stay in call order across the switch: the new
    // stream waits for what the old one holds (split-K launches on the two
    // would otherwise share the workspace's partials and counters at once).
    // A stream under graph capture may not wait on work outside it, so
    // around a capture the caller orders the two streams itself.  The new
    // stream is asked first: entering a capture, the old one (often the
    // legacy null stream, which must not be queried while another stream
    // captures) is left alone.
    hipStreamCaptureStatus a = hipStreamCaptureStatusNone, b = hipStreamCaptureStatusNone;
    if (ns != g_stream && hipStreamIsCapturing(ns, &b) == hipSuccess &&
        b == hipStreamCaptureStatusNone && hipStreamIsCapturing(g_stream, &a) == hipSuccess &&
        a == hipStreamCaptureStatusNone) {
      hipError_t e = hipEventRecord(g_switch, g_stream);
      if (e == hipSuccess) e = hipStreamWaitEvent(ns, g_switch, 0);
      if (e != hipSuccess)
        return fail(MADI_ERR_DISPATCH, "madi_set_stream: ordering the new stream: %s",
                    hipGetErrorString(e));
    }
  }
  g_stream = ns;
  return MADI_OK;
}

extern "C" const char *madi_last_error(void) { return g_err; }

extern "C" int madi_device_cu_count(void) { return g_init ? g_cu_count : 0; }
