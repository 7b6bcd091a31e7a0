// hb_* runtime half: device selection, memory, streams and events behind the
// plain C ABI of include/htp_ops/hb.h.  One library stream per device is
// created on first use; every kernel entry point accepts a caller stream.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>

#include "hb_internal.h"

namespace {

thread_local char g_last_error[256] = "";

constexpr int kMaxDevices = 16;
std::mutex g_mutex;
hipStream_t g_streams[kMaxDevices] = {};

}  // namespace

int hb_fail(hipError_t err, const char *what) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
  return err == hipErrorOutOfMemory ? HB_E_NOMEM : HB_E_HIP;
}

int hb_invalid(const char *what) {
  std::snprintf(g_last_error, sizeof(g_last_error), "invalid argument: %s", what);
  return HB_E_INVAL;
}

hipStream_t hb_resolve_stream(hb_stream s) {
  if (s != nullptr) return (hipStream_t)s;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  return g_streams[dev];
}

extern "C" {

const char *hb_last_error(void) { return g_last_error; }

int hb_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int hb_init(int device) {
  int n = 0;
  hipError_t err = hipGetDeviceCount(&n);
  if (err != hipSuccess || n <= 0) {
    std::snprintf(g_last_error, sizeof(g_last_error), "no GPU visible to HIP (%s)",
                  err == hipSuccess ? "0 devices" : hipGetErrorString(err));
    return HB_E_NODEV;
  }
  if (device < 0 || device >= n || device >= kMaxDevices) return hb_invalid("device index");
  err = hipSetDevice(device);
  if (err != hipSuccess) return hb_fail(err, "hipSetDevice");
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_streams[device] == nullptr) {
    hipStream_t st = nullptr;
    err = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    if (err != hipSuccess) return hb_fail(err, "hipStreamCreateWithFlags");
    g_streams[device] = st;
  }
  // the no-allocation entry point's static workspace on this device
  return hb_w8a8_static_setup(device);
}

hb_stream hb_default_stream(void) { return (hb_stream)hb_resolve_stream(nullptr); }

int hb_malloc(void **d_ptr, size_t bytes) {
  if (d_ptr == nullptr) return hb_invalid("hb_malloc out");
  *d_ptr = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t err = hipMalloc(d_ptr, bytes);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipMalloc");
}

int hb_free(void *d_ptr) {
  if (d_ptr == nullptr) return HB_OK;
  hipError_t err = hipFree(d_ptr);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipFree");
}

int hb_host_malloc(void **h_ptr, size_t bytes) {
  if (h_ptr == nullptr) return hb_invalid("hb_host_malloc out");
  *h_ptr = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t err = hipHostMalloc(h_ptr, bytes, hipHostMallocDefault);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipHostMalloc");
}

int hb_host_free(void *h_ptr) {
  if (h_ptr == nullptr) return HB_OK;
  hipError_t err = hipHostFree(h_ptr);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipHostFree");
}

static int copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hb_stream s, const char *what) {
  if (bytes == 0) return HB_OK;
  if (dst == nullptr || src == nullptr) return hb_invalid(what);
  hipStream_t st = hb_resolve_stream(s);
  hipError_t err = hipMemcpyAsync(dst, src, bytes, kind, st);
  if (err != hipSuccess) return hb_fail(err, what);
  err = hipStreamSynchronize(st);
  return err == hipSuccess ? HB_OK : hb_fail(err, what);
}

int hb_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, hb_stream s) {
  return copy(d_dst, h_src, bytes, hipMemcpyHostToDevice, s, "hb_memcpy_h2d");
}

int hb_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, hb_stream s) {
  return copy(h_dst, d_src, bytes, hipMemcpyDeviceToHost, s, "hb_memcpy_d2h");
}

int hb_memcpy_d2h_async(void *h_dst, const void *d_src, size_t bytes, hb_stream s) {
  if (bytes == 0) return HB_OK;
  if (h_dst == nullptr || d_src == nullptr) return hb_invalid("hb_memcpy_d2h_async");
  hipError_t err = hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hb_memcpy_d2h_async");
}

int hb_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, hb_stream s) {
  if (bytes == 0) return HB_OK;
  if (d_dst == nullptr || d_src == nullptr) return hb_invalid("hb_memcpy_d2d");
  hipError_t err = hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hb_memcpy_d2d");
}

int hb_memset(void *d_dst, int value, size_t bytes, hb_stream s) {
  if (bytes == 0) return HB_OK;
  if (d_dst == nullptr) return hb_invalid("hb_memset");
  hipError_t err = hipMemsetAsync(d_dst, value, bytes, hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipMemsetAsync");
}

int hb_stream_create(hb_stream *s) {
  if (s == nullptr) return hb_invalid("hb_stream_create out");
  hipStream_t st = nullptr;
  hipError_t err = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
  if (err != hipSuccess) return hb_fail(err, "hipStreamCreateWithFlags");
  *s = (hb_stream)st;
  return HB_OK;
}

int hb_stream_destroy(hb_stream s) {
  if (s == nullptr) return HB_OK;
  hipError_t err = hipStreamDestroy((hipStream_t)s);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipStreamDestroy");
}

int hb_stream_sync(hb_stream s) {
  hipError_t err = hipStreamSynchronize(hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipStreamSynchronize");
}

int hb_device_sync(void) {
  hipError_t err = hipDeviceSynchronize();
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipDeviceSynchronize");
}

int hb_event_create(hb_event *e) {
  if (e == nullptr) return hb_invalid("hb_event_create out");
  hipEvent_t ev = nullptr;
  hipError_t err = hipEventCreate(&ev);
  if (err != hipSuccess) return hb_fail(err, "hipEventCreate");
  *e = (hb_event)ev;
  return HB_OK;
}

int hb_event_destroy(hb_event e) {
  if (e == nullptr) return HB_OK;
  hipError_t err = hipEventDestroy((hipEvent_t)e);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipEventDestroy");
}

int hb_event_record(hb_event e, hb_stream s) {
  hipError_t err = hipEventRecord((hipEvent_t)e, hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipEventRecord");
}

int hb_event_sync(hb_event e) {
  hipError_t err = hipEventSynchronize((hipEvent_t)e);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipEventSynchronize");
}

int hb_event_elapsed_ms(float *ms, hb_event start, hb_event stop) {
  if (ms == nullptr) return hb_invalid("hb_event_elapsed_ms out");
  hipError_t err = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipEventElapsedTime");
}

// Stream capture into a HIP graph (relaxed mode: host-side library calls
// made while capturing, such as attribute queries, stay legal).
int hb_graph_begin(hb_stream s) {
  hipStream_t st = hb_resolve_stream(s);
  if (st == nullptr) return hb_invalid("hb_graph_begin stream");
  hipError_t err = hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipStreamBeginCapture");
}

int hb_graph_end(hb_graph *g, hb_stream s) {
  if (g == nullptr) return hb_invalid("hb_graph_end out");
  *g = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t err = hipStreamEndCapture(hb_resolve_stream(s), &graph);
  if (err != hipSuccess) return hb_fail(err, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  hipError_t derr = hipGraphDestroy(graph);
  if (err != hipSuccess) return hb_fail(err, "hipGraphInstantiate");
  if (derr != hipSuccess) {
    (void)hipGraphExecDestroy(exec);
    return hb_fail(derr, "hipGraphDestroy");
  }
  *g = (hb_graph)exec;
  return HB_OK;
}

int hb_graph_launch(hb_graph g, hb_stream s) {
  if (g == nullptr) return hb_invalid("hb_graph_launch graph");
  hipError_t err = hipGraphLaunch((hipGraphExec_t)g, hb_resolve_stream(s));
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipGraphLaunch");
}

int hb_graph_destroy(hb_graph g) {
  if (g == nullptr) return HB_OK;
  hipError_t err = hipGraphExecDestroy((hipGraphExec_t)g);
  return err == hipSuccess ? HB_OK : hb_fail(err, "hipGraphExecDestroy");
}

}  // extern "C"
