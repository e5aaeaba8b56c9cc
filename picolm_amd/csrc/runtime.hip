// runtime.hip -- device selection, stream, memory, events and the workspace
// behind the C ABI declared in include/picolm_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "picolm_hip.h"
#include "plh_internal.h"

namespace plh {

static Context g_ctx;
static char g_err[512] = "";

Context& ctx() { return g_ctx; }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  set_error("%s: %s", what, hipGetErrorString(e));
  fprintf(stderr, "picolm_hip: %s\n", g_err);
  return -1;
}

int grow_buffer(void** p, size_t* bytes, size_t want, const char* what) {
  Context& c = g_ctx;
  if (*p) {
    if (c.n_retired == c.cap_retired) {
      const int cap = c.cap_retired ? 2 * c.cap_retired : 16;
      void** r = (void**)realloc(c.retired, sizeof(void*) * (size_t)cap);
      if (!r) {
        set_error("%s: out of host memory for the retired-buffer list", what);
        return -1;
      }
      c.retired = r;
      c.cap_retired = cap;
    }
    c.retired[c.n_retired++] = *p;
    *p = nullptr;
    *bytes = 0;
  }
  if (check_hip(hipMalloc(p, want), what)) {
    *p = nullptr;
    return -1;
  }
  *bytes = want;
  return 0;
}

int ensure_workspace(size_t bytes) {
  Context& c = g_ctx;
  if (c.ws && c.ws_bytes >= bytes) return 0;
  return grow_buffer(&c.ws, &c.ws_bytes, bytes + bytes / 2, "hipMalloc(workspace)");
}

}  // namespace plh

using namespace plh;

extern "C" {

const char* plh_last_error(void) { return g_err; }

int plh_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int plh_init(int device) {
  Context& c = g_ctx;
  if (c.device == device && c.stream) return 0;
  if (c.stream) plh_shutdown();
  int n = 0;
  if (check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount")) return -1;
  if (device < 0 || device >= n) {
    set_error("plh_init: device %d not present (%d devices)", device, n);
    return -1;
  }
  if (check_hip(hipSetDevice(device), "hipSetDevice")) return -1;
  hipDeviceProp_t prop;
  if (check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) return -1;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    set_error("plh_init: device %d is %s, this library is built for gfx950 only", device,
              prop.gcnArchName);
    return -1;
  }
  // Default-priority stream (no priority games on this hardware).
  if (check_hip(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking), "hipStreamCreate"))
    return -1;
  if (decode_scratch_setup(device)) {
    (void)hipStreamDestroy(c.stream);
    c.stream = nullptr;
    return -1;
  }
  if (check_hip(hipMalloc(&c.decode_ctr, kDecodeCounters * sizeof(unsigned)),
                "hipMalloc(decode counters)") ||
      check_hip(hipMemsetAsync(c.decode_ctr, 0, kDecodeCounters * sizeof(unsigned), c.stream),
                "hipMemsetAsync(decode counters)") ||
      check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize")) {
    if (c.decode_ctr) (void)hipFree(c.decode_ctr);
    (void)hipStreamDestroy(c.stream);
    c = Context();
    return -1;
  }
  c.device = device;
  c.num_cus = prop.multiProcessorCount;
  return 0;
}

void plh_shutdown(void) {
  Context& c = g_ctx;
  if (c.stream) {
    (void)hipStreamSynchronize(c.stream);
    if (c.ws) (void)hipFree(c.ws);
    if (c.pf_ws) (void)hipFree(c.pf_ws);
    if (c.decode_ctr) (void)hipFree(c.decode_ctr);
    for (int i = 0; i < c.n_retired; ++i) (void)hipFree(c.retired[i]);
    (void)hipStreamDestroy(c.stream);
  }
  free(c.retired);
  c = Context();
}

int plh_available(void) { return g_ctx.stream != nullptr; }

void* plh_malloc(size_t bytes) {
  void* p = nullptr;
  if (!g_ctx.stream) {
    set_error("plh_malloc: library not initialised");
    return nullptr;
  }
  if (check_hip(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
  return p;
}

int plh_free(void* p) {
  if (!p) return 0;
  // Work queued on the stream may still use p.
  if (g_ctx.stream && check_hip(hipStreamSynchronize(g_ctx.stream), "hipStreamSynchronize"))
    return -1;
  return check_hip(hipFree(p), "hipFree");
}

int plh_memcpy_htod(void* dst, const void* src, size_t bytes) {
  if (check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx.stream), "htod"))
    return -1;
  return check_hip(hipStreamSynchronize(g_ctx.stream), "htod sync");
}

int plh_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  if (check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx.stream), "dtoh"))
    return -1;
  return check_hip(hipStreamSynchronize(g_ctx.stream), "dtoh sync");
}

int plh_memcpy2d_dtoh(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                      size_t height) {
  if (height == 0 || width == 0) return 0;
  if (check_hip(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToHost,
                                 g_ctx.stream),
                "dtoh 2d"))
    return -1;
  return check_hip(hipStreamSynchronize(g_ctx.stream), "dtoh 2d sync");
}

void* plh_host_alloc(size_t bytes) {
  void* p = nullptr;
  if (check_hip(hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc"))
    return nullptr;
  return p;
}

int plh_host_free(void* p) {
  if (!p) return 0;
  // queued copies may still read or write it
  if (g_ctx.stream && check_hip(hipStreamSynchronize(g_ctx.stream), "hipStreamSynchronize"))
    return -1;
  return check_hip(hipHostFree(p), "hipHostFree");
}

int plh_memcpy_htod_async(void* dst, const void* src, size_t bytes) {
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx.stream),
                   "htod async");
}

int plh_memcpy_dtoh_async(void* dst, const void* src, size_t bytes) {
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx.stream),
                   "dtoh async");
}

int plh_memcpy2d_dtoh_async(void* dst, size_t dpitch, const void* src, size_t spitch,
                            size_t width, size_t height) {
  if (height == 0 || width == 0) return 0;
  return check_hip(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height,
                                    hipMemcpyDeviceToHost, g_ctx.stream),
                   "dtoh 2d async");
}

int plh_memcpy_dtod(void* dst, const void* src, size_t bytes) {
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_ctx.stream), "dtod");
}

int plh_memset(void* dst, int value, size_t bytes) {
  return check_hip(hipMemsetAsync(dst, value, bytes, g_ctx.stream), "memset");
}

int plh_synchronize(void) {
  if (!g_ctx.stream) {
    set_error("plh_synchronize: library not initialised");
    return -1;
  }
  return check_hip(hipStreamSynchronize(g_ctx.stream), "hipStreamSynchronize");
}

void* plh_event_create(void) {
  hipEvent_t e = nullptr;
  if (check_hip(hipEventCreate(&e), "hipEventCreate")) return nullptr;
  return (void*)e;
}

int plh_event_record(void* ev) {
  return check_hip(hipEventRecord((hipEvent_t)ev, g_ctx.stream), "hipEventRecord");
}

float plh_event_elapsed_ms(void* a, void* b) {
  if (check_hip(hipEventSynchronize((hipEvent_t)b), "hipEventSynchronize")) return -1.0f;
  float ms = -1.0f;
  if (check_hip(hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime"))
    return -1.0f;
  return ms;
}

void plh_event_destroy(void* ev) {
  if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}

int plh_capture_begin(void) {
  if (!g_ctx.stream) {
    set_error("plh_capture_begin: library not initialised");
    return -1;
  }
  return check_hip(hipStreamBeginCapture(g_ctx.stream, hipStreamCaptureModeThreadLocal),
                   "hipStreamBeginCapture");
}

void* plh_capture_end(void) {
  hipGraph_t graph = nullptr;
  if (check_hip(hipStreamEndCapture(g_ctx.stream, &graph), "hipStreamEndCapture")) return nullptr;
  hipGraphExec_t exec = nullptr;
  int rc = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  (void)hipGraphDestroy(graph);
  return rc ? nullptr : (void*)exec;
}

int plh_graph_launch(void* exec) {
  return check_hip(hipGraphLaunch((hipGraphExec_t)exec, g_ctx.stream), "hipGraphLaunch");
}

void plh_graph_destroy(void* exec) {
  if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

}  // extern "C"
