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

namespace {

// One copy of plh_copy2d_batch_async in units of the launch's unit type.
struct Copy2D {
  const uint8_t* src;
  uint8_t* dst;
  uint64_t spitch, dpitch;
  uint32_t row_units, units;  // units per row, units in all (< 2^31)
};

struct Copy2DBatch {
  Copy2D c[4];
};

// blockIdx.y picks the copy (the same for the whole workgroup); the x
// workgroups stride over its units.  Stores to pinned host memory go out over
// PCIe and are visible to the host once the stream has been synchronised.
template <typename U>
__global__ __launch_bounds__(256) void copy2d_batch_kernel(Copy2DBatch b) {
  const Copy2D& c = b.c[blockIdx.y];
  const uint32_t stride = gridDim.x * 256u;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < c.units; u += stride) {
    const uint32_t row = u / c.row_units, col = u - row * c.row_units;
    *reinterpret_cast<U*>(c.dst + row * c.dpitch + (uint64_t)col * sizeof(U)) =
        *reinterpret_cast<const U*>(c.src + row * c.spitch + (uint64_t)col * sizeof(U));
  }
}

}  // namespace

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

int plh_memcpy2d_htod(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                      size_t height) {
  if (height == 0 || width == 0) return 0;
  if (check_hip(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyHostToDevice,
                                 g_ctx.stream),
                "htod 2d"))
    return -1;
  return check_hip(hipStreamSynchronize(g_ctx.stream), "htod 2d sync");
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

int plh_copy2d_batch_async(const plh_copy2d* copies, int n) {
  if (!g_ctx.stream) {
    set_error("plh_copy2d_batch_async: library not initialised");
    return -1;
  }
  if (!copies || n < 1 || n > 4) {
    set_error("plh_copy2d_batch_async: %d copies (1..4 taken)", copies ? n : 0);
    return -1;
  }
  const plh_copy2d* live[4];
  int m = 0;
  uintptr_t bits = 0;  // every address, width and used pitch: their common alignment
  for (int i = 0; i < n; ++i) {
    const plh_copy2d& c = copies[i];
    if (c.width == 0 || c.height == 0) continue;
    if (!c.dst || !c.src) {
      set_error("plh_copy2d_batch_async: copy %d has a null pointer", i);
      return -1;
    }
    if (c.dpitch < c.width || c.spitch < c.width) {
      set_error("plh_copy2d_batch_async: copy %d has a pitch below its width", i);
      return -1;
    }
    if (c.width > (1ull << 31) || c.height > (1ull << 31)) {
      set_error("plh_copy2d_batch_async: copy %d is too large", i);
      return -1;
    }
    bits |= (uintptr_t)c.dst | (uintptr_t)c.src | c.width;
    if (c.height > 1) bits |= c.dpitch | c.spitch;
    live[m++] = &c;
  }
  if (m == 0) return 0;
  const size_t unit = (bits & 15) == 0 ? 16 : (bits & 3) == 0 ? 4 : 1;
  Copy2DBatch b{};
  uint32_t blocks = 1;
  for (int i = 0; i < m; ++i) {
    const size_t units = live[i]->width / unit * live[i]->height;
    if (units >= (1ull << 31)) {
      set_error("plh_copy2d_batch_async: copy of %zu units of %zu bytes is too large", units,
                unit);
      return -1;
    }
    b.c[i] = Copy2D{(const uint8_t*)live[i]->src, (uint8_t*)live[i]->dst, live[i]->spitch,
                    live[i]->dpitch, (uint32_t)(live[i]->width / unit), (uint32_t)units};
    const size_t need = (units + 255) / 256;
    if (need > blocks) blocks = need > 512 ? 512 : (uint32_t)need;
  }
  const dim3 grid(blocks, (unsigned)m);
  if (unit == 16)
    hipLaunchKernelGGL(copy2d_batch_kernel<uint4>, grid, dim3(256), 0, g_ctx.stream, b);
  else if (unit == 4)
    hipLaunchKernelGGL(copy2d_batch_kernel<uint32_t>, grid, dim3(256), 0, g_ctx.stream, b);
  else
    hipLaunchKernelGGL(copy2d_batch_kernel<uint8_t>, grid, dim3(256), 0, g_ctx.stream, b);
  return check_hip(hipGetLastError(), "copy2d_batch_kernel");
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
