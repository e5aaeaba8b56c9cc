// fp16_ops.hip -- elementwise fp32 -> fp16 conversion with the reference's
// rounding (quant.c:41-78) and an exhaustive-sweep checksum of it.
#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ src,
                                                         uint16_t* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = f16_bits_rha(src[i]);
}

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 27;
  x *= 0x94D049BB133111EBull;
  x ^= x >> 31;
  return x;
}

__global__ __launch_bounds__(256) void f16_checksum_kernel(uint64_t first, uint64_t count,
                                                           unsigned long long* result) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t s = 0;
  for (; i < count; i += stride) {
    uint64_t x = first + i;
    float f = __uint_as_float((uint32_t)x);
    s += ((uint64_t)f16_bits_rha(f) + 1u) * (mix64(x) | 1u);
  }
  // wave reduction, then one atomic per wave (wrap-around sums commute)
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)s, off, 64);
    uint32_t hi = __shfl_xor((uint32_t)(s >> 32), off, 64);
    s += ((uint64_t)hi << 32) | lo;
  }
  if ((threadIdx.x & 63) == 0) atomicAdd(result, (unsigned long long)s);
}

extern "C" int plh_f32_to_f16(const float* src, uint16_t* dst, size_t n) {
  if (!ctx().stream) {
    set_error("plh_f32_to_f16: library not initialised");
    return -1;
  }
  if (n == 0) return 0;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx().stream, src,
                     dst, n);
  return check_hip(hipGetLastError(), "f32_to_f16_kernel");
}

extern "C" int plh_f16_checksum(uint64_t first, uint64_t count, uint64_t* checksum) {
  Context& c = ctx();
  if (!c.stream) {
    set_error("plh_f16_checksum: library not initialised");
    return -1;
  }
  unsigned long long* d_res = nullptr;
  if (check_hip(hipMalloc(&d_res, sizeof *d_res), "hipMalloc")) return -1;
  int rc = check_hip(hipMemsetAsync(d_res, 0, sizeof *d_res, c.stream), "hipMemsetAsync");
  if (!rc) {
    hipLaunchKernelGGL(f16_checksum_kernel, dim3(4096), dim3(256), 0, c.stream, first, count,
                       d_res);
    rc = check_hip(hipGetLastError(), "f16_checksum_kernel");
  }
  unsigned long long h = 0;
  if (!rc) rc = check_hip(hipMemcpyAsync(&h, d_res, sizeof h, hipMemcpyDeviceToHost, c.stream),
                          "dtoh");
  if (!rc) rc = check_hip(hipStreamSynchronize(c.stream), "sync");
  (void)hipFree(d_res);
  if (!rc) *checksum = (uint64_t)h;
  return rc;
}
