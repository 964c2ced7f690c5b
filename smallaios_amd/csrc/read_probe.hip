// Streaming-read probe: the HBM read rate a plain kernel reaches on this
// device, measured beside the decode kernel so that its roofline fraction can
// be read against an achievable ceiling as well as the 8 TB/s spec value.
// Built into its own library (libsai_read_probe.so); not part of the C ABI of
// the attention path.
//
// Each workgroup streams a contiguous slice of the buffer with 16-byte
// non-temporal loads, UNROLL loads in flight per lane, and writes the xor of
// what it read to sink[blockIdx.x] (so the loads cannot be dropped). Every
// index stays below the buffer's 16-byte count.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const v4u* __restrict__ in,
                                                               size_t n16, size_t per_wg,
                                                               unsigned* __restrict__ sink) {
  const size_t begin = (size_t)blockIdx.x * per_wg;
  const size_t end = begin + per_wg < n16 ? begin + per_wg : n16;
  v4u acc = {0u, 0u, 0u, 0u};
  size_t i = begin + threadIdx.x;
  for (; i + (size_t)(kUnroll - 1) * kThreads < end; i += (size_t)kUnroll * kThreads) {
    v4u v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(in + i + u * kThreads);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  for (; i < end; i += kThreads) acc ^= in[i];
  unsigned x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
  __shared__ unsigned sm[kThreads / 64];
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned y = 0;
    for (int w = 0; w < kThreads / 64; ++w) y ^= sm[w];
    sink[blockIdx.x] = y;
  }
}

}  // namespace

// Reads `bytes` (a multiple of 16) of device memory `buf` with `workgroups`
// workgroups, `warmup` untimed then `reps` timed back-to-back launches on
// `stream`; sink: device u32[workgroups]. Writes the mean microseconds per
// launch (HIP events around the timed launches). Returns 0, or a hipError_t.
extern "C" __attribute__((visibility("default"))) int sai_probe_stream_read(
    const void* buf, size_t bytes, int workgroups, int warmup, int reps, void* sink,
    void* stream, float* us_per_launch) {
  if (!buf || !sink || !us_per_launch || bytes % 16 != 0 || workgroups <= 0 || reps <= 0 ||
      warmup < 0)
    return (int)hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  const size_t per_wg = (n16 + (size_t)workgroups - 1) / (size_t)workgroups;
  const hipStream_t st = (hipStream_t)stream;
  auto launch = [&]() {
    hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(kThreads), 0, st,
                       (const v4u*)buf, n16, per_wg, (unsigned*)sink);
    return hipGetLastError();
  };
  for (int i = 0; i < warmup; ++i)
    if (hipError_t e = launch(); e != hipSuccess) return (int)e;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, st);
  for (int i = 0; i < reps && e == hipSuccess; ++i) e = launch();
  if (e == hipSuccess) e = hipEventRecord(e1, st);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (e != hipSuccess) return (int)e;
  *us_per_launch = ms * 1000.0f / (float)reps;
  return 0;
}
