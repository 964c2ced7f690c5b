// Row copy between the [B, H, S, D] and [B, S, H*D] layouts with a sequence
// offset: the concatenation of a past K/V tensor with a step's new rows
// (kv_concat / kv_copy_block, onnx-rt/src/ops/microsoft.rs:733-792) and the
// head-major reshapes around it (reshape_to_bhsd / reshape_from_bhsd,
// microsoft.rs:660-704), for f32 or bf16 rows. An HBM-bound copy: a thread
// moves one 16-byte chunk of a row (or one element when rows are not
// 16-byte multiples or the buffers not 16-byte aligned); threads walk the
// source in memory order, so reads are contiguous and every row lands as
// one contiguous run.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sai_internal.h"

namespace sai {
namespace {

constexpr int kThreads = 256;

template <int BYTES>
struct Chunk;
template <>
struct Chunk<2> {
  typedef uint16_t type;
};
template <>
struct Chunk<4> {
  typedef uint32_t type;
};
template <>
struct Chunk<16> {
  typedef uint4 type;
};

template <int BYTES>
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(const CopyRowsArgs a) {
  typedef typename Chunk<BYTES>::type C;
  const uint64_t gi = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gi >= a.total) return;
  const uint64_t row = gi / (uint64_t)a.chunks;
  const uint32_t c = (uint32_t)(gi - row * (uint64_t)a.chunks);
  const uint64_t H = (uint64_t)a.heads, S = (uint64_t)a.seq;
  uint64_t b, h, s;
  if (a.src_layout == 0) {  // (b, h, s)
    s = row % S;
    const uint64_t q = row / S;
    h = q % H;
    b = q / H;
  } else {  // (b, s, h)
    h = row % H;
    const uint64_t q = row / H;
    s = q % S;
    b = q / S;
  }
  const uint64_t ds = (uint64_t)a.dst_offset + s, DS = (uint64_t)a.dst_seq;
  const uint64_t drow = a.dst_layout == 0 ? (b * H + h) * DS + ds : (b * DS + ds) * H + h;
  const C* src = reinterpret_cast<const C*>(a.src) + row * (uint64_t)a.chunks + c;
  C* dst = reinterpret_cast<C*>(a.dst) + drow * (uint64_t)a.chunks + c;
  *dst = *src;
}

__global__ __launch_bounds__(kThreads) void fill_i32_kernel(int32_t* p, uint32_t n, int32_t v) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

hipError_t launch_fill_i32(int32_t* p, size_t n, int32_t v, hipStream_t st) {
  if (n == 0) return hipSuccess;
  if (n > 0xFFFFFFFFull - kThreads) return hipErrorInvalidValue;
  const dim3 g((uint32_t)((n + kThreads - 1) / kThreads)), t(kThreads);
  hipLaunchKernelGGL(fill_i32_kernel, g, t, 0, st, p, (uint32_t)n, v);
  return hipGetLastError();
}

hipError_t launch_copy_rows(const CopyRowsArgs& a, int chunk_bytes, hipStream_t st) {
  if (a.total == 0) return hipSuccess;
  const uint64_t blocks = (a.total + kThreads - 1) / kThreads;
  if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
  const dim3 g((uint32_t)blocks), t(kThreads);
  switch (chunk_bytes) {
    case 16: hipLaunchKernelGGL(copy_rows_kernel<16>, g, t, 0, st, a); break;
    case 4: hipLaunchKernelGGL(copy_rows_kernel<4>, g, t, 0, st, a); break;
    case 2: hipLaunchKernelGGL(copy_rows_kernel<2>, g, t, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sai
