// Kernel 1: KV append -- RoPE on K, per-token quantisation, packed stores into
// the paged cache.
//
// One wave64 per (sequence b, new token s, kv head h) row. With head_dim
// D = 64*J each lane owns elements lane + 64*j, so the split-half RoPE pair
// (i, i + D/2) of D = 128 sits in one lane (no cross-lane traffic); D = 64 and
// the interleaved layout fetch their partner with one shuffle. The row's
// absolute maximum (int8) or the group's min/max (int4, 32 lanes per group) are
// wave reductions; max/min are exact, so the reduction order cannot change the
// scale.
// The row arithmetic (and why it is bit-exact with the reference's f32
// semantics) is in append_row.h; this file is also built with
// -ffp-contract=off.
#include "append_row.h"
#include "sai_internal.h"

#pragma clang fp contract(off)

namespace sai {

namespace {

template <int D>
__device__ __forceinline__ void decode_row(const AppendParams& p, long row, int& b, int& s,
                                           int& h) {
  h = (int)(row % p.kv_heads);
  const long bs = row / p.kv_heads;
  s = (int)(bs % p.s_new);
  b = (int)(bs / p.s_new);
}

// ---------------------------------------------------------------- int8 ----
template <int D>
__global__ __launch_bounds__(256) void kv_append_int8_kernel(AppendParams p) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long rows = (long)p.batch * p.s_new * p.kv_heads;
  if (row >= rows) return;
  int b, s, h;
  decode_row<D>(p, row, b, s, h);
  const int pos = p.seq_lens[b] + s;
  const int page = p.page_table[(size_t)b * p.max_pages + pos / kPageTokens];
  uint8_t* blk = p.pool + block_offset(page, h, p.num_pages, block_bytes_int8(D));
  const size_t src = (size_t)row * D;  // [b][s][h][D] == row * D
  const size_t esz = p.dtype == kDtypeBf16 ? 2 : 4;
  append_row_int8<D>((const uint8_t*)p.k + src * esz, (const uint8_t*)p.v + src * esz, p.dtype,
                     lane, pos, blk, pos % kPageTokens, p.do_rotary, p.interleaved != 0,
                     p.cos_cache, p.sin_cache);
}

// ---------------------------------------------------------------- int4 ----
// One wave per (b, token pair, h): the two tokens of a pair share the bytes of
// the dim-major V block, so one wave owns both nibbles of every byte it
// writes. Tokens of the pair outside [seq_len, seq_len + s_new) keep their
// stored nibbles.
template <int D>
__global__ __launch_bounds__(256) void kv_append_int4_kernel(AppendParams p, int pairs_per_seq) {
  constexpr int J = D / 64;
  constexpr int NG = D / 32;
  const int lane = threadIdx.x & 63;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long items = (long)p.batch * pairs_per_seq * p.kv_heads;
  if (item >= items) return;
  const int h = (int)(item % p.kv_heads);
  const long bp = item / p.kv_heads;
  const int pair = (int)(bp % pairs_per_seq);
  const int b = (int)(bp / pairs_per_seq);
  const int start = p.seq_lens[b];
  const int pos0 = (start & ~1) + 2 * pair;  // even position of this pair

  bool fresh[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int s = pos0 + t - start;
    fresh[t] = (s >= 0) && (s < p.s_new);
  }
  if (!fresh[0] && !fresh[1]) return;  // pair past the new tokens: nothing to write
  const int page = p.page_table[(size_t)b * p.max_pages + pos0 / kPageTokens];
  const int slot0 = pos0 % kPageTokens;
  uint8_t* blk = p.pool + block_offset(page, h, p.num_pages, block_bytes_int4(D));

  // new nibble codes of V for (token 0/1 of the pair, element lane + 64j)
  uint32_t vq[2][J];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int pos = pos0 + t;
    const int s = pos - start;
#pragma unroll
    for (int j = 0; j < J; ++j) vq[t][j] = 0u;
    if (!fresh[t]) continue;  // wave-uniform
    const int slot = slot0 + t;
    const size_t src = (((size_t)b * p.s_new + s) * p.kv_heads + h) * D;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      float x[J];
      const void* in = which == 0 ? p.k : p.v;
#pragma unroll
      for (int j = 0; j < J; ++j) x[j] = load_elem(in, src + lane + 64 * j, p.dtype);
      if (which == 0 && p.do_rotary) {
        rope_row_wave<D>(x, lane, pos, p.cos_cache, p.sin_cache, p.interleaved != 0);
      }
      uint16_t* sz = (uint16_t*)(blk + 16 * D + 64 * NG * which) + (size_t)slot * NG * 2;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        uint32_t q;
        uint16_t s16, z16;
        quant_int4_elem(x[j], q, s16, z16);
        const int e = lane + 64 * j;
        if ((lane & 31) == 0) {
          const int gidx = e / 32;
          sz[gidx * 2 + 0] = s16;
          sz[gidx * 2 + 1] = z16;
        }
        if (which == 0) {
          // K row, LSB-first along D: byte e/2 = code(e even) | code(e odd) << 4
          const uint32_t other = (uint32_t)__shfl_xor((int)q, 1, 64);
          if ((lane & 1) == 0) blk[(size_t)slot * (D / 2) + e / 2] = (uint8_t)(q | (other << 4));
        } else {
          vq[t][j] = q;
        }
      }
    }
  }
  // V, dim-major: row e holds 16 slots as 8 bytes, slot 2i in the low nibble.
  const int byte_idx = slot0 >> 1;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    uint8_t* dst = blk + (size_t)8 * D + (size_t)e * 8 + byte_idx;
    uint8_t cur = *dst;
    uint8_t lo = fresh[0] ? (uint8_t)vq[0][j] : (uint8_t)(cur & 0x0F);
    uint8_t hi = fresh[1] ? (uint8_t)vq[1][j] : (uint8_t)(cur >> 4);
    *dst = (uint8_t)(lo | (hi << 4));
  }
}

__global__ void seq_advance_kernel(int32_t* seq_lens, int batch, int pending) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) seq_lens[i] += pending;
}

}  // namespace

hipError_t launch_kv_append(const AppendParams& p, int head_dim, int quant, hipStream_t st) {
  if (quant == kQuantInt8) {
    const long rows = (long)p.batch * p.s_new * p.kv_heads;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (head_dim == 64)
      hipLaunchKernelGGL(kv_append_int8_kernel<64>, grid, dim3(256), 0, st, p);
    else if (head_dim == 128)
      hipLaunchKernelGGL(kv_append_int8_kernel<128>, grid, dim3(256), 0, st, p);
    else if (head_dim == 256)
      hipLaunchKernelGGL(kv_append_int8_kernel<256>, grid, dim3(256), 0, st, p);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (quant == kQuantInt4) {
    // pairs covering positions [start, start + s_new) for any start parity
    const int pairs = p.s_new / 2 + 1;
    const long items = (long)p.batch * pairs * p.kv_heads;
    const dim3 grid((unsigned)((items + 3) / 4));
    if (head_dim == 64)
      hipLaunchKernelGGL(kv_append_int4_kernel<64>, grid, dim3(256), 0, st, p, pairs);
    else if (head_dim == 128)
      hipLaunchKernelGGL(kv_append_int4_kernel<128>, grid, dim3(256), 0, st, p, pairs);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

hipError_t launch_seq_advance(int32_t* seq_lens, int batch, int pending, hipStream_t st) {
  hipLaunchKernelGGL(seq_advance_kernel, dim3((batch + 255) / 256), dim3(256), 0, st, seq_lens,
                     batch, pending);
  return hipGetLastError();
}

}  // namespace sai
