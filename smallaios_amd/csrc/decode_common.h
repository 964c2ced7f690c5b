// Device helpers shared by the int8 and int4 decode kernels: lane-group
// reductions, the hi/lo pair swap, vector loads of a Q chunk, RoPE of one
// element, and the (sequence, split) mapping of a decode workgroup.
//
// Wave layout used by both kernels: lane = r + 16 g (r = lane & 15 is the
// MFMA row/column index, g = lane >> 4 the lane group, i.e. the page of the
// current 64-token tile).
#pragma once

#include "sai_internal.h"

namespace sai {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMaxSplitPages = 1024;  // split_tokens <= 16384 (page ids staged in LDS)

// RoPE of one element; `first` = this element is x0 of its pair. Both
// products are rounded on their own and the select picks the sign of the
// second, so x0: c*x0 - s*x1 and x1: s*x0 + c*x1 (== c*x1 + s*x0) without a
// branch per lane.
__device__ __forceinline__ float rope_elem(float c, float s, float own, float partner,
                                           bool first) {
#pragma clang fp contract(off)
  const float a = c * own;
  const float b = s * partner;
  return a + (first ? -b : b);
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// exchange with the neighbouring lane: quad_perm(1,0,3,2)
__device__ __forceinline__ int swap_pair(int v) {
  return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}

// max / sum over the four lane groups (lanes r, r+16, r+32, r+48)
__device__ __forceinline__ float xgroup_max(float v) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xgroup_sum(float v) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16 consecutive elements (f32 or bf16) starting at element `off`; the
// offset is a multiple of 16 and the row 32-byte aligned.
__device__ __forceinline__ void load16(const void* base, size_t off, int dtype, float (&x)[16]) {
  if (dtype == kDtypeBf16) {
    const uint4* p = (const uint4*)((const uint16_t*)base + off);
    const uint4 a = p[0], b = p[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    const float4* p = (const float4*)((const float*)base + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = p[i];
      x[4 * i] = v.x, x[4 * i + 1] = v.y, x[4 * i + 2] = v.z, x[4 * i + 3] = v.w;
    }
  }
}

// (sequence, split) of a decode workgroup. Uniform split count: direct
// mapping; otherwise a prefix scan over the per-sequence split counts of
// seq_lens[b] + pending tokens. Returns b = -1 past the last work item.
__device__ __forceinline__ void decode_work_item(const DecodeParams& p, int work, int lane, int& b,
                                                 int& split, int& nsplit, int& split_base) {
  b = -1;
  split = nsplit = split_base = 0;
  if (p.uniform_nsplit > 0) {
    nsplit = p.uniform_nsplit;
    b = work / nsplit;
    split = work - b * nsplit;
    split_base = b * nsplit;
    return;
  }
  int base = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) {
    const int bi = c0 + lane;
    const int Lb = bi < p.batch ? p.seq_lens[bi] + p.pending : 0;
    const int n = (Lb - window_origin(Lb, p.window) + p.split_tokens - 1) / p.split_tokens;
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const int total = __shfl(incl, 63, 64);
    if (work < base + total) {
      const unsigned long long m = __ballot(base + incl > work);
      const int first = __ffsll((long long)m) - 1;
      b = c0 + first;
      split_base = base + __shfl(incl - n, first, 64);
      nsplit = __shfl(n, first, 64);
      split = work - split_base;
      return;
    }
    base += total;
  }
}



}  // namespace sai
