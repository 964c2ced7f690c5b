// One (token, kv head) row of the int8 KV append, done by one wave64: RoPE
// on K, absolute maximum, scale, codes, stores into the page block. Shared by
// the standalone append kernel and the fused decode step so both produce the
// same bits.
//
// Bit-exactness with the reference's Rust f32 semantics:
//   * RoPE is `c*x0 - s*x1`, `s*x0 + c*x1` with every product rounded on its
//     own (contraction is off inside these functions);
//   * x / s is the IEEE correctly rounded division (hipcc
//     -fhip-fp32-correctly-rounded-divide-sqrt);
//   * round_half_even(x) == rintf(x) for every f32 once clamped to the int8
//     code range (checked exhaustively on the CPU by the test suite);
//   * float -> int conversions restate Rust's saturating `as` casts.
#pragma once

#include "sai_internal.h"

namespace sai {

// RoPE of one element. `first` = this element is x0 of its pair.
// Reference: rotate_rope_block, onnx-rt/src/ops/microsoft.rs:137-160.
__device__ __forceinline__ float rope_pair_elem(float c, float s, float own, float partner,
                                                bool first) {
#pragma clang fp contract(off)
  return first ? (c * own - s * partner) : (s * partner + c * own);
}

// x[j] = element lane + 64*j of the row; rotates in place at position `pos`.
template <int D>
__device__ __forceinline__ void rope_row_wave(float (&x)[D / 64], int lane, int pos,
                                              const float* __restrict__ cos_cache,
                                              const float* __restrict__ sin_cache,
                                              bool interleaved) {
  constexpr int J = D / 64;
  constexpr int HALF = D / 2;
  float xp[J];
  if (interleaved) {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = __shfl_xor(x[j], 1, 64);
  } else if constexpr (HALF >= 64) {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = x[j ^ (HALF / 64)];
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = __shfl_xor(x[j], HALF, 64);
  }
  const float* cr = cos_cache + (size_t)pos * HALF;
  const float* sr = sin_cache + (size_t)pos * HALF;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    int i;
    bool first;
    if (interleaved) {
      i = e >> 1;
      first = (e & 1) == 0;
    } else {
      first = e < HALF;
      i = first ? e : e - HALF;
    }
    x[j] = rope_pair_elem(cr[i], sr[i], x[j], xp[j], first);
  }
}

// Quantise one row (int8, symmetric, per row) and store it into the page
// block: K token-major (which == 0) or V dim-major (which == 1).
template <int D>
__device__ __forceinline__ void quant_store_row_int8(float (&x)[D / 64], int lane, uint8_t* blk,
                                                     int slot, int which) {
#pragma clang fp contract(off)
  constexpr int J = D / 64;
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) a = fmaxf(a, fabsf(x[j]));
  a = wave_max(a);
  const float sc = (a > 0.0f) ? a / 127.0f : 1.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int32_t q = sat_i32(rintf(x[j] / sc));
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    const int e = lane + 64 * j;
    if (which == 0)
      blk[(size_t)slot * D + e] = (uint8_t)(int8_t)q;
    else
      blk[(size_t)16 * D + (size_t)e * 16 + slot] = (uint8_t)(int8_t)q;
  }
  if (lane == 0) ((float*)(blk + 32 * D + 64 * which))[slot] = sc;
}

// Full K+V append of one (token, kv head) row. k_row / v_row point at the
// row's D elements (f32 or bf16).
template <int D>
__device__ __forceinline__ void append_row_int8(const void* k_row, const void* v_row, int dtype,
                                                int lane, int pos, uint8_t* blk, int slot,
                                                int do_rotary, bool interleaved,
                                                const float* cos_cache, const float* sin_cache) {
  constexpr int J = D / 64;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    float x[J];
    const void* in = which == 0 ? k_row : v_row;
#pragma unroll
    for (int j = 0; j < J; ++j) x[j] = load_elem(in, lane + 64 * j, dtype);
    if (which == 0 && do_rotary) rope_row_wave<D>(x, lane, pos, cos_cache, sin_cache, interleaved);
    quant_store_row_int8<D>(x, lane, blk, slot, which);
  }
}

}  // namespace sai
