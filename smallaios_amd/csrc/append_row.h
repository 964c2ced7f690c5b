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
// Branch-free: both products rounded on their own, then a - b for x0 and
// a + b (== s*x0 + c*x1, IEEE addition commutes) for x1.
__device__ __forceinline__ float rope_pair_elem(float c, float s, float own, float partner,
                                                bool first) {
#pragma clang fp contract(off)
  const float a = c * own;
  const float b = s * partner;
  return a + (first ? -b : b);
}

// Stored dim of a row held by lane `lane` as its element j. Up to head_dim
// 256 that is lane + 64 j. At the stored width 192 (head_dim 168) element 0
// is dim lane and element 1 its split-half partner lane + 96, while element 2
// is dim 64 + lane on lanes 0-31 and 128 + lane on lanes 32-63 (dims 64-95
// and 160-191), whose partners are 32 lanes apart.
template <int D>
__device__ __forceinline__ int row_elem(int lane, int j) {
  if constexpr (D == 192)
    return j == 0 ? lane : (j == 1 ? lane + 96 : (lane < 32 ? 64 + lane : 128 + lane));
  else
    return lane + 64 * j;
}

// x[j] = element j of the row (row_elem); rotates in place at position `pos`
// with tables of kLogicalDim<D> / 2 entries per position. Padding dims stay 0.
// The cos / sin loads come first so that they overlap the row's own loads.
template <int D>
__device__ __forceinline__ void rope_row_wave(float (&x)[D / 64], int lane, int pos,
                                              const float* __restrict__ cos_cache,
                                              const float* __restrict__ sin_cache,
                                              bool interleaved) {
  constexpr int J = D / 64;
  constexpr int HALF = D / 2;
  constexpr int HL = kLogicalDim<D> / 2;  // table entries per position
  const float* cr = cos_cache + (size_t)pos * HL;
  const float* sr = sin_cache + (size_t)pos * HL;
  float c[J], s[J];
  bool first[J], pad[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = row_elem<D>(lane, j);
    const int el = logical_dim<D>(e);
    first[j] = interleaved ? (e & 1) == 0 : e < HALF;
    pad[j] = el < 0;
    const int i = pad[j] ? 0 : (interleaved ? (el >> 1) : (first[j] ? e : e - HALF));
    c[j] = cr[i];
    s[j] = sr[i];
  }
  float xp[J];
  if (interleaved) {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = __shfl_xor(x[j], 1, 64);
  } else if constexpr (D == 192) {
    xp[0] = x[1];
    xp[1] = x[0];
    xp[2] = __shfl_xor(x[2], 32, 64);
  } else if constexpr (HALF >= 64) {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = x[j ^ (HALF / 64)];
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) xp[j] = __shfl_xor(x[j], HALF, 64);
  }
#pragma unroll
  for (int j = 0; j < J; ++j)
    x[j] = pad[j] ? 0.0f : rope_pair_elem(c[j], s[j], x[j], xp[j], first[j]);
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
    const int e = row_elem<D>(lane, j);
    if (which == 0)
      blk[(size_t)slot * D + e] = (uint8_t)(int8_t)q;
    else
      blk[(size_t)16 * D + (size_t)e * 16 + slot] = (uint8_t)(int8_t)q;
  }
  if (lane == 0) ((float*)(blk + 32 * D + 64 * which))[slot] = sc;
}

// Full K+V append of one (token, kv head) row. k_row / v_row point at the
// row's kLogicalDim<D> elements (f32 or bf16); padding dims are stored as 0.
// Every load is issued before the first store, so the row costs one memory
// round trip.
template <int D>
__device__ __forceinline__ void append_row_int8(const void* k_row, const void* v_row, int dtype,
                                                int lane, int pos, uint8_t* blk, int slot,
                                                int do_rotary, bool interleaved,
                                                const float* cos_cache, const float* sin_cache) {
  constexpr int J = D / 64;
  float xk[J], xv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int el = logical_dim<D>(row_elem<D>(lane, j));
    const int ec = el < 0 ? 0 : el;
    xk[j] = load_elem(k_row, ec, dtype);
    xv[j] = load_elem(v_row, ec, dtype);
    if (el < 0) xk[j] = xv[j] = 0.0f;
  }
  if (do_rotary) rope_row_wave<D>(xk, lane, pos, cos_cache, sin_cache, interleaved);
  quant_store_row_int8<D>(xk, lane, blk, slot, 0);
  quant_store_row_int8<D>(xv, lane, blk, slot, 1);
}

// int4 code of element x of a group of 32 = one half-wave (lanes 0-31 /
// 32-63): min/max over the group, scale (max-min)/15 (1.0 for an empty range)
// and zero point min stored as binary16 and used as stored, code =
// min(round_half_away((x - z)/s) as u32, 15) (onnx-rt/src/kv_compression.rs:223-253).
__device__ __forceinline__ void quant_int4_elem(float x, uint32_t& q, uint16_t& s16,
                                                uint16_t& z16) {
#pragma clang fp contract(off)
  // group of 32 = one half-wave (lanes 0-31 / 32-63) for each j
  // NaN never wins a `<` / `>` comparison in the reference loop
  float mn = (x != x) ? INFINITY : x;
  float mx = (x != x) ? -INFINITY : x;
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) {
    const float omn = __shfl_xor(mn, off, 64);
    const float omx = __shfl_xor(mx, off, 64);
    // `if v < min { min = v }` ignores NaN, like fminf/fmaxf
    mn = fminf(mn, omn);
    mx = fmaxf(mx, omx);
  }
  if (mn == 0.0f) {
    // The scan keeps the first of equal minima, so a zero minimum has the
    // sign of the group's first zero in dim order (lane order; the stored
    // binary16 zero point keeps it). All 32 lanes of the group are here.
    const uint64_t zb = __ballot(x == 0.0f);
    const int base = (int)__lane_id() & 32;
    mn = __shfl(x, base + __builtin_ctz((uint32_t)(zb >> base)), 64);
  }
  const float range = mx - mn;
  const float scale = (range > 0.0f) ? range / 15.0f : 1.0f;
  const _Float16 hs = (_Float16)scale;  // v_cvt_f16_f32, round to nearest even
  const _Float16 hz = (_Float16)mn;
  const float sf = (float)hs;
  const float zf = (float)hz;
  uint32_t v = 0u;
  if (sf > 0.0f) {
    // round_f32 of onnx-rt/src/kv_compression.rs:27-37, then `as u32`
    const float t = (x - zf) / sf;
    const float tr = (float)sat_i32(t);
    const float fr = t - tr;
    const float rr = (fr >= 0.5f) ? tr + 1.0f : ((fr <= -0.5f) ? tr - 1.0f : tr);
    v = sat_u32(rr);
  }
  q = v < 15u ? v : 15u;
  s16 = __builtin_bit_cast(uint16_t, hs);
  z16 = __builtin_bit_cast(uint16_t, hz);
}

// Full K+V append of one (token, kv head) row into an int4 page block, one
// wave (head_dim 64, 128 or 256: element lane + 64 j, a group of 32 = a half-wave).
// K is packed LSB-first along D; V is dim-major and shares each byte with the
// neighbouring slot, whose nibble is kept (read-modify-write; the caller
// guarantees no other wave writes that byte concurrently). Every load is
// issued before the first store.
template <int D>
__device__ __forceinline__ void append_row_int4(const void* k_row, const void* v_row, int dtype,
                                                int lane, int pos, uint8_t* blk, int slot,
                                                int do_rotary, bool interleaved,
                                                const float* cos_cache, const float* sin_cache) {
  static_assert(D == 64 || D == 128 || D == 256, "int4 row append: head_dim 64, 128 or 256");
  constexpr int NG = D / 32;
  constexpr int J = D / 64;
  float xk[J], xv[J];
  uint8_t* vdst[J];
  uint8_t vcur[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    xk[j] = load_elem(k_row, e, dtype);
    xv[j] = load_elem(v_row, e, dtype);
    vdst[j] = blk + (size_t)8 * D + (size_t)e * 8 + (slot >> 1);
    vcur[j] = *vdst[j];
  }
  if (do_rotary) rope_row_wave<D>(xk, lane, pos, cos_cache, sin_cache, interleaved);
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    uint16_t* sz = (uint16_t*)(blk + 16 * D + 64 * NG * which) + (size_t)slot * NG * 2;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      uint32_t q;
      uint16_t s16, z16;
      quant_int4_elem(which == 0 ? xk[j] : xv[j], q, s16, z16);
      const int e = lane + 64 * j;
      if ((lane & 31) == 0) {
        sz[(e / 32) * 2 + 0] = s16;
        sz[(e / 32) * 2 + 1] = z16;
      }
      if (which == 0) {
        const uint32_t other = (uint32_t)__shfl_xor((int)q, 1, 64);
        if ((lane & 1) == 0) blk[(size_t)slot * (D / 2) + e / 2] = (uint8_t)(q | (other << 4));
      } else {
        *vdst[j] = (slot & 1) ? (uint8_t)((vcur[j] & 0x0F) | (q << 4))
                              : (uint8_t)((vcur[j] & 0xF0) | q);
      }
    }
  }
}

}  // namespace sai
