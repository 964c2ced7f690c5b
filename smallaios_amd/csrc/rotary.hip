// Standalone rotary embedding (com.microsoft.RotaryEmbedding) and the
// generation of bf16 RoPE tables, for gfx950.
//
// rotary_kernel: an elementwise, HBM-bound pass. Rows of head_dim elements
// are contiguous in both supported layouts ([B, H, S, D] and [B, S, H*D]);
// they differ only in which sequence index a row belongs to, and so in the
// table row its cos/sin come from. One thread handles one item: P rotation
// pairs (or P pass-through elements past rotary_dim when the output is a
// separate buffer) of NH heads of one (b, s) step, loading the step's cos/sin
// once. Vector path: (P, NH) = (8, 2) for bf16 rows (16-byte loads), (4, 4)
// for f32 rows (16-byte loads) -- the fastest of P in {2, 4, 8} x NH in
// {1, 2, 4, 8} on a [2, 2048, 32*128] chunk; scalar path (1, 1) for odd half
// widths or unaligned buffers. Rotation (onnx-rt/src/ops/microsoft.rs:137-160):
//   y0 = c*x0 - s*x1,  y1 = s*x0 + c*x1
// in f32 with every product rounded on its own (no contraction), pairs
// (i, i + rotary_dim/2) or (2i, 2i+1). bf16 outputs round to nearest even
// (onnx-rt/src/tensor.rs:312-329, NaN kept quiet).
//
// Positions travel in the kernel argument block (at most kRotaryTab per
// launch), either one start per sequence (row position = start + s) or one
// per sequence index of a chunk; the host validates every position against
// the table length before launch, so every table row read here exists.
//
// rope_tables_kernel: precompute_rope_tables of
// onnx-rt/src/model_loader/gemma.rs:458-472 with its f32 approximations
// (gemma.rs:480-541): every value is an IEEE f32 operation sequence
// (correctly rounded division, no contraction), so the tables match the
// reference's bit for bit.
#include <hip/hip_runtime.h>

#include <cstdint>

#include <type_traits>

#include "sai_internal.h"

namespace sai {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// f32 -> bf16, round to nearest even; NaN stays a quiet NaN of the same sign
// (onnx-rt/src/tensor.rs:312-329).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  const uint32_t bits = __float_as_uint(v);
  if (v != v) return (uint16_t)((bits >> 16) | 0x0040u);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

template <typename T>
__device__ __forceinline__ float load_elem(const T* p);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t* p) {
  return bf16_bits_to_f32(*p);
}

template <typename T>
__device__ __forceinline__ void store_elem(T* p, float v);
template <>
__device__ __forceinline__ void store_elem<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_elem<uint16_t>(uint16_t* p, float v) {
  *p = f32_to_bf16_bits(v);
}

// N consecutive elements of a row or table, widened to f32.
template <typename T, int N>
struct Vec {
  float v[N];
};

template <int BYTES>
struct Raw;
template <>
struct Raw<2> {
  typedef uint16_t type;
};
template <>
struct Raw<4> {
  typedef uint32_t type;
};
template <>
struct Raw<8> {
  typedef uint2 type;
};
template <>
struct Raw<16> {
  typedef uint4 type;
};
template <>
struct Raw<32> {
  struct type {
    uint4 a, b;
  };
};
template <>
struct Raw<64> {
  struct type {
    uint4 a, b, c, d;
  };
};

// VEC: one load / store of N * sizeof(T) bytes (the caller guarantees that
// alignment); otherwise N element accesses.
template <typename T, int N, bool VEC>
__device__ __forceinline__ Vec<T, N> load_vec(const T* p) {
  Vec<T, N> out;
  if constexpr (VEC) {
    typedef typename Raw<N * sizeof(T)>::type R;
    union {
      R r;
      T e[N];
    } u;
    u.r = *reinterpret_cast<const R*>(p);
#pragma unroll
    for (int j = 0; j < N; ++j) out.v[j] = load_elem<T>(&u.e[j]);
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out.v[j] = load_elem<T>(p + j);
  }
  return out;
}

// Two f32 -> two bf16 in one word (a in the low half), rounded to nearest
// even by v_cvt_pk_bf16_f32 (NaN excepted: see store_vec).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), bf2));
}

template <typename T, int N, bool VEC>
__device__ __forceinline__ void store_vec(T* p, const float (&v)[N]) {
  if constexpr (VEC && std::is_same<T, uint16_t>::value && N % 2 == 0) {
    // bf16 pairs by the conversion instruction; a vector holding a NaN takes
    // f32_to_bf16_bits for every element (a quiet NaN keeping the sign and
    // the high payload bits, as the reference's conversion)
    typedef typename Raw<N * sizeof(T)>::type R;
    union {
      R r;
      uint32_t w[N / 2];
    } u;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      u.w[j] = f32x2_to_bf16x2(v[2 * j], v[2 * j + 1]);
      nan = nan || v[2 * j] != v[2 * j] || v[2 * j + 1] != v[2 * j + 1];
    }
    if (nan) {
#pragma unroll
      for (int j = 0; j < N / 2; ++j)
        u.w[j] = (uint32_t)f32_to_bf16_bits(v[2 * j]) |
                 ((uint32_t)f32_to_bf16_bits(v[2 * j + 1]) << 16);
    }
    *reinterpret_cast<R*>(p) = u.r;
  } else if constexpr (VEC) {
    typedef typename Raw<N * sizeof(T)>::type R;
    union {
      R r;
      T e[N];
    } u;
#pragma unroll
    for (int j = 0; j < N; ++j) store_elem<T>(&u.e[j], v[j]);
    *reinterpret_cast<R*>(p) = u.r;
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) store_elem<T>(p + j, v[j]);
  }
}

// One work item: pair group `it` (P pairs; or, past rot_items, P
// pass-through elements) of NH consecutive heads of one (b, s) step. The
// step's cos/sin are loaded once for the NH heads, and every head's loads are
// issued before the first store, so a thread keeps 2*NH loads in flight.
// T: element type of x / y (float or bf16 bits), TT: table element type,
// IL: interleaved pairs.
template <typename T, typename TT, bool IL, int P, int NH>
__global__ __launch_bounds__(kThreads) void rotary_kernel(const RotaryArgs a) {
#pragma clang fp contract(off)
  constexpr bool V = P > 1;
  constexpr int XN = IL ? 2 * P : P;  // elements of one load
  const uint32_t gi = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
  if (gi >= a.total) return;
  const uint32_t items = (uint32_t)a.items;
  const uint32_t q = gi / items;
  const uint32_t it = gi - q * items;
  const uint32_t groups = (uint32_t)a.head_groups;
  const uint32_t r = q / groups;  // step (bl, sl)
  const uint32_t hg = q - r * groups;
  const uint32_t ns = (uint32_t)a.ns;
  const uint32_t bl = r / ns;
  const uint32_t sl = r - bl * ns;
  const int64_t b = (int64_t)a.b0 + bl;
  const int64_t s = (int64_t)a.s0 + sl;
  const int h0 = (int)hg * NH;
  const int nh = a.heads - h0 < NH ? a.heads - h0 : NH;
  int64_t row0, hstride;  // row of head h0, rows between consecutive heads
  if (a.layout == 0) {  // rows (b, h, s)
    row0 = (b * a.heads + h0) * a.seq + s;
    hstride = a.seq;
  } else {  // rows (b, s, h)
    row0 = (b * a.seq + s) * a.heads + h0;
    hstride = 1;
  }
  const int64_t hs = hstride * a.head_dim;
  const T* xr = reinterpret_cast<const T*>(a.x) + row0 * a.head_dim;
  T* yr = reinterpret_cast<T*>(a.y) + row0 * a.head_dim;

  if (it >= (uint32_t)a.rot_items) {  // elements past rotary_dim, copied as they are
    const int e = a.rot_dim + (int)(it - (uint32_t)a.rot_items) * P;
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      if (j < nh) {
        if constexpr (V) {
          typedef typename Raw<P * sizeof(T)>::type R;
          *reinterpret_cast<R*>(yr + j * hs + e) = *reinterpret_cast<const R*>(xr + j * hs + e);
        } else {
          yr[j * hs + e] = xr[j * hs + e];
        }
      }
    }
    return;
  }
  const int pos = a.mode == 0 ? a.tab[bl] + (int)s : a.tab[sl];
  const int e = (int)it * P;  // first pair of this item
  const int64_t t = (int64_t)pos * a.cache_cols + e;
  const Vec<TT, P> c = load_vec<TT, P, V>(reinterpret_cast<const TT*>(a.cos) + t);
  const Vec<TT, P> sn = load_vec<TT, P, V>(reinterpret_cast<const TT*>(a.sin) + t);
  const int half = a.rot_dim >> 1;
  // first element of each load: interleaved rows hold the item's pairs
  // contiguously; split-half rows hold x0 at e and x1 at half + e
  const int o0 = IL ? 2 * e : e;
  const int o1 = half + e;
  Vec<T, XN> x0[NH];
  Vec<T, P> x1[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    if (j < nh) {
      x0[j] = load_vec<T, XN, V>(xr + j * hs + o0);
      if (!IL) x1[j] = load_vec<T, P, V>(xr + j * hs + o1);
    }
  }
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    if (j < nh) {
      if (IL) {
        float y[2 * P];
#pragma unroll
        for (int k = 0; k < P; ++k) {
          const float u = x0[j].v[2 * k], w = x0[j].v[2 * k + 1];
          const float a0 = c.v[k] * u, b0 = sn.v[k] * w;
          const float a1 = sn.v[k] * u, b1 = c.v[k] * w;
          y[2 * k] = a0 - b0;
          y[2 * k + 1] = a1 + b1;
        }
        store_vec<T, 2 * P, V>(yr + j * hs + o0, y);
      } else {
        float y0[P], y1[P];
#pragma unroll
        for (int k = 0; k < P; ++k) {
          const float a0 = c.v[k] * x0[j].v[k], b0 = sn.v[k] * x1[j].v[k];
          const float a1 = sn.v[k] * x0[j].v[k], b1 = c.v[k] * x1[j].v[k];
          y0[k] = a0 - b0;
          y1[k] = a1 + b1;
        }
        store_vec<T, P, V>(yr + j * hs + o0, y0);
        store_vec<T, P, V>(yr + j * hs + o1, y1);
      }
    }
  }
}

// ---- RoPE tables (gemma.rs:458-541) ------------------------------------
// f32 constants of Rust's core::f32::consts, rounded to f32 by the compiler.
constexpr float kLn2 = 0.693147180559945309417232121458176568f;
constexpr float kLog2E = 1.44269504088896340735992468100189214f;
constexpr float kTau = 6.28318530717958647692528676655900577f;
constexpr float kPi = 3.14159265358979323846264338327950288f;
constexpr float kHalfPi = 1.57079632679489661923132169163975144f;

// `x as i32 as f32`, then one step down below x (libm_floor_f32, gemma.rs:517-524).
__device__ __forceinline__ float floor_approx(float x) {
  const float xi = (float)(int)x;  // v_cvt_i32_f32 saturates and maps NaN to 0, like Rust's `as`
  return x < xi ? xi - 1.0f : xi;
}

// ln via exponent split and the atanh series to y^7 (gemma.rs:485-500).
__device__ __forceinline__ float ln_approx(float x) {
#pragma clang fp contract(off)
  if (x <= 0.0f) return -__builtin_huge_valf();
  const uint32_t bits = __float_as_uint(x);
  const int e = (int)((bits >> 23) & 0xFFu) - 127;
  const float m = __uint_as_float((bits & 0x7FFFFFu) | (127u << 23));
  const float y = (m - 1.0f) / (m + 1.0f);
  const float y2 = y * y;
  const float t3 = y2 * y / 3.0f;
  const float t5 = y2 * y2 * y / 5.0f;
  const float t7 = y2 * y2 * y2 * y / 7.0f;
  const float ln_m = 2.0f * (y + t3 + t5 + t7);
  return (float)e * kLn2 + ln_m;
}

// exp via 2^k and a degree-6 Taylor polynomial on the remainder (gemma.rs:502-513).
__device__ __forceinline__ float exp_approx(float x) {
#pragma clang fp contract(off)
  const float y = x * kLog2E;
  const int k = (int)floor_approx(y);
  const float r = x - (float)k * kLn2;
  const float e_r =
      1.0f +
      r * (1.0f + r * (0.5f + r * (1.0f / 6.0f + r * (1.0f / 24.0f + r * (1.0f / 120.0f)))));
  const int kc = k < -126 ? -126 : (k > 127 ? 127 : k);
  const float two_k = __uint_as_float((uint32_t)(kc + 127) << 23);
  return e_r * two_k;
}

// sin after reduction to [-pi, pi], Taylor to y^9 (gemma.rs:526-535).
__device__ __forceinline__ float sin_approx(float x) {
#pragma clang fp contract(off)
  float y = x - floor_approx(x / kTau) * kTau;
  if (y > kPi) y -= kTau;
  const float y2 = y * y;
  return y * (1.0f -
              y2 * (1.0f / 6.0f -
                    y2 * (1.0f / 120.0f - y2 * (1.0f / 5040.0f - y2 * (1.0f / 362880.0f)))));
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void rope_tables_kernel(float theta, uint32_t n,
                                                               uint32_t half, void* cos_out,
                                                               void* sin_out) {
#pragma clang fp contract(off)
  const uint32_t idx = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
  if (idx >= n) return;
  const uint32_t pos = idx / half;
  const uint32_t i = idx - pos * half;
  const float head_dim = (float)(half * 2u);
  const float ex = (2.0f * (float)i) / head_dim;
  const float inv_freq = 1.0f / exp_approx(ex * ln_approx(theta));
  const float angle = (float)pos * inv_freq;
  const uint16_t cb = f32_to_bf16_bits(sin_approx(angle + kHalfPi));
  const uint16_t sb = f32_to_bf16_bits(sin_approx(angle));
  if (BF16) {
    reinterpret_cast<uint16_t*>(cos_out)[idx] = cb;
    reinterpret_cast<uint16_t*>(sin_out)[idx] = sb;
  } else {  // the bf16 values widened, as a cast to f32 of the bf16 table gives
    reinterpret_cast<float*>(cos_out)[idx] = bf16_bits_to_f32(cb);
    reinterpret_cast<float*>(sin_out)[idx] = bf16_bits_to_f32(sb);
  }
}

template <typename T, typename TT, bool IL>
hipError_t launch_rotary_p(const RotaryArgs& a, hipStream_t st) {
  const uint32_t blocks = (uint32_t)((a.total + kThreads - 1) / kThreads);
  const dim3 g(blocks), t(kThreads);
  if (a.pairs_per_item == 8)
    hipLaunchKernelGGL((rotary_kernel<T, TT, IL, 8, 2>), g, t, 0, st, a);
  else if (a.pairs_per_item == 4)
    hipLaunchKernelGGL((rotary_kernel<T, TT, IL, 4, 4>), g, t, 0, st, a);
  else
    hipLaunchKernelGGL((rotary_kernel<T, TT, IL, 1, 1>), g, t, 0, st, a);
  return hipGetLastError();
}

template <typename T, typename TT>
hipError_t launch_rotary_t(const RotaryArgs& a, bool interleaved, hipStream_t st) {
  return interleaved ? launch_rotary_p<T, TT, true>(a, st) : launch_rotary_p<T, TT, false>(a, st);
}

}  // namespace

hipError_t launch_rotary(const RotaryArgs& a, bool x_bf16, bool table_bf16, bool interleaved,
                         hipStream_t st) {
  if (a.total == 0) return hipSuccess;
  if (x_bf16)
    return table_bf16 ? launch_rotary_t<uint16_t, uint16_t>(a, interleaved, st)
                      : launch_rotary_t<uint16_t, float>(a, interleaved, st);
  return table_bf16 ? launch_rotary_t<float, uint16_t>(a, interleaved, st)
                    : launch_rotary_t<float, float>(a, interleaved, st);
}

hipError_t launch_rope_tables(float theta, uint32_t max_pos, uint32_t half, bool bf16,
                              void* cos_out, void* sin_out, hipStream_t st) {
  const uint32_t n = max_pos * half;
  if (n == 0) return hipSuccess;
  const uint32_t blocks = (n + kThreads - 1) / kThreads;
  if (bf16)
    hipLaunchKernelGGL(rope_tables_kernel<true>, dim3(blocks), dim3(kThreads), 0, st, theta, n,
                       half, cos_out, sin_out);
  else
    hipLaunchKernelGGL(rope_tables_kernel<false>, dim3(blocks), dim3(kThreads), 0, st, theta, n,
                       half, cos_out, sin_out);
  return hipGetLastError();
}

}  // namespace sai
