// TurboQuant compressed KV cache (CompressedKVCache of
// onnx-rt/src/kv_compression.rs:738-963, without the optional low-rank K)
// on gfx950: write, read, and the decode-attention fast path of the design
// (docs/kv-compression-design.md section 9) over the stored codes.
//
// A row (one token of one kv head, K or V) is PolarQuant-encoded
// (kv_compression.rs:216-268): signs s (the head's xorshift +-1 vector),
// normalised Walsh-Hadamard butterfly y = H(s*x)/sqrt(D), one min/max
// quantiser over y (codes of 3, 4 or 8 bits), and, with QJL on (:365-395),
// the sign bits of r = x - decode(codes) and C = mean|r|. One wave encodes a
// row, lane l holding dims l + 64 e (D = 64, 128 or 256): every f32 step is the reference's
// (same operands, same order, no contraction, IEEE division; the running
// sum of |r| is taken in dim order), so codes, scale, zero point, sign bits
// and C are the reference's bit for bit.
//
// Attention never decodes a key. Decoding is linear and orthonormal, so with
// the query encoded by the same quantiser (codes qc, scale qs, zero qz):
//   <decode(q), decode(k_t)> = sum_i (qs qc_i + qz)(ks_t kc_ti + kz_t),
// an integer dot product sum_i qc_i kc_ti (exact on the int8 MFMA, the
// query codes centred so that the f32 terms around it stay small) plus
// per-row terms; the logit adds the QJL popcount correction
// C_q C_t (D - 2 popcount(sq ^ s_t)) / D. The values are summed in the
// rotated domain on the f16 MFMA (weights p_t vs_t / S in f16, codes as exact
// f16 subnormals code * 2^-24) and rotated back once per output (inverse
// butterfly, signs) by the attention kernel: for a single split by its
// workgroup, otherwise by the workgroup that stores the last split partial.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode_common.h"
#include "sai_internal.h"

namespace sai {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef int intx4_t __attribute__((ext_vector_type(4)));

// round_f32 of kv_compression.rs:27-37 (half away from zero through a
// truncation); x >= 0 here.
__device__ __forceinline__ float round_half_away(float x) {
#pragma clang fp contract(off)
  const float t = (float)sat_i32(x);
  const float f = x - t;
  // selects, not branches (the values are the same)
  const float up = t + 1.0f, dn = t - 1.0f;
  return f >= 0.5f ? up : (f <= -0.5f ? dn : t);
}

// The value of lane `lane ^ H`, on VALU lane moves rather than LDS permutes:
// DPP quad_perm (H = 1, 2), row_shl / row_shr by 4 (lane i reads i + 4 or
// i - 4 within its row of 16; H = 4), row_ror by 8 (H = 8), and the gfx950
// lane-swap instructions (H = 16, 32; swap(x, x) returns the even and the odd
// halves, rows, each on both).
template <int H>
__device__ __forceinline__ float lane_xor(float v, int lane) {
  const int x = __float_as_int(v);
  if constexpr (H == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  } else if constexpr (H == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  } else if constexpr (H == 4) {
    const int up = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, false);
    const int dn = __builtin_amdgcn_mov_dpp(x, 0x114, 0xF, 0xF, false);
    return __int_as_float((lane & 4) ? dn : up);
  } else if constexpr (H == 8) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));
  } else if constexpr (H == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
    return __uint_as_float((lane & 16) ? s[0] : s[1]);
  } else {
    static_assert(H == 32, "lane_xor: H is a power of two up to 32");
    const auto s = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
    return __uint_as_float((lane & 32) ? s[0] : s[1]);
  }
}

// Wave reductions over lane_xor (the same partners, hence the same results,
// as the __shfl_xor forms).
__device__ __forceinline__ float wave_min(float v) {
  const int lane = threadIdx.x & 63;
  v = fminf(v, lane_xor<32>(v, lane));
  v = fminf(v, lane_xor<16>(v, lane));
  v = fminf(v, lane_xor<8>(v, lane));
  v = fminf(v, lane_xor<4>(v, lane));
  v = fminf(v, lane_xor<2>(v, lane));
  return fminf(v, lane_xor<1>(v, lane));
}
__device__ __forceinline__ float tq_wave_max(float v) {
  const int lane = threadIdx.x & 63;
  v = fmaxf(v, lane_xor<32>(v, lane));
  v = fmaxf(v, lane_xor<16>(v, lane));
  v = fmaxf(v, lane_xor<8>(v, lane));
  v = fmaxf(v, lane_xor<4>(v, lane));
  v = fmaxf(v, lane_xor<2>(v, lane));
  return fmaxf(v, lane_xor<1>(v, lane));
}
__device__ __forceinline__ float tq_wave_sum(float v) {
  const int lane = threadIdx.x & 63;
  v += lane_xor<32>(v, lane);
  v += lane_xor<16>(v, lane);
  v += lane_xor<8>(v, lane);
  v += lane_xor<4>(v, lane);
  v += lane_xor<2>(v, lane);
  return v + lane_xor<1>(v, lane);
}

// Element i of an f32 or bf16 row. One aligned dword load either way (for
// bf16 the word holding elements i & ~1 and i | 1) and a select, no branch:
// the compiler then counts the load's place among later loads exactly and
// waits for it alone.
__device__ __forceinline__ float load_row_elem(const void* p, size_t i, bool bf16) {
  const uint32_t w = *(const uint32_t*)((const char*)p + (bf16 ? (i * 2) & ~(size_t)3 : i * 4));
  return __uint_as_float(bf16 ? ((i & 1) ? (w & 0xFFFF0000u) : (w << 16)) : w);
}

// One butterfly stage below 64: dims l and l ^ H of each lane pair into
// (a + b, a - b), the sum at the lower dim.
template <int H, int E>
__device__ __forceinline__ void butterfly_stage(float (&y)[E], int lane) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float p = lane_xor<H>(y[e], lane);
    y[e] = (lane & H) ? p - y[e] : y[e] + p;
  }
}

// The reference's butterfly (wht_butterfly_normalize, :81-110) over a row
// spread across the wave (lane l: dims l + 64 e): stage h pairs dims (j, j+h)
// into (a + b, a - b); stages below 64 pair lanes l and l ^ h, stages 64 and
// up the dims of a lane. Then * norm.
template <int D>
__device__ __forceinline__ void wave_butterfly(float (&y)[D / 64], int lane, float norm) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  butterfly_stage<1>(y, lane);
  butterfly_stage<2>(y, lane);
  butterfly_stage<4>(y, lane);
  butterfly_stage<8>(y, lane);
  butterfly_stage<16>(y, lane);
  butterfly_stage<32>(y, lane);
  // stages 64, 128, ...: pairs of the lane's own dims, (e, e + h/64)
#pragma unroll
  for (int hs = 1; hs < E; hs <<= 1)
#pragma unroll
    for (int e = 0; e < E; ++e)
      if ((e & hs) == 0) {
        const float a0 = y[e], a1 = y[e + hs];
        y[e] = a0 + a1;
        y[e + hs] = a0 - a1;
      }
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] *= norm;
}

// PolarQuantizer::encode of the row x (lane l: dims l + 64 e): rotated
// values y, codes, scale, zero point.
template <int D, int BITS>
__device__ __forceinline__ void wave_encode(const float (&x)[D / 64], const float (&sgn)[D / 64],
                                            int lane, float norm, float (&y)[D / 64],
                                            uint32_t (&code)[D / 64], float& scale, float& zero) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  constexpr uint32_t LEVELS = (1u << BITS) - 1u;
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] = x[e] * sgn[e];
  wave_butterfly<D>(y, lane, norm);
  float mn = y[0], mx = y[0];
#pragma unroll
  for (int e = 1; e < E; ++e) {
    mn = fminf(mn, y[e]);
    mx = fmaxf(mx, y[e]);
  }
  mn = wave_min(mn);
  mx = tq_wave_max(mx);
  if (mn == 0.0f) {
    // the reference keeps the first minimum in dim order: with a zero
    // minimum, the sign of the first zero
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint64_t m = __ballot(y[e] == 0.0f);
      if (m) {
        mn = __shfl(y[e], __builtin_ctzll(m), 64);
        break;
      }
    }
  }
  const float range = mx - mn;
  scale = range > 0.0f ? range / (float)LEVELS : 1.0f;
  zero = mn;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t q = scale > 0.0f ? sat_u32(round_half_away((y[e] - zero) / scale)) : 0u;
    code[e] = q < LEVELS ? q : LEVELS;
  }
}

// Orders a wave's LDS stores before its later LDS loads (the wave's LDS
// operations complete in order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// QJLResidualEncoder::encode (:365-395) of x against decode(code): the sign
// words (uniform, word j = dims 32j .. 32j+31) and C = sum|r| / D. Stored rows
// (DIM_ORDER) sum in dim order on lane 0, as the reference does, through
// sres (the wave's D floats of LDS); the attention's query, whose C only
// scales its logit correction, sums by a wave reduction.
template <int D, bool DIM_ORDER = true>
__device__ __forceinline__ float wave_qjl(const uint32_t (&code)[D / 64], float scale, float zero,
                                          const float (&x)[D / 64], const float (&sgn)[D / 64],
                                          int lane, float norm, float* sres,
                                          uint64_t (&sbits)[D / 64]) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  float y[E];
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] = (float)code[e] * scale + zero;
  wave_butterfly<D>(y, lane, norm);
  float ra[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float r = x[e] - y[e] * sgn[e];
    sbits[e] = __ballot(r >= 0.0f);
    ra[e] = fabsf(r);
  }
  if constexpr (!DIM_ORDER) {
    float part = ra[0];
#pragma unroll
    for (int e = 1; e < E; ++e) part += ra[e];
    return tq_wave_sum(part) / (float)D;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) sres[lane + 64 * e] = ra[e];
  wave_lds_sync();
  float c = 0.0f;
  if (lane == 0) {
    float sum = 0.0f;
#pragma unroll 16
    for (int i = 0; i < D; ++i) sum += sres[i];
    c = sum / (float)D;
  }
  c = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(c)));
  wave_lds_sync();  // sres is reused by the wave's next row
  return c;
}

// Encodes the row x (lane l: dims l + 64 e) as position r of (kv head h,
// sequence b), K (kind 0) or V (kind 1), and stores it: K codes row-major; V
// codes into the position's bits of its tile, in the LDS copy `stile` of the
// tile's words when given, else by read-modify-write of the words in memory
// (the caller guarantees that no other wave writes that tile meanwhile);
// then the parameters (scale, zero point, QJL mean, sum of the codes) and the
// QJL sign words. Orders its LDS use at wave level only.
template <int D, int BITS>
__device__ __forceinline__ void wave_store_row(const TqArgs& a, const float (&x)[D / 64],
                                               const float (&sgn)[D / 64], int lane, int h, int b,
                                               int r, int kind, uint32_t (*stile)[2 * BITS + 1],
                                               float* sres, uint32_t* scode) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  constexpr int W = D * BITS / 32;  // K code words per row
  constexpr int TBW = 2 * BITS;     // V words per dim per tile
  constexpr uint32_t LEVELS = (1u << BITS) - 1u;
  float y[E], scale, zero;
  uint32_t code[E];
  wave_encode<D, BITS>(x, sgn, lane, a.norm, y, code, scale, zero);
  float csum = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) csum += (float)code[e];
  csum = tq_wave_sum(csum);  // integers below 2^24: exact
  const size_t row = ((size_t)h * a.batch_cap + b) * a.rows_cap + r;
  if (kind == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) scode[lane + 64 * e] = code[e];
    wave_lds_sync();
    if (lane < W) {
      uint32_t wd = 0u;
      const int i0 = (32 * lane) / BITS, i1 = (32 * lane + 31) / BITS;
      for (int i = i0; i <= i1; ++i) {
        const int bp = BITS * i - 32 * lane;
        wd |= bp >= 0 ? (scode[i] << bp) : (scode[i] >> -bp);
      }
      ((uint32_t*)(a.codes_k + row * a.code_stride))[lane] = wd;
    }
    wave_lds_sync();  // scode is reused by the wave's next row
  } else {
    const int p = (r % 64) * BITS, w = p >> 5, sh = p & 31;
    uint32_t* vt = (uint32_t*)(a.codes_v + (((size_t)h * a.batch_cap + b) * a.tiles_cap + r / 64) *
                                               tq_vtile_bytes(D, BITS));
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane + 64 * e;
      uint32_t* tw = stile ? stile[d] : vt + d * TBW;
      tw[w] = (tw[w] & ~(LEVELS << sh)) | (code[e] << sh);
      if (sh + BITS > 32) tw[w + 1] = (tw[w + 1] & ~(LEVELS >> (32 - sh))) | (code[e] >> (32 - sh));
    }
  }
  float c = 0.0f;
  if (a.qjl) {
    uint64_t sb[E];
    c = wave_qjl<D>(code, scale, zero, x, sgn, lane, a.norm, sres, sb);
    if (lane < D / 32) {
      uint64_t m = sb[0];
#pragma unroll
      for (int e = 1; e < E; ++e) m = (lane >> 1) == e ? sb[e] : m;
      ((kind ? a.signs_v : a.signs_k) + row * (D / 32))[lane] =
          (uint32_t)((lane & 1) ? (m >> 32) : m);
    }
  }
  if (lane == 0) (kind ? a.par_v : a.par_k)[row] = make_float4(scale, zero, c, csum);
}

// ---- write: one wave per (sequence, kv head, K|V, 64-position tile) --------
// The wave encodes the tile's rows of this pass in order. K rows go out
// row-major; V codes are merged into the tile's words (read, modified in LDS,
// written back) by the one wave that owns the tile.
template <int D, int BITS>
__global__ __launch_bounds__(64) void tq_write_kernel(const TqArgs a, const void* k, const void* v,
                                                      int bf16, int s_new) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  constexpr int TBW = 2 * BITS;  // V words per dim per tile
  const int lane = threadIdx.x;
  const int kind = blockIdx.y & 1, h = blockIdx.y >> 1, b = blockIdx.z;
  const int len = a.seq_lens[b];
  const int tile = len / 64 + (int)blockIdx.x;
  const int r_lo = max(len, tile * 64), r_hi = min(len + s_new, tile * 64 + 64);
  if (r_lo >= r_hi) return;  // uniform
  __shared__ uint32_t scode[D];
  __shared__ float sres[D];
  __shared__ uint32_t stile[D][TBW + 1];
  const void* src = kind ? v : k;
  const bool is_bf16 = bf16 != 0;
  float sgn[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sgn[e] = (float)a.signs[(size_t)h * D + lane + 64 * e];
  uint32_t* vt = (uint32_t*)(a.codes_v + (((size_t)h * a.batch_cap + b) * a.tiles_cap + tile) *
                                             tq_vtile_bytes(D, BITS));
  const int w_lo = ((r_lo - tile * 64) * BITS) >> 5;
  const int w_hi = ((r_hi - tile * 64) * BITS - 1) >> 5;
  if (kind) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      for (int w = w_lo; w <= w_hi; ++w) stile[lane + 64 * e][w] = vt[(lane + 64 * e) * TBW + w];
    wave_lds_sync();
  }
  for (int r = r_lo; r < r_hi; ++r) {
    const size_t in_off = (((size_t)b * s_new + (r - len)) * a.heads + h) * D;
    float x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = load_row_elem(src, in_off + lane + 64 * e, is_bf16);
    wave_store_row<D, BITS>(a, x, sgn, lane, h, b, r, kind, stile, sres, scode);
  }
  if (kind) {
    wave_lds_sync();
#pragma unroll
    for (int e = 0; e < E; ++e)
      for (int w = w_lo; w <= w_hi; ++w) vt[(lane + 64 * e) * TBW + w] = stile[lane + 64 * e][w];
  }
}

// V code of (position r, dim d) from the tile layout.
template <int D, int BITS>
__device__ __forceinline__ uint32_t v_code(const TqArgs& a, int h, int b, int r, int d) {
  const uint32_t* e = (const uint32_t*)(a.codes_v + (((size_t)h * a.batch_cap + b) * a.tiles_cap +
                                                     r / 64) * tq_vtile_bytes(D, BITS)) +
                      d * (2 * BITS);
  const int p = (r % 64) * BITS, w = p >> 5, sh = p & 31;
  uint32_t c = e[w] >> sh;
  if (sh + BITS > 32) c |= e[w + 1] << (32 - sh);
  return c & ((1u << BITS) - 1u);
}

// ---- read: one thread per (row, K|V), decode to f32 (a checking path) -------
template <int D, int BITS>
__global__ __launch_bounds__(64) void tq_read_kernel(const TqArgs a, int b, int h, int start,
                                                     int len, float* k_out, float* v_out) {
#pragma clang fp contract(off)
  const int idx = blockIdx.x * 64 + threadIdx.x;
  if (idx >= 2 * len) return;
  const int kind = idx & 1;
  const int t = idx >> 1;
  const size_t row = ((size_t)h * a.batch_cap + b) * a.rows_cap + start + t;
  if (kind == 0 && a.lr_us) {
    // read_k prefers the low-rank K (:871-881): reconstruct's 0 + U_S Vt
    const float u = a.lr_us[row];
    const float* vt = a.lr_vt + ((size_t)h * a.batch_cap + b) * D;
    float* out = k_out + (size_t)t * D;
    for (int i = 0; i < D; ++i) out[i] = 0.0f + u * vt[i];
    return;
  }
  const float4 par = (kind ? a.par_v : a.par_k)[row];
  const uint8_t* kc = a.codes_k + row * a.code_stride;
  float y[D];
  for (int i = 0; i < D; ++i) {
    uint32_t c;
    if (kind) {
      c = v_code<D, BITS>(a, h, b, start + t, i);
    } else {
      const int p = BITS * i, w = p >> 5, sh = p & 31;
      const uint32_t* cw = (const uint32_t*)kc;
      c = cw[w] >> sh;
      if (sh + BITS > 32) c |= cw[w + 1] << (32 - sh);
      c &= (1u << BITS) - 1u;
    }
    y[i] = (float)c * par.x + par.y;
  }
  for (int hh = 1; hh < D; hh *= 2)
    for (int i = 0; i < D; i += 2 * hh)
      for (int j = i; j < i + hh; ++j) {
        const float p = y[j], q = y[j + hh];
        y[j] = p + q;
        y[j + hh] = p - q;
      }
  const int8_t* sg = a.signs + (size_t)h * D;
  float* out = (kind ? v_out : k_out) + (size_t)t * D;
  for (int i = 0; i < D; ++i) out[i] = y[i] * a.norm * (float)sg[i];
}

// ---- Low-rank K (LowRankKeyDecomposer, kv_compression.rs:451-690) ----
// CompressedKVCache::write_kv (:840-852) decomposes a head's first K row on
// its own, so the kept rank is min(rank, 1, D) = 1, and update (:529-561)
// and reorthogonalize (:564-577) keep it: U_S is one float per row, Vt one
// row of D. Per row after the first, U_S[r] = k_r . Vt; when the write
// counter (rows - 1 mod 512) reaches 512, i.e. at rows 513, 1025, ...,
// U_S Vt is rebuilt and decomposed again by power iteration. Every dot
// product and norm is summed serially in the reference's index order with
// the product and the sum rounded apart (contraction off), so the state
// matches the reference bit for bit. One workgroup per (kv head, sequence)
// walks the pass's rows in order.
constexpr int LR_THREADS = 256;
constexpr int LR_CHUNK = 1024;
constexpr int LR_ROW_FLOATS = 16384;  // LDS for staged K rows, stride D + 1

// sqrt_approx (onnx-rt/src/operators.rs:3311-3320): ten Newton steps from x.
__device__ __forceinline__ float lr_sqrt_approx(float x) {
  if (x <= 0.0f) return 0.0f;
  float s = x;
  for (int i = 0; i < 10; ++i) s = 0.5f * (s + x / s);
  return s;
}

// normalize_vec (:683-690) of v_s[D]: thread 0 sums the squares in order.
template <int D>
__device__ void lr_normalize(float* v_s, float* bc) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  if (tid == 0) {
    float s = 0.0f;
#pragma unroll 16
    for (int j = 0; j < D; ++j) s = s + v_s[j] * v_s[j];
    *bc = lr_sqrt_approx(s);
  }
  __syncthreads();
  const float n = *bc;
  if (n > 1e-30f && tid < D) v_s[tid] = v_s[tid] / n;
  __syncthreads();
}

// v_s = the +-1 start of component 0 ((j + 0) even: +1), normalised.
template <int D>
__device__ void lr_start(float* v_s, float* bc) {
  if (threadIdx.x < D) v_s[threadIdx.x] = (threadIdx.x & 1) == 0 ? 1.0f : -1.0f;
  __syncthreads();
  lr_normalize<D>(v_s, bc);
}

// u[i] = sum_j (0 + us[i] vt_s[j]) v_s[j] for rows i < R: the rank-1
// reconstruction times v, each row's sum serial over j.
template <int D>
__device__ void lr_upass(const float* us, float* u, int R, const float* vt_s, const float* v_s) {
#pragma clang fp contract(off)
  for (int i = threadIdx.x; i < R; i += LR_THREADS) {
    const float ui = us[i];
    float dot = 0.0f;
    for (int j = 0; j < D; ++j) {
      const float x = 0.0f + ui * vt_s[j];
      dot = dot + x * v_s[j];
    }
    u[i] = dot;
  }
  __syncthreads();
}

// Re-decomposition of rows [0, R) (reorthogonalize + power_iteration_svd,
// :564-671, rank 1). vt_s holds the current Vt on entry and the new one on
// exit; us[0..R) is rewritten.
template <int D>
__device__ void lr_redecompose(float* us, float* u, int R, float* vt_s, float* v_s, float* c_us,
                               float* c_u, float* bc) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  lr_start<D>(v_s, bc);
  for (int it = 0; it < 10; ++it) {
    lr_upass<D>(us, u, R, vt_s, v_s);
    // v[j] = sum_i x_ij u[i], rows in order: thread j, rows staged in LDS
    float acc = 0.0f;
    for (int i0 = 0; i0 < R; i0 += LR_CHUNK) {
      const int n = min(LR_CHUNK, R - i0);
      for (int i = tid; i < n; i += LR_THREADS) {
        c_us[i] = us[i0 + i];
        c_u[i] = u[i0 + i];
      }
      __syncthreads();
      if (tid < D) {
        const float vj = vt_s[tid];
#pragma unroll 8
        for (int i = 0; i < n; ++i) {
          const float x = 0.0f + c_us[i] * vj;
          acc = acc + x * c_u[i];
        }
      }
      __syncthreads();
    }
    if (tid < D) v_s[tid] = acc;
    __syncthreads();
    lr_normalize<D>(v_s, bc);
  }
  lr_upass<D>(us, u, R, vt_s, v_s);
  // sigma = norm_vec(u), rows in order
  float s = 0.0f;
  for (int i0 = 0; i0 < R; i0 += LR_CHUNK) {
    const int n = min(LR_CHUNK, R - i0);
    for (int i = tid; i < n; i += LR_THREADS) c_u[i] = u[i0 + i];
    __syncthreads();
    if (tid == 0) {
#pragma unroll 8
      for (int i = 0; i < n; ++i) s = s + c_u[i] * c_u[i];
    }
    __syncthreads();
  }
  if (tid == 0) *bc = lr_sqrt_approx(s);
  __syncthreads();
  const float sigma = *bc;
  const bool zero = sigma < 1e-12f;  // the loop breaks: factors stay zero
  for (int i = tid; i < R; i += LR_THREADS) us[i] = zero ? 0.0f : (u[i] / sigma) * sigma;
  if (tid < D) vt_s[tid] = zero ? 0.0f : v_s[tid];
  __syncthreads();
}

template <int D>
__global__ __launch_bounds__(LR_THREADS) void tq_lowrank_kernel(const TqArgs a, const void* k,
                                                               int bf16, int s_new) {
#pragma clang fp contract(off)
  constexpr int NR = LR_ROW_FLOATS / (D + 1) < LR_THREADS ? LR_ROW_FLOATS / (D + 1) : LR_THREADS;
  __shared__ float vt_s[D], v_s[D], row_s[D], c_us[LR_CHUNK], c_u[LR_CHUNK];
  __shared__ float rows_s[NR * (D + 1)];
  __shared__ float bc;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int r0 = a.seq_lens[b];
  const size_t hb = (size_t)h * a.batch_cap + b;
  float* us = a.lr_us + hb * a.rows_cap;
  float* u = a.lr_u + hb * a.rows_cap;
  float* vtg = a.lr_vt + hb * D;
  const bool is_bf16 = bf16 != 0;
  auto in_off = [&](int t) { return (((size_t)b * s_new + t) * a.heads + h) * D; };
  if (tid < D) vt_s[tid] = r0 > 0 ? vtg[tid] : 0.0f;
  int t = 0;
  if (r0 == 0) {
    // decompose(k, 1, D) (:470-498): power iteration on the single row
    if (tid < D) row_s[tid] = load_row_elem(k, in_off(0) + tid, is_bf16);
    lr_start<D>(v_s, &bc);
    for (int it = 0; it < 10; ++it) {
      if (tid == 0) {
        float dot = 0.0f;
#pragma unroll 16
        for (int j = 0; j < D; ++j) dot = dot + row_s[j] * v_s[j];
        bc = dot;
      }
      __syncthreads();
      const float u0 = bc;
      __syncthreads();
      if (tid < D) v_s[tid] = 0.0f + row_s[tid] * u0;
      __syncthreads();
      lr_normalize<D>(v_s, &bc);
    }
    if (tid == 0) {
      float dot = 0.0f;
#pragma unroll 16
      for (int j = 0; j < D; ++j) dot = dot + row_s[j] * v_s[j];
      const float sigma = lr_sqrt_approx(0.0f + dot * dot);
      const bool zero = sigma < 1e-12f;
      us[0] = zero ? 0.0f : (dot / sigma) * sigma;
      bc = zero ? 0.0f : 1.0f;
    }
    __syncthreads();
    if (tid < D) vt_s[tid] = bc != 0.0f ? v_s[tid] : 0.0f;
    __syncthreads();
    t = 1;
  }
  while (t < s_new) {
    const int r = r0 + t;                       // >= 1
    const int rr = (r + 511) / 512 * 512;       // the next row whose write re-decomposes
    const int t_end = min(s_new, rr - r0 + 1);  // rows [t, t_end) project onto this Vt
    // rows staged in LDS by coalesced loads, then one thread per row
    for (int t0 = t; t0 < t_end; t0 += NR) {
      const int nr = min(NR, t_end - t0);
      for (int e = tid; e < nr * D; e += LR_THREADS) {
        const int q = e / D, c = e - q * D;
        rows_s[q * (D + 1) + c] = load_row_elem(k, in_off(t0 + q) + c, is_bf16);
      }
      __syncthreads();
      if (tid < nr) {
        const float* x = rows_s + tid * (D + 1);
        float dot = 0.0f;
#pragma unroll 16
        for (int c = 0; c < D; ++c) dot = dot + x[c] * vt_s[c];
        us[r0 + t0 + tid] = dot;
      }
      __syncthreads();
    }
    if (r0 + t_end - 1 == rr) lr_redecompose<D>(us, u, rr + 1, vt_s, v_s, c_us, c_u, &bc);
    t = t_end;
  }
  if (tid < D) vtg[tid] = vt_s[tid];
}

// Byte position of dim d's code in a query record: the order in which the
// attention kernel unpacks a K row into int8 MFMA operands (4 dims a step).
// 4-bit: step 2w takes the low nibbles of word w (dims 8w, 8w+2, 8w+4,
// 8w+6), step 2w+1 the high ones; 3- and 8-bit: dims in order.
template <int BITS>
__device__ __forceinline__ int q_code_pos(int d) {
  if constexpr (BITS == 4) return 4 * (2 * (d >> 3) + (d & 1)) + ((d & 7) >> 1);
  return d;
}

// ---- query encoding: one wave per query head -------------------------------
// The query row through its kv head's quantizer, into LDS:
//   codes[D/4]  codes - 2^(bits-1) as int8, in q_code_pos order
//   coef[4]     alpha = qs, beta = qz', gamma = qs sum(qc') + D qz',
//               kappa = C / D, each times scale * log2(e)
//   sgn[D/32]   QJL sign words
// where qc' = qc - 2^(bits-1) and qz' = qz + qs 2^(bits-1), so that
// decode(q) rotated = qs qc' + qz'. x: the query row (lane l: dims l + 64 e),
// sgn: the kv head's signs, both loaded by the caller.
template <int D, int BITS>
__device__ __forceinline__ void wave_encode_query(const TqArgs& a, const TqAttendArgs& t,
                                                  const float (&x)[D / 64],
                                                  const float (&sgn)[D / 64], int lane,
                                                  float* sres, uint32_t* codes, float* coef,
                                                  uint32_t* sgw) {
#pragma clang fp contract(off)
  constexpr int E = D / 64;
  constexpr int C0 = 1 << (BITS - 1);
  float y[E], scale, zero;
  uint32_t code[E];
  wave_encode<D, BITS>(x, sgn, lane, a.norm, y, code, scale, zero);
  float sq = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int cc = (int)code[e] - C0;
    sq += (float)cc;
    ((int8_t*)codes)[q_code_pos<BITS>(lane + 64 * e)] = (int8_t)cc;
  }
  sq = tq_wave_sum(sq);
  float c = 0.0f;
  uint64_t sb[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sb[e] = 0;
  if (a.qjl) c = wave_qjl<D, false>(code, scale, zero, x, sgn, lane, a.norm, sres, sb);
  if (lane == 0) {
    const float qz = zero + scale * (float)C0;
    coef[0] = scale * t.scale_log2;
    coef[1] = qz * t.scale_log2;
    coef[2] = (scale * sq + (float)D * qz) * t.scale_log2;
    coef[3] = c / (float)D * t.scale_log2;
  }
  if (lane < D / 32) {
    uint64_t m = sb[0];
#pragma unroll
    for (int e = 1; e < E; ++e) m = (lane >> 1) == e ? sb[e] : m;
    sgw[lane] = (uint32_t)((lane & 1) ? (m >> 32) : m);
  }
}

// int8 MFMA operand of K row codes for logit step s (4 dims).
template <int BITS, int KW>
__device__ __forceinline__ int k_operand(const uint32_t (&kc)[KW], int s) {
  if constexpr (BITS == 4) {
    const uint32_t w = kc[s >> 1];
    return (int)((s & 1) ? ((w >> 4) & 0x0F0F0F0Fu) : (w & 0x0F0F0F0Fu));
  } else if constexpr (BITS == 8) {
    return (int)(kc[s] ^ 0x80808080u);  // codes - 128
  } else {
    // dims 4s .. 4s+3: 12 bits at 12 s, spread to bytes
    const int p = 12 * s, w = p >> 5, sh = p & 31;
    uint32_t x = kc[w] >> sh;
    if (sh > 20) x |= kc[w + 1] << (32 - sh);
    x &= 0xFFFu;
    x = (x | (x << 10)) & 0x003F003Fu;
    return (int)((x | (x << 5)) & 0x07070707u);
  }
}

// f16 MFMA operand (4 positions of one dim) of V codes, as subnormals
// code * 2^-24, for value step s. 4-bit: word s/2 gives positions
// (0, 4, 1, 5) + 8 (s/2) for even s and (2, 6, 3, 7) + 8 (s/2) for odd s;
// with MIXED the odd positions' nibbles stay in place, code * 2^-20 (one mask
// instead of a shift and a mask), and the caller takes the even positions'
// weights 16x larger. 3- and 8-bit: positions 4s .. 4s+3 in order.
template <int BITS, int TBW, bool MIXED = false>
__device__ __forceinline__ half4_t v_operand(const uint32_t (&vc)[TBW], int s) {
  uint32_t lo, hi;
  if constexpr (BITS == 4) {
    const uint32_t w = vc[s >> 1] >> ((s & 1) * 8);
    lo = w & 0x000F000Fu;
    hi = MIXED ? (w & 0x00F000F0u) : ((w >> 4) & 0x000F000Fu);
  } else if constexpr (BITS == 8) {
    lo = __builtin_amdgcn_perm(0u, vc[s], 0x0C010C00u);
    hi = __builtin_amdgcn_perm(0u, vc[s], 0x0C030C02u);
  } else {
    const int p = 12 * s, w = p >> 5, sh = p & 31;
    uint32_t x = vc[w] >> sh;
    if (sh > 20) x |= vc[w + 1] << (32 - sh);
    x &= 0xFFFu;
    const uint32_t u = x | (x << 13);
    lo = u & 0x00070007u;
    hi = (u >> 6) & 0x00070007u;
  }
  const uint32_t pr[2] = {lo, hi};
  half4_t r;
  __builtin_memcpy(&r, pr, sizeof(r));
  return r;
}

// Slot of tile position r in the P' rows, matching v_operand's order.
template <int BITS>
__device__ __forceinline__ int p_slot(int r) {
  if constexpr (BITS == 4) return (r & ~7) + 2 * (r & 3) + ((r >> 2) & 1);
  return r;
}

// Rows sy[g] (the group's outputs in the rotated domain) back to the model's
// domain: wave g takes row g (lane l: dims l + 64 e) through the butterfly's
// stages on lane moves and * norm (wave_butterfly, the same stages and
// roundings as over LDS), then * the signs, written to out. Waves past the
// group return.
template <int D, int G, int NW>
__device__ __forceinline__ void rotate_back(const TqArgs& a, const TqAttendArgs& t, int b,
                                            int kvh, const float (&sy)[G][D]) {
#pragma clang fp contract(off)
  static_assert(G <= NW, "one wave per row of the group");
  constexpr int E = D / 64;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  if (wave >= G) return;
  float y[E];
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] = sy[wave][lane + 64 * e];
  wave_butterfly<D>(y, lane, a.norm);
  float* o = t.out + ((size_t)b * t.num_heads + kvh * G + wave) * D;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = lane + 64 * e;
    o[i] = y[e] * (float)a.signs[(size_t)kvh * D + i];
  }
}

// ---- attention ---------------------------------------------------------------
// One lane's share of a 64-position tile: its position's K codes, parameters
// and sign words, and the V codes of its dims over the tile's positions.
template <int D, int BITS, int MODE>
struct TqTile {
  static constexpr int KWL = (D * BITS / 32 + 3) / 4 * 4;  // K words loaded
  static constexpr int DH = D / 64;
  static constexpr int TBW = 2 * BITS;  // V words per dim per tile
  uint32_t kc[MODE != 2 ? KWL : 1];
  uint32_t ks[D / 32];
  uint32_t vc[DH][MODE != 1 ? TBW : 1];
  float4 kp, vp;
};

// Loads tile tile0's share for this lane (positions past r1 read the tile's
// first row, a valid one; the caller masks them). Branch-free, so that the
// compiler knows at every later use how many loads were issued after each
// one: without QJL the sign-word loads read K code bytes instead (rows of
// code_stride >= D/8 bytes), whose values are never used.
template <int D, int BITS, int MODE>
__device__ __forceinline__ void tq_load_tile(const TqArgs& a, size_t rbase, const uint8_t* vbase,
                                             int tile0, int r1, int lane,
                                             TqTile<D, BITS, MODE>& T) {
  using Tl = TqTile<D, BITS, MODE>;
  const int row = tile0 + lane;
  const size_t rr = rbase + (row < r1 ? row : tile0);
  if constexpr (MODE != 2) {
    const uint4* src = (const uint4*)(a.codes_k + rr * a.code_stride);
#pragma unroll
    for (int j = 0; j < Tl::KWL / 4; ++j) {
      const uint4 w4 = src[j];
      T.kc[4 * j] = w4.x;
      T.kc[4 * j + 1] = w4.y;
      T.kc[4 * j + 2] = w4.z;
      T.kc[4 * j + 3] = w4.w;
    }
  }
  T.kp = a.par_k[rr];
  T.vp = a.par_v[rr];
  if constexpr (MODE != 2) {
    const uint8_t* sbase = a.qjl ? (const uint8_t*)a.signs_k : a.codes_k;
    const size_t sstride = a.qjl ? (size_t)(D / 8) : a.code_stride;
    const uint8_t* srow = sbase + rr * sstride;
#pragma unroll
    for (int j = 0; j < D / 128; ++j) {
      const uint4 w4 = ((const uint4*)srow)[j];
      T.ks[4 * j] = w4.x;
      T.ks[4 * j + 1] = w4.y;
      T.ks[4 * j + 2] = w4.z;
      T.ks[4 * j + 3] = w4.w;
    }
    if constexpr (D == 64) {  // two words
      const uint2 w2 = *(const uint2*)srow;
      T.ks[0] = w2.x;
      T.ks[1] = w2.y;
    }
  }
  if constexpr (MODE != 1) {
    const uint8_t* vt = vbase + (size_t)(tile0 / 64) * tq_vtile_bytes(D, BITS);
#pragma unroll
    for (int e = 0; e < Tl::DH; ++e) {
      const uint2* src = (const uint2*)(vt + (size_t)(64 * e + lane) * (8 * BITS));
#pragma unroll
      for (int j = 0; j < Tl::TBW / 2; ++j) {
        const uint2 w2 = src[j];
        T.vc[e][2 * j] = w2.x;
        T.vc[e][2 * j + 1] = w2.y;
      }
    }
  }
}

// Workgroup = (split of split_rows positions, kv head, sequence), NW waves; a
// wave takes 64-position tiles. Logits: lane = position, the group's heads in
// quads (4x4x4 int8 MFMA: A = four heads' query codes, B = the lane's K row,
// so lane l's result i is head 4u + i at position l). Values: lane = dim
// (4x4x4 f16 MFMA: A = four heads' weights, B = the lane's dim over four
// positions, so lane l's result i is head 4u + i at dim 64 e + l).
// MODE 0: attention (softmax of scale * logits, weighted value sum, rotated
// back). MODE 1: the logits alone (the design's attention_logits), written to
// t.out[(b, head)][position] with row stride t.ld, coefficients at scale 1.
// MODE 2: the weighted value sum alone (weighted_value_sum) of the weights
// t.weights[(b, head)][position], not normalised.
template <int D, int BITS, int G, int NW, int MODE>
__global__ __launch_bounds__(64 * NW, NW >= 8 ? 2 : 1) void tq_attend_kernel(
    const TqArgs a, TqAttendArgs t) {
  constexpr int NQ = (G + 3) / 4;
  constexpr int KW = D * BITS / 32;
  constexpr int KWL = (KW + 3) / 4 * 4;  // words loaded (within code_stride)
  constexpr int NS = D / 4;              // logit steps
  constexpr int DH = D / 64;             // value dim halves
  constexpr int TBW = 2 * BITS;          // V words per dim per tile
  constexpr int KOFF = BITS == 8 ? 128 : 0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int L = a.seq_lens[b] + a.pending;
  const int r0 = split * t.split_rows;
  if (L == 0) {
    // no rows: the reference's zero row (sdpa_write_zero_row, microsoft.rs:322-326)
    if (MODE != 1 && split == 0)
      for (int e = threadIdx.x; e < G * D; e += 64 * NW)
        t.out[((size_t)b * t.num_heads + kvh * G + e / D) * D + e % D] = 0.0f;
    return;
  }
  if (r0 >= L) return;  // uniform: this split is past the sequence
  const int r1 = min(L, r0 + t.split_rows);
  const size_t rbase = ((size_t)kvh * a.batch_cap + b) * a.rows_cap;
  const uint8_t* vbase =
      a.codes_v + ((size_t)kvh * a.batch_cap + b) * a.tiles_cap * tq_vtile_bytes(D, BITS);
  // The group's query rows (one wave per head) and the kv head's signs are
  // loaded first: the prologue waits for them, and loads complete in order.
  constexpr int HPW = (G + NW - 1) / NW;  // query heads per wave
  float qx[HPW][D / 64], qsg[D / 64];
  // Every load below is unconditional (a wave without a head or a tile reads
  // a valid one it does not use): the compiler's wait before each use then
  // counts exactly the loads issued after it, on every path.
  if constexpr (MODE != 2) {
#pragma unroll
    for (int e = 0; e < D / 64; ++e) qsg[e] = (float)a.signs[(size_t)kvh * D + lane + 64 * e];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const int g = min(wave + NW * h, G - 1);
#pragma unroll
      for (int e = 0; e < D / 64; ++e)
        qx[h][e] = load_row_elem(t.q, ((size_t)b * t.num_heads + kvh * G + g) * D + lane + 64 * e,
                                 t.q_bf16 != 0);
    }
  }
  // Tiles of the split: wave w starts with tile w, the rest come from a
  // workgroup counter. In a fused step the last split's workgroup stores the
  // pass's new row, which lies in its last tile T. One wave (T's holder, else
  // the last wave, whose own first tile then goes to the counter) stores the
  // row's K and V after the prologue barrier, while the other waves already
  // stream, and then computes T first; no other wave touches T. Stored in the
  // prologue instead, the row held the whole workgroup at the barrier, and
  // that split's loop ended 2-3 us after the others.
  const int ntile = (r1 - r0 + 63) / 64;
  const int T = ntile - 1;
  const bool fused_store = MODE == 0 && t.k_new != nullptr && r1 == L;
  const int store_wave = T < NW ? T : NW - 1;
  const bool storer = fused_store && wave == store_wave;
  const bool t_pooled = fused_store && T >= NW;  // tile NW - 1 goes to the counter
  const int first_tile = storer ? T : wave;
  // the new row's K and V elements, loaded by every wave with the query's
  // (branch-free; without a fused row they read the query, unused)
  float xnk[D / 64], xnv[D / 64];
  if constexpr (MODE == 0) {
    const bool have = t.k_new != nullptr;
    const void* kn = have ? t.k_new : t.q;
    const void* vn = have ? t.v_new : t.q;
    const bool bf = have ? t.kv_bf16 != 0 : t.q_bf16 != 0;
    const size_t in_off = ((size_t)b * a.heads + kvh) * D;
#pragma unroll
    for (int e = 0; e < D / 64; ++e) {
      xnk[e] = load_row_elem(kn, in_off + lane + 64 * e, bf);
      xnv[e] = load_row_elem(vn, in_off + lane + 64 * e, bf);
    }
  }
  // Two tile buffers: a wave loads its next tile before it computes the
  // current one. The first tile's loads follow the query's, before the
  // prologue (the query's wait then counts them as later loads).
  TqTile<D, BITS, MODE> tb[2];
  const int first = r0 + first_tile * 64;
  tq_load_tile<D, BITS, MODE>(a, rbase, vbase, first < r1 ? first : r0, r1, lane, tb[0]);

  __shared__ uint32_t sqc[NQ * 4][NS];           // query code words (padding heads 0)
  __shared__ float sqf[G][4];                    // alpha, beta, gamma, kappa
  __shared__ uint32_t sqs[G][D / 32];            // query QJL sign words
  __shared__ float sres[NW][D];
  __shared__ _Float16 sp[NW][NQ * 4][64 + 4];    // a wave's P' rows
  if constexpr (MODE != 2) {
    for (int e = threadIdx.x; e < (NQ * 4 - G) * NS; e += 64 * NW) sqc[G + e / NS][e % NS] = 0u;
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const int g = wave + NW * h;
      if (g < G)
        wave_encode_query<D, BITS>(a, t, qx[h], qsg, lane, sres[wave], sqc[g], sqf[g], sqs[g]);
    }
  }
  // tiles past each wave's first are handed out from this counter, one
  // index at a time
  __shared__ int sm_next;
  if (threadIdx.x == 0) sm_next = 0;
  __syncthreads();
  if constexpr (MODE == 0) {
    if (storer) {
      __shared__ uint32_t scode[D];
      float sgn[D / 64];
#pragma unroll
      for (int e = 0; e < D / 64; ++e) sgn[e] = (float)a.signs[(size_t)kvh * D + lane + 64 * e];
      wave_store_row<D, BITS>(a, xnk, sgn, lane, kvh, b, L - 1, 0, nullptr, sres[wave], scode);
      wave_store_row<D, BITS>(a, xnv, sgn, lane, kvh, b, L - 1, 1, nullptr, sres[wave], scode);
      __threadfence_block();
      tq_load_tile<D, BITS, MODE>(a, rbase, vbase, first, r1, lane, tb[0]);
    }
  }
  // the query's coefficients and sign words are uniform: scalar registers
  float qa[G], qb[G], qg[G], qk[G];
  uint32_t qs[G][D / 32];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qa[g] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sqf[g][0])));
    qb[g] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sqf[g][1])));
    qg[g] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sqf[g][2])));
    qk[g] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sqf[g][3])));
#pragma unroll
    for (int j = 0; j < D / 32; ++j) qs[g][j] = __builtin_amdgcn_readfirstlane(sqs[g][j]);
  }

  float m_run[G], l_run[G], z_run[G];
  floatx4_t o_run[NQ][DH];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = MODE == 2 ? 0.0f : -INFINITY;  // given weights: no running max
    l_run[g] = 0.0f;
    z_run[g] = 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u)
#pragma unroll
    for (int e = 0; e < DH; ++e) o_run[u][e] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // one tile of this wave: logits, online softmax, value sums
  auto process = [&](const TqTile<D, BITS, MODE>& T, int tile0) __attribute__((always_inline)) {
    const int row = tile0 + lane;
    const bool live = row < r1;
    const float4 kp = T.kp;
    const float4 vp = T.vp;
    float lg[G];
    if constexpr (MODE != 2) {
    // logits: exact integer dot products on the int8 MFMA
    intx4_t ip[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) ip[u] = intx4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int kb = k_operand<BITS, KWL>(T.kc, s);
#pragma unroll
      for (int u = 0; u < NQ; ++u)
        ip[u] = __builtin_amdgcn_mfma_i32_4x4x4i8((int)sqc[4 * u + (lane & 3)][s], kb, ip[u], 0, 0,
                                                 0);
    }
    const float sk = kp.w - (float)(KOFF * D);
    const float kz = kp.y + (float)KOFF * kp.x;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float ipf = (float)ip[g >> 2][g & 3];
      float dot = kp.x * (qa[g] * ipf + qb[g] * sk) + kz * qg[g];
      if (a.qjl) {
        int pop = 0;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) pop += __popc(qs[g][j] ^ T.ks[j]);
        dot += qk[g] * kp.z * (float)(D - 2 * pop);
      }
      lg[g] = live ? dot : -INFINITY;
    }
    }  // MODE != 2
    if constexpr (MODE == 1) {
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (live) t.out[((size_t)b * t.num_heads + kvh * G + g) * t.ld + row] = lg[g];
    } else {
    // online softmax (log2 domain); the running max moves only when a lane
    // exceeds it
    float alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      alpha[g] = 1.0f;
      if (MODE == 0 && __ballot(lg[g] > m_run[g])) {
        const float m_new = fmaxf(m_run[g], wave_max_rows(lg[g]));
        alpha[g] = fast_exp2(m_run[g] - m_new);
        m_run[g] = m_new;
      }
    }
    // weights: P' = f16(p vs / S); the row's whole value (vs code + vz) and
    // the normaliser take the same rounded weight p' = P' S / vs, so the
    // f16 rounding perturbs each weight instead of splitting the row
    const float vsmax = wave_max_rows(live ? vp.x : 0.0f);
    // 4-bit codes of odd positions enter the values' MFMA at 2^-20 (v_operand's
    // MIXED form), so the even positions' P' are taken 16x larger (exact; the
    // softmax weights are <= 1, so P' <= 16). Not for the caller's weights
    // (MODE 2), whose range binary16 would then shrink 16-fold.
    constexpr bool kMixed = BITS == 4 && MODE != 2;
    const float up = (kMixed && (lane & 1) == 0) ? 16.0f : 1.0f;
    // hardware reciprocals (1 ulp) instead of IEEE divisions: the two ratios
    // only need to be each other's inverse far below the f16 rounding of P'
    const float vsn = vp.x * __builtin_amdgcn_rcpf(vsmax) * up;
    const float rvsn = vsmax * __builtin_amdgcn_rcpf(vp.x) * (1.0f / up);
    const int slot = p_slot<BITS>(lane);
#pragma unroll
    for (int g = 0; g < NQ * 4; ++g) {
      _Float16 ph = (_Float16)0.0f;
      if (g < G) {
        const float pw =
            MODE == 2 ? (live ? t.weights[((size_t)b * t.num_heads + kvh * G + g) * t.ld + row]
                              : 0.0f)
                      : fast_exp2(lg[g] - m_run[g]);
        ph = (_Float16)(pw * vsn);
        const float p = (float)ph * rvsn;
        l_run[g] = l_run[g] * alpha[g] + p;
        z_run[g] = z_run[g] * alpha[g] + p * vp.y;
      }
      sp[wave][g][slot] = ph;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // values: sum_t P'_t code_t on the f16 MFMA
    floatx4_t mf[NQ][DH];
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int e = 0; e < DH; ++e) mf[u][e] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      half4_t pa[NQ];
#pragma unroll
      for (int u = 0; u < NQ; ++u) pa[u] = *(const half4_t*)&sp[wave][4 * u + (lane & 3)][4 * s];
#pragma unroll
      for (int e = 0; e < DH; ++e) {
        const half4_t vb = v_operand<BITS, TBW, kMixed>(T.vc[e], s);
#pragma unroll
        for (int u = 0; u < NQ; ++u)
          mf[u][e] = __builtin_amdgcn_mfma_f32_4x4x4f16(pa[u], vb, mf[u][e], 0, 0, 0);
      }
    }
    // the codes' subnormal scale: 2^24, or 2^20 with the even positions' P' x 16
    const float sc = vsmax * (kMixed ? 1048576.0f : 16777216.0f);
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int e = 0; e < DH; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 4 * u + i;
          if (g < G) o_run[u][e][i] = o_run[u][e][i] * alpha[g] + mf[u][e][i] * sc;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    }  // MODE != 1
  };
  // Wave w's first tile is tile w of the split; the rest are taken from the
  // workgroup's counter, each index asked for one tile ahead, so the waves
  // of a workgroup finish together however their loads are served (with a
  // fixed share, the last wave of a workgroup ended ~6 us after the first).
  // The next tile's loads are issued before the current tile is computed;
  // only the loop's exits branch around a load.
  // With t.static_tiles the order is fixed instead: wave w takes tiles w,
  // w + NW, ... (a storer whose first tile went to the pool takes NW - 1,
  // 2 NW - 1, ... after T), so repeated launches give bit-identical outputs.
  const int static_base = storer && t_pooled ? NW - 1 : wave + NW;
  int grabs = 0;
  auto grab_issue = [&]() {  // dynamic: lane 0 holds the counter's old value
    int v = 0;
    if (t.static_tiles)
      v = grabs++;
    else if (lane == 0)
      v = atomicAdd(&sm_next, 1);
    return v;
  };
  // counter value c: tile NW + c, or with T kept out, NW - 1 first, then
  // NW + c - 1 (T itself is never handed out: the values stop at T)
  auto grab_value = [&](int v) {
    if (t.static_tiles) return static_base + NW * v;
    const int c = __builtin_amdgcn_readfirstlane(v);
    return t_pooled ? (c == 0 ? NW - 1 : NW + c - 1) : NW + c;
  };
  const int pool_end = t_pooled ? T : ntile;  // grab values from here on stop
  if (first_tile < ntile) {
    int cur = first_tile;
    int gq = grab_issue();
    for (;;) {
      const int n1 = grab_value(gq);
      if (n1 >= pool_end) {
        process(tb[0], r0 + 64 * cur);
        break;
      }
      gq = grab_issue();
      tq_load_tile<D, BITS, MODE>(a, rbase, vbase, r0 + 64 * n1, r1, lane, tb[1]);
      process(tb[0], r0 + 64 * cur);
      const int n2 = grab_value(gq);
      if (n2 >= pool_end) {
        process(tb[1], r0 + 64 * n1);
        break;
      }
      gq = grab_issue();
      tq_load_tile<D, BITS, MODE>(a, rbase, vbase, r0 + 64 * n2, r1, lane, tb[0]);
      process(tb[1], r0 + 64 * n1);
      cur = n2;
    }
  }
  if constexpr (MODE == 1) return;
  // merge the waves through LDS
  __shared__ float sm_m[NW][G], sm_l[NW][G], sm_z[NW][G];
  __shared__ float sm_o[NW][G][D];
  __shared__ float sy[G][D];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lsum = tq_wave_sum(l_run[g]);
    const float zsum = tq_wave_sum(z_run[g]);
    if (lane == 0) {
      sm_m[wave][g] = m_run[g];
      sm_l[wave][g] = lsum;
      sm_z[wave][g] = zsum;
    }
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u)
#pragma unroll
    for (int e = 0; e < DH; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * u + i < G) sm_o[wave][4 * u + i][64 * e + lane] = o_run[u][e][i];
  __syncthreads();
  const int nsplit = (L + t.split_rows - 1) / t.split_rows;
  const size_t pstride = (size_t)G * (D + 2);
  float* part0 = t.partials + ((size_t)b * a.heads + kvh) * t.max_splits * pstride;
  for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
    const int g = e / D, i = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w][g]);
    float Ls = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (sm_m[w][g] == -INFINITY) continue;
      const float f = fast_exp2(sm_m[w][g] - M);
      Ls += sm_l[w][g] * f;
      O += (sm_o[w][g][i] + sm_z[w][g]) * f;
    }
    if (nsplit == 1) {
      sy[g][i] = MODE == 2 ? O : (Ls > 0.0f ? O / Ls : 0.0f);
    } else {
      float* part = part0 + split * pstride + g * (D + 2);
      store_partial(part + 2 + i, O);
      if (i == 0) {
        store_partial(part, M);
        store_partial(part + 1, Ls);
      }
    }
  }
  if (nsplit > 1) {
    // The workgroup with the last ticket of (sequence, kv head) merges every
    // split's partial, its own included, in split order (the result does not
    // depend on which one finished last). The partial stores are agent-scope
    // and complete before the ticket is taken, so the other XCDs see them.
    __shared__ int sm_last;
    partials_complete();
    __syncthreads();
    int* counter = t.counters + (size_t)b * a.heads + kvh;
    if (threadIdx.x == 0) sm_last = last_ticket(counter, nsplit);
    __syncthreads();
    if (!sm_last) return;
    for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
      const int g = e / D, i = e % D;
      float M = -INFINITY, Ls = 0.0f, O = 0.0f;
      const float* ph = part0 + g * (D + 2);
      if (nsplit <= 4)
        merge_partials<4>(ph, pstride, i, nsplit, -1, M, Ls, O);
      else if (nsplit <= 8)
        merge_partials<8>(ph, pstride, i, nsplit, -1, M, Ls, O);
      else
        merge_partials<16>(ph, pstride, i, nsplit, -1, M, Ls, O);
      sy[g][i] = MODE == 2 ? O : (Ls > 0.0f ? O / Ls : 0.0f);
    }
    if (threadIdx.x == 0) reset_ticket(counter);
  }
  __syncthreads();
  rotate_back<D, G, NW>(a, t, b, kvh, sy);
}

// Waves per workgroup: 8 (two per SIMD, one workgroup per CU) up to head_dim
// 128; at 256 the tile buffers need more registers than two waves per SIMD
// leave, so 4.
template <int D>
constexpr int tq_attend_waves() {
  return D <= 128 ? 8 : 4;
}

template <int D, int BITS, int MODE>
hipError_t attend_db(const TqArgs& a, const TqAttendArgs& t, int group, int nsplit, int batch,
                     hipStream_t st) {
  constexpr int NW = tq_attend_waves<D>();
  const dim3 grid(nsplit, a.heads, batch), block(64 * NW);
  switch (group) {
    case 1: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 1, NW, MODE>), grid, block, 0, st, a, t); break;
    case 2: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 2, NW, MODE>), grid, block, 0, st, a, t); break;
    case 4: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 4, NW, MODE>), grid, block, 0, st, a, t); break;
    case 8:
      if constexpr (D <= 128) {
        hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 8, NW, MODE>), grid, block, 0, st, a, t);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename F>
hipError_t dispatch_dbits(int d, int bits, F&& f) {
  auto by_bits = [&](auto dd) -> hipError_t {
    switch (bits) {
      case 3: return f(dd, std::integral_constant<int, 3>{});
      case 4: return f(dd, std::integral_constant<int, 4>{});
      case 8: return f(dd, std::integral_constant<int, 8>{});
      default: return hipErrorInvalidValue;
    }
  };
  if (d == 64) return by_bits(std::integral_constant<int, 64>{});
  if (d == 128) return by_bits(std::integral_constant<int, 128>{});
  if (d == 256) return by_bits(std::integral_constant<int, 256>{});
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_tq_write(const TqArgs& a, const void* k, const void* v, int bf16, int batch,
                           int s_new, hipStream_t st) {
  if (batch <= 0 || s_new <= 0) return hipSuccess;
  // tiles a pass of s_new positions can touch, whatever the start's offset
  const dim3 grid((s_new + 126) / 64, 2 * a.heads, batch);
  return dispatch_dbits(a.head_dim, a.bits, [&](auto dd, auto bb) -> hipError_t {
    constexpr int D = decltype(dd)::value, B = decltype(bb)::value;
    hipLaunchKernelGGL((tq_write_kernel<D, B>), grid, dim3(64), 0, st, a, k, v, bf16, s_new);
    return hipGetLastError();
  });
}

hipError_t launch_tq_lowrank(const TqArgs& a, const void* k, int bf16, int batch, int s_new,
                             hipStream_t st) {
  if (batch <= 0 || s_new <= 0 || !a.lr_us) return hipSuccess;
  const dim3 grid(a.heads, batch);
  switch (a.head_dim) {
    case 64:
      hipLaunchKernelGGL(tq_lowrank_kernel<64>, grid, dim3(LR_THREADS), 0, st, a, k, bf16, s_new);
      break;
    case 128:
      hipLaunchKernelGGL(tq_lowrank_kernel<128>, grid, dim3(LR_THREADS), 0, st, a, k, bf16, s_new);
      break;
    case 256:
      hipLaunchKernelGGL(tq_lowrank_kernel<256>, grid, dim3(LR_THREADS), 0, st, a, k, bf16, s_new);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_tq_read(const TqArgs& a, int b, int h, int start, int len, float* k_out,
                          float* v_out, hipStream_t st) {
  if (len <= 0) return hipSuccess;
  return dispatch_dbits(a.head_dim, a.bits, [&](auto dd, auto bb) -> hipError_t {
    constexpr int D = decltype(dd)::value, B = decltype(bb)::value;
    hipLaunchKernelGGL((tq_read_kernel<D, B>), dim3((2 * len + 63) / 64), dim3(64), 0, st, a, b,
                       h, start, len, k_out, v_out);
    return hipGetLastError();
  });
}

hipError_t launch_tq_attend(const TqArgs& a, const TqAttendArgs& t, int mode, int group,
                            int nsplit, int batch, hipStream_t st) {
  return dispatch_dbits(a.head_dim, a.bits, [&](auto dd, auto bb) -> hipError_t {
    constexpr int D = decltype(dd)::value, B = decltype(bb)::value;
    switch (mode) {
      case 0: return attend_db<D, B, 0>(a, t, group, nsplit, batch, st);
      case 1: return attend_db<D, B, 1>(a, t, group, nsplit, batch, st);
      case 2: return attend_db<D, B, 2>(a, t, group, nsplit, batch, st);
      default: return hipErrorInvalidValue;
    }
  });
}

}  // namespace sai
