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

// appends of at least this many tokens per sequence go by page blocks
constexpr int kPageAppendMin = 4;

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
  const size_t src = (size_t)row * kLogicalDim<D>;  // [b][s][h][head_dim]
  const size_t esz = p.dtype == kDtypeBf16 ? 2 : 4;
  append_row_int8<D>((const uint8_t*)p.k + src * esz, (const uint8_t*)p.v + src * esz, p.dtype,
                     lane, pos, blk, pos % kPageTokens, p.do_rotary, p.interleaved != 0,
                     p.cos_cache, p.sin_cache);
}

// ---------------------------------------------------- int8, page blocks ----
// Multi-token appends: one workgroup per (sequence b, page, kv head h) block
// that receives new tokens, W = 16 L / 64 waves. Each wave takes 64/L slots,
// one per group of L lanes (wave w, group g: slot g*W + w); L = D/8, or 32 at
// the stored width 192. Lane c of a group holds stored dims [4c, 4c+4) and
// [D/2 + 4c, D/2 + 4c + 4): both elements of every split-half RoPE pair, and
// whole interleaved pairs, so RoPE needs no other lane (at width 192, lanes
// 21-23 hold the padding dims as zeros and lanes 24-31 nothing); a token's
// absolute maximum is a reduction over its group (DPP within rows of 16
// lanes, permlane16_swap across two rows). The codes
// are staged in LDS (K rows with a 16-byte pad, V as one 16-byte column per
// dim, placed so that one instruction's writes fall in distinct banks) and
// leave it in 16-byte stores, one per thread: K rows as contiguous pieces of
// the block, V columns whole, with the old bytes of slots outside the
// appended range kept. Per element the arithmetic is append_row_int8's (the
// quotient by the scale as in quant4_int8), so the codes and
// scales are the same bits.
// Four consecutive elements (f32 or bf16) at byte offset `off` of `base`.
template <bool BF16>
__device__ __forceinline__ void load4(const uint8_t* base, uint32_t off, float (&x)[4]) {
  if constexpr (BF16) {
    const uint2 w = *(const uint2*)(base + off);
    x[0] = __uint_as_float(w.x << 16), x[1] = __uint_as_float(w.x & 0xFFFF0000u);
    x[2] = __uint_as_float(w.y << 16), x[3] = __uint_as_float(w.y & 0xFFFF0000u);
  } else {
    const float4 v = *(const float4*)(base + off);
    x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
  }
}

template <int CTRL>
__device__ __forceinline__ uint32_t max_dpp(uint32_t v) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
  return v > o ? v : o;
}

// Maximum over aligned groups of L lanes (8, 16 or 32) of a non-negative,
// non-NaN float: its bits order as unsigned integers, and the maximum is
// order-free, so this equals wave_max over the same elements.
template <int L>
__device__ __forceinline__ float group_max(float x) {
  uint32_t v = __float_as_uint(x);
  v = max_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v = max_dpp<0x4E>(v);   // quad_perm [2,3,0,1]: every quad holds its maximum
  v = max_dpp<0x141>(v);  // row_half_mirror: the other quad of each 8
  if constexpr (L >= 16) v = max_dpp<0x140>(v);  // row_mirror: the other 8 of 16
  if constexpr (L >= 32) {
    // rows 0 and 1 (2 and 3) meet: one copy in each result
    const auto sw = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = sw[0] > sw[1] ? sw[0] : sw[1];
  }
  return __uint_as_float(v);
}

// a / 127 correctly rounded for a > 0, as q0 = a * RN(1/127) corrected once
// by its exact fma residual: equal to the IEEE quotient for every positive
// finite f32 (checked exhaustively on the CPU); for a = +inf, q is NaN and
// fminf gives +inf.
__device__ __forceinline__ float div127(float a) {
  constexpr float kInv127 = 0x1.020408p-7f;  // RN(1/127)
  const float q0 = a * kInv127;
  return fminf(__builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), kInv127, q0), a);
}

// The quotient x / s of append_row_int8 (s = fl(m / 127) for the row's
// maximum m >= |x|), taken without the division. r = 1/s from v_rcp_f32
// (within 1 ulp) when s is a normal finite float, NaN otherwise. Then
// |x / s| <= 127 (1 + 2^-23), x * r is within 1.5 * 2^-23 relative (2.3e-5)
// of x / s, and the correctly rounded quotient fl(x / s) within another
// 3.8e-6 (half an ulp at 128). Where x * r lies farther than 2^-14 from
// every half-integer, fl(x / s) falls in the same unit interval around the
// same integer n = rintf(x * r), which is then rintf(fl(x / s)), a code in
// [-127, 127]. quant4_fast returns those codes (packed LSB first) and flags
// the other elements (near a half-integer, or NaN) in `near`.
__device__ __forceinline__ uint32_t quant4_fast(const float (&x)[4], float r, bool (&near)[4]) {
#pragma clang fp contract(off)
  uint32_t w = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = x[j] * r;
    const float n = rintf(a);
    near[j] = !(fabsf(a - n) < 0.5f - 0x1p-14f);       // NaN too
    w |= ((uint32_t)(int32_t)n & 0xFFu) << (8 * j);  // a flagged element is redone
  }
  return w;
}

// Code of an element quant4_fast flagged. Near the half-integer h (|h| >= 1,
// s within [2^-100, 2^100]) it is settled exactly from e = fma(-h, s, x):
// its sign is that of x / s - h, and u = s * ulp(h)/2 is exact, so |e| < u
// means |x / s - h| < ulp(h)/2, fl(x / s) == h and the code is rintf(h)
// (the even neighbour); |e| > u means fl(x / s) lies beyond h on the side of
// e, inside the unit interval, and the code is h -+ 1/2. Everything else
// (|e| == u, NaN, tiny h, extreme scales) takes append_row_int8's own steps:
// the correctly rounded division, rintf, the saturating cast and the clamp
// (in float first, which gives the same integer; NaN gives 0).
__device__ __forceinline__ uint32_t quant_settle(float x, float s, float r) {
#pragma clang fp contract(off)
  const float a = x * r;
  const float h = floorf(a) + 0.5f;
  const float e = fmaf(-h, s, x);
  const float p2 = __uint_as_float(__float_as_uint(h) & 0x7F800000u);  // 2^exponent(h)
  const float u = s * p2 * 0x1p-24f;
  const bool ok = s >= 0x1p-100f && s <= 0x1p100f && fabsf(h) >= 1.0f && e == e;
  float code = fabsf(e) < u ? rintf(h) : (e > 0.0f ? h + 0.5f : h - 0.5f);
  if (!(ok && fabsf(e) != u)) code = rintf(x / s);
  const int32_t q = code == code ? (int32_t)fminf(fmaxf(code, -128.0f), 127.0f) : 0;
  return (uint32_t)q & 0xFFu;
}

// quant4_fast, then quant_settle for the flagged elements (a branch each,
// taken only when some lane flagged that element).
__device__ __forceinline__ uint32_t quant4_int8(const float (&x)[4], float s, float r) {
  bool near[4];
  uint32_t w = quant4_fast(x, r, near);
  if (near[0] | near[1] | near[2] | near[3]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (near[j]) w = (w & ~(0xFFu << (8 * j))) | (quant_settle(x[j], s, r) << (8 * j));
  }
  return w;
}

// ROPE: 0 none, 1 split halves (d, d + D/2), 2 interleaved (2i, 2i + 1).
// Grid (kv_heads, pages_per_seq, batch). The launch keeps s_new * kv_heads *
// D * 4 (the byte offset of a row within a sequence's new K or V) below 2^31.
template <int D>
constexpr int kPageLanes = D == 192 ? 32 : D / 8;  // lanes per token (a power of two)
template <int D>
constexpr int kPageThreads = kPageTokens * kPageLanes<D>;  // 2 D up to 256, 512 at 192

template <int D, bool BF16, int ROPE>
__global__ __launch_bounds__(kPageThreads<D>) void kv_append_page_int8_kernel(AppendParams p) {
  constexpr int L = kPageLanes<D>;
  constexpr int W = kPageThreads<D> / 64;  // waves: kPageTokens / (64 / L)
  constexpr int DL = kLogicalDim<D>;        // the caller's row width
  constexpr int HALF = D / 2;
  constexpr int HL = DL / 2;                // table entries per position
  constexpr int CS = D / 8;                 // lanes holding stored dims
  constexpr int CL = DL / 8;                // lanes holding the caller's dims
  constexpr int KS = D + 16;                // LDS K row stride (bytes)
  constexpr uint32_t ESZ = BF16 ? 2 : 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x, b = blockIdx.z;
  const int start = p.seq_lens[b];
  const int page_idx = start / kPageTokens + (int)blockIdx.y;
  const int t0 = page_idx * kPageTokens;  // position of slot 0
  const int lo = max(start, t0) - t0;     // new slots [lo, hi)
  const int hi = min(start + p.s_new, t0 + kPageTokens) - t0;
  if (lo >= hi) return;  // a page past the new tokens (the whole workgroup)
  const int page = p.page_table[(size_t)b * p.max_pages + page_idx];
  uint8_t* blk = p.pool + block_offset(page, h, p.num_pages, block_bytes_int8(D));
  const bool partial = lo > 0 || hi < kPageTokens;

  // threads D .. 2D-1 (waves from D/64 on) store V column tid - D: the old
  // column of a partial page first, so that its latency overlaps the work below
  const bool v_thread = tid >= D && tid < 2 * D;  // wave-uniform
  uint4 vold = uint4{0u, 0u, 0u, 0u};
  if (partial && v_thread) vold = *(const uint4*)(blk + (size_t)16 * D + (size_t)(tid - D) * 16);

  const int c = lane % L, g = lane / L;
  const int t = g * W + w;  // this group's slot
  // lanes past the caller's dims read lane CL-1's (and then hold zeros)
  const bool real = c < CL;
  const int cr = real ? c : CL - 1;
  // a slot outside the new range reads the nearest new row (its codes are
  // never stored), so every address stays inside the inputs
  const uint32_t srow = (uint32_t)min(max(t0 + t - start, 0), p.s_new - 1);
  const size_t row0 = ((size_t)b * p.s_new * p.kv_heads + h) * DL * ESZ;  // (b, token 0, h)
  const uint8_t* kbase = (const uint8_t*)p.k + row0;
  const uint8_t* vbase = (const uint8_t*)p.v + row0;
  const uint32_t off = (srow * (uint32_t)p.kv_heads * DL + 4 * cr) * ESZ;  // bytes
  float xa[4], xb[4], va[4], vb[4];
  load4<BF16>(kbase, off, xa);
  load4<BF16>(kbase, off + HL * ESZ, xb);
  load4<BF16>(vbase, off, va);
  load4<BF16>(vbase, off + HL * ESZ, vb);
  // the tables' rows from position start on
  const uint8_t* cos0 = (const uint8_t*)(p.cos_cache + (size_t)start * HL);
  const uint8_t* sin0 = (const uint8_t*)(p.sin_cache + (size_t)start * HL);
  if constexpr (ROPE == 1) {
    // dims 4c + j and HALF + 4c + j share table entry 4c + j
    const uint32_t o = (srow * HL + 4 * cr) * 4;
    const float4 cv = *(const float4*)(cos0 + o);
    const float4 sv = *(const float4*)(sin0 + o);
    const float ca[4] = {cv.x, cv.y, cv.z, cv.w}, sa[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x0 = xa[j], x1 = xb[j];
      xa[j] = rope_pair_elem(ca[j], sa[j], x0, x1, true);
      xb[j] = rope_pair_elem(ca[j], sa[j], x1, x0, false);
    }
  } else if constexpr (ROPE == 2) {
    // pair (2i, 2i + 1) uses entry i: 2c, 2c + 1 and HL/2 + 2c, + 1
    const uint32_t o = (srow * HL + 2 * cr) * 4;
    const float2 c0 = *(const float2*)(cos0 + o);
    const float2 s0 = *(const float2*)(sin0 + o);
    const float2 c1 = *(const float2*)(cos0 + o + HL * 2);
    const float2 s1 = *(const float2*)(sin0 + o + HL * 2);
    const float ca[2] = {c0.x, c0.y}, sa[2] = {s0.x, s0.y};
    const float cb[2] = {c1.x, c1.y}, sb[2] = {s1.x, s1.y};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float x0 = xa[2 * e], x1 = xa[2 * e + 1];
      xa[2 * e] = rope_pair_elem(ca[e], sa[e], x0, x1, true);
      xa[2 * e + 1] = rope_pair_elem(ca[e], sa[e], x1, x0, false);
      x0 = xb[2 * e], x1 = xb[2 * e + 1];
      xb[2 * e] = rope_pair_elem(cb[e], sb[e], x0, x1, true);
      xb[2 * e + 1] = rope_pair_elem(cb[e], sb[e], x1, x0, false);
    }
  }
  if constexpr (CL < L) {
    if (!real) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[j] = xb[j] = va[j] = vb[j] = 0.0f;
    }
  }
  // fmaxf from 0 skips NaN elements, as in append_row_int8: the lane maxima
  // are non-negative and never NaN
  float ak = 0.0f, av = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ak = fmaxf(ak, fmaxf(fabsf(xa[j]), fabsf(xb[j])));
    av = fmaxf(av, fmaxf(fabsf(va[j]), fabsf(vb[j])));
  }
  ak = group_max<L>(ak);
  av = group_max<L>(av);
  const float sk = (ak > 0.0f) ? div127(ak) : 1.0f;
  const float sv = (av > 0.0f) ? div127(av) : 1.0f;
  const float rk = (sk >= 0x1p-126f && sk <= 0x1.fffffep127f) ? __builtin_amdgcn_rcpf(sk)
                                                              : __builtin_nanf("");
  const float rv = (sv >= 0x1p-126f && sv <= 0x1.fffffep127f) ? __builtin_amdgcn_rcpf(sv)
                                                              : __builtin_nanf("");
  const uint32_t ka = quant4_int8(xa, sk, rk), kb = quant4_int8(xb, sk, rk);
  const uint32_t qa = quant4_int8(va, sv, rv), qb = quant4_int8(vb, sv, rv);

  __shared__ __align__(16) uint8_t sm_k[kPageTokens * KS];
  __shared__ __align__(16) uint8_t sm_v[kPageTokens * D];  // column d at 16 d
  if (CS == L || c < CS) {
    *(uint32_t*)&sm_k[t * KS + 4 * c] = ka;
    *(uint32_t*)&sm_k[t * KS + HALF + 4 * c] = kb;
    uint8_t* vcol = &sm_v[64 * c + t];  // dim 4c, slot t
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vcol[16 * j] = (uint8_t)(qa >> (8 * j));
      vcol[16 * (HALF + j)] = (uint8_t)(qb >> (8 * j));
    }
  }
  if (t >= lo && t < hi) {
    if (c == 0) ((float*)(blk + 32 * D))[t] = sk;
    if (c == 1) ((float*)(blk + 32 * D + 64))[t] = sv;
  }
  __syncthreads();

  if (tid < D) {
    // K: 16-byte piece tid of the 16 rows, stored when its row is new
    constexpr int CHUNKS = D / 16;  // pieces of a row
    const int tr = tid / CHUNKS;
    const uint4 v = *(const uint4*)&sm_k[tr * KS + 16 * (tid % CHUNKS)];
    if (tr >= lo && tr < hi) *(uint4*)(blk + (size_t)tid * 16) = v;
  } else if (v_thread) {
    // V: column d (16 slots), new slots from the tile, on a partial page the
    // others kept
    const int d = tid - D;
    uint4 v = *(const uint4*)&sm_v[16 * d];
    if (partial) {
      // byte k of word q is slot 4q + k: 0xFF where the slot keeps its code
      const uint32_t fresh = (1u << hi) - (1u << lo);  // bits lo .. hi-1
      uint32_t keep[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t nib = (~fresh >> (4 * q)) & 15u;
        keep[q] = ((nib * 0x00204081u) & 0x01010101u) * 0xFFu;
      }
      v.x = (v.x & ~keep[0]) | (vold.x & keep[0]);
      v.y = (v.y & ~keep[1]) | (vold.y & keep[1]);
      v.z = (v.z & ~keep[2]) | (vold.z & keep[2]);
      v.w = (v.w & ~keep[3]) | (vold.w & keep[3]);
    }
    *(uint4*)(blk + (size_t)16 * D + (size_t)d * 16) = v;
  }
}

// ---------------------------------------------------- int4, page blocks ----
// Multi-token int4 appends, one workgroup per (sequence b, page, kv head h)
// block, the int8 page kernel's thread layout: lane c of a token's L = D/8
// lanes holds dims [4c, 4c+4) and [D/2 + 4c, D/2 + 4c + 4), so a group of 32
// dims is 8 aligned lanes (its min/max: DPP within half-rows of 8) and RoPE
// stays in-lane. Per element the arithmetic is quant_int4_elem's (min/max
// over the group, scale and zero point rounded to binary16, the correctly
// rounded quotient and round_f32), so codes and parameters are the same
// bits. Codes are staged in LDS (K rows; V one byte per (dim, slot)) and
// leave in 16-byte stores: K rows of the new slots, V two dims' packed
// columns per thread with the nibbles of slots outside the appended range
// kept, and the (scale, zero) pairs of the new slots.

// min and max over the 8 aligned lanes of a group (quad swaps, then the other
// quad of the half-row); exact and order-free
__device__ __forceinline__ void group8_minmax(float& mn, float& mx) {
  mn = min_quad1032(mn);
  mx = max_quad1032(mx);
  mn = min_quad2301(mn);
  mx = max_quad2301(mx);
  mn = min_half_mirror(mn);
  mx = max_half_mirror(mx);
}

// Codes of this lane's 4 elements of a group held by 8 lanes (dims in lane
// order, then element order), and the group's binary16 (scale, zero) as one
// word (scale in the low half).
__device__ __forceinline__ uint32_t quant4_int4(const float (&x)[4], uint32_t& sz) {
#pragma clang fp contract(off)
  // The reference scans `if v < min { min = v }` / `if v > max { max = v }`
  // from +-inf: NaN never wins, as in fminf / fmaxf (the other operand).
  float mn = fminf(fminf(fminf(x[0], x[1]), fminf(x[2], x[3])), INFINITY);
  float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), -INFINITY);
  group8_minmax(mn, mx);
  if (mn == 0.0f) {
    // The scan keeps the first of equal minima, so a zero minimum has the
    // sign of the group's first zero in dim order (the stored binary16 zero
    // point keeps it). All 8 lanes of the group are here.
    float z = x[3] == 0.0f ? x[3] : 1.0f;
    z = x[2] == 0.0f ? x[2] : z;
    z = x[1] == 0.0f ? x[1] : z;
    z = x[0] == 0.0f ? x[0] : z;
    const uint64_t has = __ballot(z == 0.0f);
    const int base = (int)__lane_id() & ~7;
    mn = __shfl(z, base + __builtin_ctz((uint32_t)(has >> base) & 0xFFu), 64);
  }
  const float range = mx - mn;
  // range / 15 correctly rounded, as q0 = range * RN(1/15) corrected once by
  // its exact fma residual: equal to the IEEE quotient for every positive
  // finite f32 (checked exhaustively on the CPU).
  constexpr float kInv15 = 0x1.111112p-4f;  // RN(1/15)
  const float q0 = range * kInv15;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, 15.0f, range), kInv15, q0);
  // (for range = +inf, q is NaN and fminf gives +inf)
  const float scale = (range > 0.0f) ? fminf(q, range) : 1.0f;
  const _Float16 hs = (_Float16)scale;  // round to nearest even
  const _Float16 hz = (_Float16)mn;
  const float sf = (float)hs;
  const float zf = (float)hz;
  // The code round_f32 takes (half away from zero, `as u32`, min 15) of the
  // correctly rounded quotient t = (x - z) / s equals med3(rint(t'), 0, 15)
  // for t' = (x - z) * rcp(s) wherever t' lies farther than 2^-14 from every
  // half-integer: for |t| <= 16, t' is within 5e-6 of t (1 ulp of v_rcp_f32,
  // the product's and the division's half ulps), and farther out both clamp
  // alike. Anything else (near a tie, NaN, inf, a zero scale) takes the
  // reference's own steps below, for the whole wave when any lane needs
  // them. Codes are packed in f32 (exact, < 2^16).
  const float rf = __builtin_amdgcn_rcpf(sf);
  uint64_t slow = __ballot(!(sf > 0.0f));
  float acc = 0.0f;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    const float t = (x[j] - zf) * rf;
    const float r = rintf(t);
    slow |= __ballot(!(fabsf(t - r) <= 0.5f - 0x1p-14f));  // true for NaN
    const float c = __builtin_amdgcn_fmed3f(r, 0.0f, 15.0f);
    acc = j == 3 ? c : __builtin_fmaf(acc, 16.0f, c);
  }
  uint32_t w = (uint32_t)acc;  // codes packed LSB first
  if (slow) {
    w = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t v = 0u;
      if (sf > 0.0f) {
        // round_f32 of onnx-rt/src/kv_compression.rs:27-37, then `as u32`
        const float t = (x[j] - zf) / sf;
        const float tr = (float)sat_i32(t);
        const float fr = t - tr;
        const float rr = (fr >= 0.5f) ? tr + 1.0f : ((fr <= -0.5f) ? tr - 1.0f : tr);
        v = sat_u32(rr);
        v = v < 15u ? v : 15u;
      }
      w |= v << (4 * j);
    }
  }
  sz = (uint32_t)__builtin_bit_cast(uint16_t, hs) | ((uint32_t)__builtin_bit_cast(uint16_t, hz) << 16);
  return w;
}

// The 16 one-byte codes of a V column (slot s at byte s) as 8 bytes of
// nibble pairs, slot 2i in the low nibble of byte i.
__device__ __forceinline__ uint2 pack_column(const uint4 c) {
  auto pk = [](uint32_t a, uint32_t b) {
    const uint32_t u = (a | (a >> 4)) & 0x00FF00FFu;  // bytes 0, 2: slot pairs of a
    const uint32_t v = (b | (b >> 4)) & 0x00FF00FFu;
    return (u & 0xFFu) | ((u >> 8) & 0xFF00u) | ((v & 0xFFu) << 16) | ((v << 8) & 0xFF000000u);
  };
  return uint2{pk(c.x, c.y), pk(c.z, c.w)};
}

// HPW kv heads per workgroup (2 D threads each, up to 1024 threads): fewer,
// larger workgroups keep more of each CU's loads in flight.
template <int D, bool BF16, int ROPE, int HPW>
__global__ __launch_bounds__(2 * D * HPW) void kv_append_page_int4_kernel(AppendParams p) {
  constexpr int L = D / 8;    // lanes per token
  constexpr int W = D / 32;   // waves: kPageTokens / (64 / L)
  constexpr int HALF = D / 2;
  constexpr int NG = D / 32;  // groups of a row
  constexpr int KS = D / 2 + 16;  // LDS K row stride (bytes)
  constexpr uint32_t ESZ = BF16 ? 2 : 4;
  constexpr int PB = D / 8 < 16 ? D / 8 : 16;  // bytes of a (scale, zero) piece
  constexpr int PPS = (D / 8) / PB;            // pieces per slot
  // the workgroup's head of this thread
  const int sub = __builtin_amdgcn_readfirstlane((int)threadIdx.x / (2 * D));
  const int tid = (int)threadIdx.x % (2 * D), lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = (int)blockIdx.x * HPW + sub, b = blockIdx.z;
  const int start = p.seq_lens[b];
  const int page_idx = start / kPageTokens + (int)blockIdx.y;
  const int t0 = page_idx * kPageTokens;  // position of slot 0
  const int lo = max(start, t0) - t0;     // new slots [lo, hi)
  const int hi = min(start + p.s_new, t0 + kPageTokens) - t0;
  if (lo >= hi) return;  // a page past the new tokens (the whole workgroup)
  const int page = p.page_table[(size_t)b * p.max_pages + page_idx];
  uint8_t* blk = p.pool + block_offset(page, h, p.num_pages, block_bytes_int4(D));
  const bool partial = lo > 0 || hi < kPageTokens;

  // threads D/2 .. D-1 store V dims 2j, 2j + 1 (j = tid - D/2): the old
  // columns of a partial page first, so that their latency overlaps the work
  const bool vstore = tid >= D / 2 && tid < D;
  uint4 vold = uint4{0u, 0u, 0u, 0u};
  if (partial && vstore) vold = *(const uint4*)(blk + (size_t)8 * D + (size_t)(tid - D / 2) * 16);

  const int c = lane % L, g = lane / L;
  const int t = g * W + w;  // this group's slot
  // a slot outside the new range reads the nearest new row (its codes are
  // never stored), so every address stays inside the inputs
  const uint32_t srow = (uint32_t)min(max(t0 + t - start, 0), p.s_new - 1);
  const size_t row0 = ((size_t)b * p.s_new * p.kv_heads + h) * D * ESZ;  // (b, token 0, h)
  const uint8_t* kbase = (const uint8_t*)p.k + row0;
  const uint8_t* vbase = (const uint8_t*)p.v + row0;
  const uint32_t off = (srow * (uint32_t)p.kv_heads * D + 4 * c) * ESZ;  // bytes
  float xa[4], xb[4], va[4], vb[4];
  load4<BF16>(kbase, off, xa);
  load4<BF16>(kbase, off + HALF * ESZ, xb);
  load4<BF16>(vbase, off, va);
  load4<BF16>(vbase, off + HALF * ESZ, vb);
  const uint8_t* cos0 = (const uint8_t*)(p.cos_cache + (size_t)start * HALF);
  const uint8_t* sin0 = (const uint8_t*)(p.sin_cache + (size_t)start * HALF);
  if constexpr (ROPE == 1) {
    const uint32_t o = (srow * HALF + 4 * c) * 4;
    const float4 cv = *(const float4*)(cos0 + o);
    const float4 sv = *(const float4*)(sin0 + o);
    const float ca[4] = {cv.x, cv.y, cv.z, cv.w}, sa[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x0 = xa[j], x1 = xb[j];
      xa[j] = rope_pair_elem(ca[j], sa[j], x0, x1, true);
      xb[j] = rope_pair_elem(ca[j], sa[j], x1, x0, false);
    }
  } else if constexpr (ROPE == 2) {
    const uint32_t o = (srow * HALF + 2 * c) * 4;
    const float2 c0 = *(const float2*)(cos0 + o);
    const float2 s0 = *(const float2*)(sin0 + o);
    const float2 c1 = *(const float2*)(cos0 + o + HALF * 2);
    const float2 s1 = *(const float2*)(sin0 + o + HALF * 2);
    const float ca[2] = {c0.x, c0.y}, sa[2] = {s0.x, s0.y};
    const float cb[2] = {c1.x, c1.y}, sb[2] = {s1.x, s1.y};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float x0 = xa[2 * e], x1 = xa[2 * e + 1];
      xa[2 * e] = rope_pair_elem(ca[e], sa[e], x0, x1, true);
      xa[2 * e + 1] = rope_pair_elem(ca[e], sa[e], x1, x0, false);
      x0 = xb[2 * e], x1 = xb[2 * e + 1];
      xb[2 * e] = rope_pair_elem(cb[e], sb[e], x0, x1, true);
      xb[2 * e + 1] = rope_pair_elem(cb[e], sb[e], x1, x0, false);
    }
  }
  uint32_t pka, pkb, pva, pvb;  // (scale, zero) of the groups of xa, xb, va, vb
  const uint32_t ka = quant4_int4(xa, pka), kb = quant4_int4(xb, pkb);
  const uint32_t qa = quant4_int4(va, pva), qb = quant4_int4(vb, pvb);

  // per head: K rows; V column d at 16 d, one byte per slot; K and V (scale,
  // zero) per slot
  __shared__ __align__(16) uint8_t sm_k_all[HPW][kPageTokens * KS];
  __shared__ __align__(16) uint8_t sm_v_all[HPW][kPageTokens * D];
  __shared__ __align__(16) uint32_t sm_p_all[HPW][2][kPageTokens][NG];
  uint8_t* sm_k = sm_k_all[sub];
  uint8_t* sm_v = sm_v_all[sub];
  uint32_t(*sm_p)[kPageTokens][NG] = sm_p_all[sub];
  // K: the 4 codes of dims 4c.. (already nibbles, LSB first) are bytes 2c,
  // 2c + 1 of the row; those of D/2 + 4c.. bytes D/4 + 2c, + 1
  *(uint16_t*)&sm_k[t * KS + 2 * c] = (uint16_t)ka;
  *(uint16_t*)&sm_k[t * KS + D / 4 + 2 * c] = (uint16_t)kb;
  uint8_t* vcol = &sm_v[64 * c + t];  // dim 4c, slot t
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    vcol[16 * j] = (uint8_t)((qa >> (4 * j)) & 0xFu);
    vcol[16 * (HALF + j)] = (uint8_t)((qb >> (4 * j)) & 0xFu);
  }
  if ((c & 7) == 0) {  // the group's first lane: groups c/8 and NG/2 + c/8
    sm_p[0][t][c / 8] = pka;
    sm_p[0][t][NG / 2 + c / 8] = pkb;
    sm_p[1][t][c / 8] = pva;
    sm_p[1][t][NG / 2 + c / 8] = pvb;
  }
  __syncthreads();

  if (tid < D / 2) {
    // K: 16-byte piece tid of the 16 rows (D/32 per row), stored when its row is new
    constexpr int CHUNKS = D / 32;
    const int tr = tid / CHUNKS;
    const uint4 v = *(const uint4*)&sm_k[tr * KS + 16 * (tid % CHUNKS)];
    if (tr >= lo && tr < hi) *(uint4*)(blk + (size_t)tid * 16) = v;
  } else if (vstore) {
    // V: dims 2j, 2j + 1 (16 contiguous bytes), new slots from the tile, on a
    // partial page the other nibbles kept
    const int j = tid - D / 2;
    const uint2 c0 = pack_column(*(const uint4*)&sm_v[16 * (2 * j)]);
    const uint2 c1 = pack_column(*(const uint4*)&sm_v[16 * (2 * j + 1)]);
    uint4 v = uint4{c0.x, c0.y, c1.x, c1.y};
    if (partial) {
      // nibble s of a column's 64 bits is slot s: 0xF where the slot keeps its code
      const uint32_t fresh = (1u << hi) - (1u << lo);  // slots lo .. hi-1
      uint32_t keep[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t bits = (~fresh >> (8 * q)) & 0xFFu;  // slots 8q .. 8q+7
        uint32_t m = 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) m |= ((bits >> k) & 1u) * (0xFu << (4 * k));
        keep[q] = m;
      }
      v.x = (v.x & ~keep[0]) | (vold.x & keep[0]);
      v.y = (v.y & ~keep[1]) | (vold.y & keep[1]);
      v.z = (v.z & ~keep[0]) | (vold.z & keep[0]);
      v.w = (v.w & ~keep[1]) | (vold.w & keep[1]);
    }
    *(uint4*)(blk + (size_t)8 * D + (size_t)j * 16) = v;
  } else if (tid < D + 2 * kPageTokens * PPS) {
    // (scale, zero) pairs: K then V, PB-byte pieces, PPS per slot
    const int i = tid - D;
    const int which = i / (kPageTokens * PPS);
    const int slot = (i % (kPageTokens * PPS)) / PPS;
    const int piece = i % PPS;
    uint8_t* dst = blk + 16 * D + 64 * NG * which + (size_t)slot * (D / 8) + piece * PB;
    const uint8_t* src = (const uint8_t*)&sm_p[which][slot][0] + piece * PB;
    if (slot >= lo && slot < hi) {
      if constexpr (PB == 16)
        *(uint4*)dst = *(const uint4*)src;
      else
        *(uint2*)dst = *(const uint2*)src;
    }
  }
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

template <int D, bool BF16>
void launch_page_int8_dt(dim3 grid, hipStream_t st, const AppendParams& p, int rope) {
  if (rope == 0)
    hipLaunchKernelGGL((kv_append_page_int8_kernel<D, BF16, 0>), grid, dim3(kPageThreads<D>), 0, st, p);
  else if (rope == 1)
    hipLaunchKernelGGL((kv_append_page_int8_kernel<D, BF16, 1>), grid, dim3(kPageThreads<D>), 0, st, p);
  else
    hipLaunchKernelGGL((kv_append_page_int8_kernel<D, BF16, 2>), grid, dim3(kPageThreads<D>), 0, st, p);
}

template <int D>
void launch_page_int8(dim3 grid, hipStream_t st, const AppendParams& p, bool bf, int rope) {
  if (bf)
    launch_page_int8_dt<D, true>(grid, st, p, rope);
  else
    launch_page_int8_dt<D, false>(grid, st, p, rope);
}

template <int D, bool BF16, int HPW>
void launch_page_int4_hpw(dim3 grid, hipStream_t st, const AppendParams& p, int rope) {
  grid.x /= HPW;
  const dim3 block(2 * D * HPW);
  if (rope == 0)
    hipLaunchKernelGGL((kv_append_page_int4_kernel<D, BF16, 0, HPW>), grid, block, 0, st, p);
  else if (rope == 1)
    hipLaunchKernelGGL((kv_append_page_int4_kernel<D, BF16, 1, HPW>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((kv_append_page_int4_kernel<D, BF16, 2, HPW>), grid, block, 0, st, p);
}

// Below head_dim 256, up to 1024 threads per workgroup: the most kv heads (a
// power of two, at most 512 / D) that divide the kv head count. (Building a
// 4 x 32768-token cache of 8 kv heads at head_dim 128 from f32 rows: 36.1 us
// per 131,072 rows with one head per workgroup, 34.8 with two, 32.1 with
// four; at head_dim 256 two heads measured the same as one.)
template <int D, bool BF16>
void launch_page_int4_dt(dim3 grid, hipStream_t st, const AppendParams& p, int rope) {
  if constexpr (D <= 64) {
    if (p.kv_heads % 8 == 0) return launch_page_int4_hpw<D, BF16, 8>(grid, st, p, rope);
  }
  if constexpr (D <= 128) {
    if (p.kv_heads % 4 == 0) return launch_page_int4_hpw<D, BF16, 4>(grid, st, p, rope);
    if (p.kv_heads % 2 == 0) return launch_page_int4_hpw<D, BF16, 2>(grid, st, p, rope);
  }
  launch_page_int4_hpw<D, BF16, 1>(grid, st, p, rope);
}

template <int D>
void launch_page_int4(dim3 grid, hipStream_t st, const AppendParams& p, bool bf, int rope) {
  if (bf)
    launch_page_int4_dt<D, true>(grid, st, p, rope);
  else
    launch_page_int4_dt<D, false>(grid, st, p, rope);
}

}  // namespace

hipError_t launch_kv_append(const AppendParams& p, int head_dim, int quant, hipStream_t st) {
  // the page kernel reads 8 or 16 bytes of a row at once: rows must start
  // 16-byte aligned; its grid is (kv_heads, pages, batch) and its in-sequence
  // row offsets are 32-bit
  const bool aligned = (((uintptr_t)p.k | (uintptr_t)p.v) & 15u) == 0;
  // the host's exact count when given, else one more than s_new spans (any
  // start)
  const int pages = p.pages > 0 ? p.pages : (p.s_new + kPageTokens - 1) / kPageTokens + 1;
  const bool fits = pages <= 65535 && p.batch <= 65535 &&
                    (long)p.s_new * p.kv_heads * head_dim * 4 < (1L << 31);
  if (p.s_new >= kPageAppendMin && aligned && fits && (quant == kQuantInt8 || quant == kQuantInt4)) {
    const dim3 grid((unsigned)p.kv_heads, (unsigned)pages, (unsigned)p.batch);
    const bool bf = p.dtype == kDtypeBf16;
    const int rope = !p.do_rotary ? 0 : (p.interleaved ? 2 : 1);
    auto by_dim = [&](auto launch64, auto launch128, auto launch256) {
      if (head_dim == 64)
        launch64(grid, st, p, bf, rope);
      else if (head_dim == 128)
        launch128(grid, st, p, bf, rope);
      else if (head_dim == 256)
        launch256(grid, st, p, bf, rope);
      else
        return hipErrorInvalidValue;
      return hipGetLastError();
    };
    if (quant == kQuantInt8 && head_dim == 168) {
      launch_page_int8<192>(grid, st, p, bf, rope);
      return hipGetLastError();
    }
    if (quant == kQuantInt8)
      return by_dim(launch_page_int8<64>, launch_page_int8<128>, launch_page_int8<256>);
    return by_dim(launch_page_int4<64>, launch_page_int4<128>, launch_page_int4<256>);
  }
  if (quant == kQuantInt8) {
    const long rows = (long)p.batch * p.s_new * p.kv_heads;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (head_dim == 64)
      hipLaunchKernelGGL(kv_append_int8_kernel<64>, grid, dim3(256), 0, st, p);
    else if (head_dim == 128)
      hipLaunchKernelGGL(kv_append_int8_kernel<128>, grid, dim3(256), 0, st, p);
    else if (head_dim == 256)
      hipLaunchKernelGGL(kv_append_int8_kernel<256>, grid, dim3(256), 0, st, p);
    else if (head_dim == 168)
      hipLaunchKernelGGL(kv_append_int8_kernel<192>, grid, dim3(256), 0, st, p);
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
    else if (head_dim == 256)
      hipLaunchKernelGGL(kv_append_int4_kernel<256>, grid, dim3(256), 0, st, p, pairs);
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
