// Kernel 3: prefill chunk -- causal GQA attention of sq new query tokens per
// sequence over the paged int8 or int4 cache (past + the chunk, already
// appended by kernel 1), on f16 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Workgroup = 8 waves = 256 attention rows = (256/G query positions) x (G
// heads of one kv head), so every K/V tile is loaded once per workgroup and
// shared by the whole GQA group; each wave owns two 16-row blocks.
// Per 64-token KV tile (4 pages):
//   staging  the next tile's codes and scales are loaded into registers while
//            the current tile is computed, then written as f16 into the other
//            half of a double-buffered LDS tile: K token-major, V in the
//            permuted k-order of the PV operand; rows padded so the 16-byte
//            LDS reads are conflict-free. One barrier per tile. int8 codes are
//            stored exactly (|code| <= 128) and their per-token scales applied
//            to the scores and to P; int4 codes are dequantised while staged.
//   S^T      A = K tile (LDS), B = Q^T (registers, f16 of q * scale * log2 e);
//            lane (row r, g) receives tokens 4g+e of each 16-token block, so
//            the row softmax is in-lane plus two cross-group reductions and P
//            feeds the PV A operand straight from registers. Each K fragment
//            read from LDS serves both row blocks of the wave.
//   PV       A = P * s_v (f16), B = V (LDS f16); each V fragment serves both
//            row blocks.
// Scores: s = <q', k> * s_k[t], online softmax in the log2 domain against a
// per-row reference point that moves only when a tile's scores rise more than
// kMaxLead above it (so most tiles skip the accumulator rescale). Only tiles
// that cross the causal diagonal (or the end of the sequence), or the first
// key of a sliding window, apply the mask.
#include <type_traits>

#include "sai_internal.h"

namespace sai {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

// RoPE of one element; both products rounded on their own, branch-free.
__device__ __forceinline__ float rope_elem(float c, float s, float own, float partner,
                                           bool first) {
#pragma clang fp contract(off)
  const float a = c * own;
  const float b = s * partner;
  return a + (first ? -b : b);
}

// 4 int8 codes (one dword) -> 4 exact f16 values, as two packed halves:
// f16 bits 0x6400 | (code ^ 0x80) = 1024 + code + 128, minus 1152.
__device__ __forceinline__ void codes4_to_f16(uint32_t w, uint32_t& h01, uint32_t& h23) {
  const uint32_t u = w ^ 0x80808080u;
  uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  v2h ha = __builtin_bit_cast(v2h, a) - v2h{(_Float16)1152.0f, (_Float16)1152.0f};
  v2h hb = __builtin_bit_cast(v2h, b) - v2h{(_Float16)1152.0f, (_Float16)1152.0f};
  h01 = __builtin_bit_cast(uint32_t, ha);
  h23 = __builtin_bit_cast(uint32_t, hb);
}

// max / sum over the four lane groups (lanes r, r+16, r+32, r+48), on the
// VALU lane-swap instructions rather than LDS permutes
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
// max over the whole wave: within each row of 16 lanes on DPP moves (quad
// swaps, then rotations by 4 and 8), then across the four rows
__device__ __forceinline__ float wave_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value,
                                                      0xF, 0xF, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm 1,0,3,2
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm 2,3,0,1
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
  return xgroup_max(v);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// How far (log2 units) a row's scores may rise above its reference point
// before the reference moves: softmax weights stay <= 2^kMaxLead = 4.
constexpr float kMaxLead = 2.0f;
// Fast-path bounds: the PV operand (p * s_v, or p * s_v / max(s_v) on a
// large-V tile) <= kFastSum (inside binary16), row sums <= kFastCap
constexpr float kFastSum = 32768.0f;
constexpr float kFastCap = 1048576.0f;
// int8 tiles whose largest V scale exceeds this (|v| above 32) take the
// exact-weight PV: the operand is p * s_v / max(s_v) (at most p, whatever
// the V magnitude) split into binary16 hi + lo (~22 significant bits instead
// of 11), and the tile's product is scaled by max(s_v) in f32. A single
// binary16 weight's 2^-11 rounding times |v| would otherwise dominate the
// error of outputs that cancel far below |v|.
constexpr float kBigVScale = 0.25f;
// int4 V is staged as f16 of v * 2^-5 and the weights as f16 of p * 2^5:
// |v| <= 16 * 65504 for binary16 (scale, zero), so the staged values stay
// finite, and the product p * v is unchanged.
constexpr float kInt4VDown = 0.03125f;
constexpr float kInt4PUp = 32.0f;
// The precise pass takes its weights 2^kPrecLift larger (an exact shift of the
// scores, undone in the row sums and at the output): its PV operand p * s_v /
// 2^vexp then spans up to 2^kPrecLift instead of 1, so the lo half of a
// small weight stays a normal binary16 rather than falling to the 2^-24
// subnormal step, which times |v| ~ 2^vexp would dominate the error.
constexpr int kPrecLift = 12;

// V fragments read ahead of the PV MFMAs that consume them
constexpr int kVPrefetch = 6;
constexpr int kVPrefetchInt4 = 3;  // int4 keeps its K lo tile reads and has fewer spare registers

template <int D, bool KLO = false>
struct PrefillTile {
  static constexpr int KROW = D + 8;      // padded f16 row of the K tile
  static constexpr int VROW = 4 * 8 + 8;  // padded f16 (kstep, dim) row: 4 groups x 8
  // every member 16-byte aligned: fragments are read with ds_read_b128
  alignas(16) _Float16 k[64 * KROW];
  alignas(16) _Float16 klo[KLO ? 64 * KROW : 8];  // int4: K - f16(K), hi + lo hold K to ~22 bits
  alignas(16) _Float16 v[2 * D * VROW];
  alignas(16) float sk[64];
  alignas(16) float sv[64];
  // int8: the V scales above are divided by the tile's power of two vsig
  // (1 unless the largest scale exceeds kBigVScale), svmax is their largest
  // (at most kBigVScale) and vexp = log2(vsig)
  float svmax;
  int vexp;
};

// Codes and scales of one 64-token tile, held in registers between the load
// and the LDS store: K chunks (token, 16 dims), V chunks (page, dim), and one
// scale per thread for the first 128 threads.
template <int D, int NT>
struct TileStage {
  static constexpr int KN = 64 * (D / 16);      // 16-byte K chunks of a tile
  static constexpr int VN = 4 * D;              // 16-byte V chunks of a tile
  static constexpr int KC = (KN + NT - 1) / NT;  // per thread
  static constexpr int VC = (VN + NT - 1) / NT;
  uint4 kc[KC];
  uint4 vc[VC];
  float sc;
};

// Page ids (pool blocks) a thread's staging loads of one 64-token tile touch:
// chunk i of the K and V loads (c = tid + NT i) lies in local page c / D for
// int8, and in c / (16 * D/32) (K) and c / D (V) for int4; the first 128
// threads (int8) also load one scale of token tid & 63. They are loaded one
// tile ahead, so the tile's code loads never wait on a page-table read.
template <int D, int NT, bool INT4>
struct StagePages {
  static constexpr int KN = INT4 ? 64 * (D / 32) : 64 * (D / 16);  // K chunks of a tile
  static constexpr int VN = 4 * D;                                  // V chunks of a tile
  static constexpr int KC = (KN + NT - 1) / NT;
  static constexpr int VC = (VN + NT - 1) / NT;
  int k[KC];
  int v[VC];
  int s;

  __device__ __forceinline__ void load(const int32_t* pt, int tile, int last_page, int tid) {
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int c = min(tid + NT * i, KN - 1);
      const int lp = INT4 ? c / (16 * (D / 32)) : c / D;
      k[i] = pt[min(4 * tile + lp, last_page)];
    }
#pragma unroll
    for (int i = 0; i < VC; ++i) {
      const int c = min(tid + NT * i, VN - 1);
      v[i] = pt[min(4 * tile + c / D, last_page)];
    }
    s = INT4 ? 0 : pt[min(4 * tile + (tid & 63) / kPageTokens, last_page)];
  }
};

// A kv head's page blocks are contiguous in the pool (block_offset), so a
// block's address is the head's base plus page * block bytes: one 32 x 32 ->
// 64-bit multiply-add (page ids are non-negative). Tiles start at multiples of
// 64 tokens, so a tile token's slot in its page is token & 15.
__device__ __forceinline__ const uint8_t* head_blocks(const PrefillParams& p, int kvh, size_t bb) {
  return p.pool + block_offset(0, kvh, p.num_pages, bb);
}
__device__ __forceinline__ const uint8_t* page_block(const uint8_t* head, int page, size_t bb) {
  return head + (uint64_t)(uint32_t)page * bb;
}

template <int D, int NT>
__device__ __forceinline__ void stage_load(TileStage<D, NT>& S, const PrefillParams& p,
                                           const StagePages<D, NT, false>& P, int kvh, int t0,
                                           int tid) {
  constexpr size_t BB = block_bytes_int8(D);
  const uint8_t* head = head_blocks(p, kvh, BB);
#pragma unroll
  for (int i = 0; i < TileStage<D, NT>::KC; ++i) {
    const int c = tid + NT * i;
    if (TileStage<D, NT>::KN % NT != 0 && c >= TileStage<D, NT>::KN) break;
    const int tok = c / (D / 16);
    const int dp = c % (D / 16);
    S.kc[i] = *(const uint4*)(page_block(head, P.k[i], BB) + (tok & 15) * D + 16 * dp);
  }
#pragma unroll
  for (int i = 0; i < TileStage<D, NT>::VC; ++i) {
    const int c = tid + NT * i;
    if (TileStage<D, NT>::VN % NT != 0 && c >= TileStage<D, NT>::VN) break;
    const int d = c % D;
    S.vc[i] = *(const uint4*)(page_block(head, P.v[i], BB) + 16 * D + d * 16);
  }
  // the first 128 threads load one scale each; tokens past the sequence end
  // are zeroed when the tile is stored (a select here would wait for the load)
  S.sc = 0.0f;
  if (tid < 128) {
    const int which = tid >> 6;
    const int tok = tid & 63;
    S.sc = ((const float*)(page_block(head, P.s, BB) + 32 * D + 64 * which))[tok & 15];
  }
}

template <int D, int NT, class Tile>
__device__ __forceinline__ void stage_store(const TileStage<D, NT>& S, Tile& T, int t0, int total,
                                            int tid) {
  constexpr int KROW = Tile::KROW;
  constexpr int VROW = Tile::VROW;
#pragma unroll
  for (int i = 0; i < TileStage<D, NT>::KC; ++i) {
    const int c = tid + NT * i;
    if (TileStage<D, NT>::KN % NT != 0 && c >= TileStage<D, NT>::KN) break;
    const int tok = c / (D / 16);
    const int dp = c % (D / 16);
    uint32_t h[8];
    codes4_to_f16(S.kc[i].x, h[0], h[1]);
    codes4_to_f16(S.kc[i].y, h[2], h[3]);
    codes4_to_f16(S.kc[i].z, h[4], h[5]);
    codes4_to_f16(S.kc[i].w, h[6], h[7]);
    uint4* dst = (uint4*)(T.k + tok * KROW + 16 * dp);
    dst[0] = uint4{h[0], h[1], h[2], h[3]};
    dst[1] = uint4{h[4], h[5], h[6], h[7]};
  }
#pragma unroll
  for (int i = 0; i < TileStage<D, NT>::VC; ++i) {
    const int c = tid + NT * i;
    if (TileStage<D, NT>::VN % NT != 0 && c >= TileStage<D, NT>::VN) break;
    const int cb = c / D;
    const int d = c % D;
    // slot s of page cb = token 16*cb + s: k step cb>>1, group s>>2, element
    // (cb&1)*4 + (s&3) of the PV operand's k-order
    _Float16* row = T.v + ((size_t)(cb >> 1) * D + d) * VROW;
    const int half = (cb & 1) * 4;
    const uint32_t ws[4] = {S.vc[i].x, S.vc[i].y, S.vc[i].z, S.vc[i].w};
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      uint32_t h01, h23;
      codes4_to_f16(ws[gg], h01, h23);
      *(uint2*)(row + gg * 8 + half) = uint2{h01, h23};
    }
  }
  if (tid < 128) {
    const float sc = t0 + (tid & 63) < total ? S.sc : 0.0f;
    if (tid < 64) {
      T.sk[tid] = sc;
    } else if (__builtin_amdgcn_readfirstlane(tid >> 6) == 1) {
      // the second wave holds the 64 V scales: their maximum m bounds the
      // PV operand. Above kBigVScale they are divided by the power of two
      // 2^e >= m / kBigVScale (exact), so the operand stays <= p * kBigVScale
      const float m = wave_max(sc);
      const int e = m > kBigVScale ? __builtin_amdgcn_frexp_expf(m * (1.0f / kBigVScale)) : 0;
      T.sv[tid - 64] = __builtin_ldexpf(sc, -e);
      if (tid == 64) {
        T.svmax = __builtin_ldexpf(m, -e);
        T.vexp = e;
      }
    }
  }
}

// ---- int4 cache: the same LDS tile, filled with dequantised f16 values -------
// A group's scale and zero vary along head_dim, so they cannot be applied after
// the dot product: K and V are dequantised while staged (code * s + z in f32,
// rounded once to f16; the binary16 parameters bound the range anyway), and
// the softmax then uses unit token scales. Tokens past the sequence end are
// zeroed so a stale slot can never inject a NaN into the PV product.
template <int D, int NT>
struct TileStage4 {
  static constexpr int NG = D / 32;
  static constexpr int KN = 64 * NG;             // K chunks: (token, group), 16 B
  static constexpr int VN = 4 * D;               // V chunks: (page, dim), 8 B
  static constexpr int KC = (KN + NT - 1) / NT;  // per thread
  static constexpr int VC = (VN + NT - 1) / NT;
  uint4 kc[KC];
  uint32_t kp[KC];      // (scale, zero) binary16 pair of the K chunk's group
  uint2 vc[VC];
  uint32_t vp[VC][16];  // (scale, zero) of each of the V chunk's 16 slots
};

__device__ __forceinline__ float half_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

template <int D, int NT>
__device__ __forceinline__ void stage_load4(TileStage4<D, NT>& S, const PrefillParams& p,
                                            const StagePages<D, NT, true>& P, int kvh, int t0,
                                            int tid) {
  constexpr size_t BB = block_bytes_int4(D);
  constexpr int NG = D / 32;
  static_assert(StagePages<D, NT, true>::KC == TileStage4<D, NT>::KC &&
                StagePages<D, NT, true>::VC == TileStage4<D, NT>::VC, "chunk counts");
  const uint8_t* head = head_blocks(p, kvh, BB);
#pragma unroll
  for (int i = 0; i < TileStage4<D, NT>::KC; ++i) {
    const int c = min(tid + NT * i, TileStage4<D, NT>::KN - 1);  // spare threads repeat the last
    const int tok = c / NG;
    const int grp = c % NG;
    const uint8_t* blk = page_block(head, P.k[i], BB);
    const int slot = tok & 15;
    S.kc[i] = *(const uint4*)(blk + slot * (D / 2) + 16 * grp);
    S.kp[i] = *(const uint32_t*)(blk + 16 * D + (slot * NG + grp) * 4);
  }
#pragma unroll
  for (int i = 0; i < TileStage4<D, NT>::VC; ++i) {
    const int c = min(tid + NT * i, TileStage4<D, NT>::VN - 1);
    const int d = c % D;
    const uint8_t* blk = page_block(head, P.v[i], BB);
    S.vc[i] = *(const uint2*)(blk + 8 * D + d * 8);
    const uint8_t* par = blk + 16 * D + 64 * NG + (d / 32) * 4;
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) S.vp[i][sl] = *(const uint32_t*)(par + (size_t)sl * NG * 4);
  }
}

template <int D, int NT>
__device__ __forceinline__ void stage_store4(const TileStage4<D, NT>& S, PrefillTile<D, true>& T,
                                             int t0, int total, int tid) {
  constexpr int KROW = PrefillTile<D, true>::KROW;
  constexpr int VROW = PrefillTile<D, true>::VROW;
  constexpr int NG = D / 32;
#pragma unroll
  for (int i = 0; i < TileStage4<D, NT>::KC; ++i) {
    const int c = tid + NT * i;
    if (c >= TileStage4<D, NT>::KN) break;
    const int tok = c / NG;
    const int grp = c % NG;
    const bool valid = t0 + tok < total;
    const float sc = half_lo(S.kp[i]), zr = half_hi(S.kp[i]);
    const uint32_t w[4] = {S.kc[i].x, S.kc[i].y, S.kc[i].z, S.kc[i].w};
    uint32_t h[16], l[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      // elements 2j, 2j+1: nibbles 2j, 2j+1 of the chunk (LSB first); the
      // value code * s + z (code * s exact in f32) as an f16 pair hi + lo
      const uint32_t wj = w[j >> 2] >> (8 * (j & 3));
      float a = valid ? (float)(wj & 0xF) * sc + zr : 0.0f;
      float b = valid ? (float)((wj >> 4) & 0xF) * sc + zr : 0.0f;
      // one rounded value feeds both halves of the split
      __asm__("" : "+v"(a), "+v"(b));
      const _Float16 ah = (_Float16)a, bh = (_Float16)b;
      h[j] = __builtin_bit_cast(uint32_t, v2h{ah, bh});
      l[j] = __builtin_bit_cast(uint32_t, v2h{(_Float16)(a - (float)ah), (_Float16)(b - (float)bh)});
    }
    uint4* dst = (uint4*)(T.k + tok * KROW + 32 * grp);
    uint4* dlo = (uint4*)(T.klo + tok * KROW + 32 * grp);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dst[q] = uint4{h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]};
      dlo[q] = uint4{l[4 * q], l[4 * q + 1], l[4 * q + 2], l[4 * q + 3]};
    }
  }
#pragma unroll
  for (int i = 0; i < TileStage4<D, NT>::VC; ++i) {
    const int c = tid + NT * i;
    if (c >= TileStage4<D, NT>::VN) break;
    const int cb = c / D;
    const int d = c % D;
    const uint32_t w[2] = {S.vc[i].x, S.vc[i].y};
    float val[16];
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) {
      const uint32_t nib = (w[sl >> 3] >> (4 * (sl & 7))) & 0xF;
      const bool valid = t0 + 16 * cb + sl < total;
      // exact power-of-two scaling after the f32 dequantisation
      val[sl] = valid ? ((float)nib * half_lo(S.vp[i][sl]) + half_hi(S.vp[i][sl])) * kInt4VDown
                      : 0.0f;
    }
    // slot s of page cb: k step cb>>1, group s>>2, element (cb&1)*4 + (s&3)
    _Float16* row = T.v + ((size_t)(cb >> 1) * D + d) * VROW;
    const int half = (cb & 1) * 4;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const uint32_t h01 = __builtin_bit_cast(
          uint32_t, v2h{(_Float16)val[4 * gg], (_Float16)val[4 * gg + 1]});
      const uint32_t h23 = __builtin_bit_cast(
          uint32_t, v2h{(_Float16)val[4 * gg + 2], (_Float16)val[4 * gg + 3]});
      *(uint2*)(row + gg * 8 + half) = uint2{h01, h23};
    }
  }
}

// RB row blocks of 16 attention rows per wave: 2 up to head_dim 128, 1 at
// the stored widths 192 and 256 (the query pair and the accumulators of two
// blocks would not fit).
// PREC: the int8 precise pass (see the tile loop below): only workgroups
// whose flag the fast pass set run, from their first tile.
template <int D, int G, int NW, int Q, bool PREC>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gqa_prefill_kernel(PrefillParams p) {
  constexpr int NT = 64 * NW;
  constexpr int KS = D / 32;      // 32-dim k steps of QK
  constexpr int JB = D / 16;      // 16-dim column blocks of PV
  constexpr int RB = D > 128 ? 1 : 2;
  constexpr int QT = 16 * RB * NW / G;  // query positions per workgroup
  constexpr bool INT4 = Q == kQuantInt4;
  typedef PrefillTile<D, INT4> Tile;
  constexpr int KROW = Tile::KROW;
  constexpr int VROW = Tile::VROW;
  constexpr int HALF = D / 2;
  constexpr int DL = kLogicalDim<D>;  // the caller's rows (q, out)
  constexpr int HL = DL / 2;          // table entries per position

  // int8 at head_dim <= 128 keeps four tiles in LDS and computes two per
  // barrier (4 x 38.4 KB at 128); int4 up to 128 and int8 at 256 keep two;
  // int4 at 256 (an f16 hi + lo K tile and the V tile, 109 KB) keeps one and
  // stages behind a second barrier
  constexpr int NSLOT = (!INT4 && D <= 128) ? 4 : ((INT4 && D > 128) ? 1 : 2);
  constexpr int PER_BARRIER = NSLOT == 4 ? 2 : 1;
  __shared__ Tile sT[NSLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  // the workgroup's large-V flag: set by the fast pass, taken (and cleared,
  // so the flags are zero between launches) by the precise pass
  int32_t* const prec_flag =
      p.prec_flags + ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  if constexpr (PREC) {
    if (__builtin_amdgcn_readfirstlane(*prec_flag) == 0) return;  // uniform
    __syncthreads();  // every wave has read it
    if (tid == 0) *prec_flag = 0;
  }
  const int n_qt = (p.sq + QT - 1) / QT;
  const int nks = p.nksplit > 1 ? p.nksplit : 1;
  const int ksp = (int)blockIdx.x % nks;               // key split
  const int qtile = n_qt - 1 - (int)blockIdx.x / nks;  // longest rows first
  const int q0 = qtile * QT;
  const int past = p.seq_lens[b];
  const int total = past + p.sq;
  const int Hq = p.kv_heads * G;
  const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
  const int last_page = (total - 1) / kPageTokens;
  const int max_pos = past + min(q0 + QT, p.sq) - 1;
  const int n_tiles = max_pos / 64 + 1;
  // tiles entirely at or below the smallest position of the workgroup need
  // no causal mask (they are also inside the sequence)
  const int full_tiles = (past + q0 + 1) / 64;
  // sliding window (W keys per row, W > 0): the rows see keys from
  // past + q0 - W + 1 on, so earlier tiles are skipped; tiles before lo_full
  // hold keys that some row of the workgroup does not see
  const int W = p.window;
  const int tile_lo = W > 0 ? max(0, past + q0 - W + 1) / 64 : 0;
  const int lo_full = W > 0 ? (max(0, max_pos - W + 1) + 63) / 64 : 0;
  // this workgroup's tiles [t_first, t_last): the rows' whole range, or its
  // key split's share of it
  const int t_first = nks > 1 ? tile_lo + ksp * p.ksplit_tiles : tile_lo;
  const int t_last = nks > 1 ? min(n_tiles, t_first + p.ksplit_tiles) : n_tiles;
  // partial of row R (position il, head R % G) of this key split
  auto partial_of = [&](int il, int hd) {
    return p.partials +
           ((((size_t)b * p.sq + il) * nks + ksp) * p.kv_heads + kvh) * (size_t)(G * (D + 2)) +
           (size_t)hd * (D + 2);
  };
  if (nks > 1 && t_first >= t_last) {
    // a split past the rows' range: empty partials (m = -inf, l = o = 0), which
    // the merge skips
    if constexpr (!PREC) {
      for (int e = tid; e < 16 * RB * NW * (D + 2); e += NT) {
        const int R = e / (D + 2), k = e % (D + 2);
        const int il = q0 + R / G;
        if (il < p.sq) partial_of(il, R % G)[k] = k == 0 ? -INFINITY : 0.0f;
      }
    }
    return;
  }

  // first tile in flight while Q is prepared
  typedef typename std::conditional<INT4, TileStage4<D, NT>, TileStage<D, NT>>::type Stage;
  Stage S;
  StagePages<D, NT, INT4> pages;  // page ids of the next tile to load
  auto load_stage = [&](int t0) {
    if constexpr (INT4)
      stage_load4<D, NT>(S, p, pages, kvh, t0, tid);
    else
      stage_load<D, NT>(S, p, pages, kvh, t0, tid);
  };
  auto store_stage = [&](Tile& T, int t0) {
    if constexpr (INT4)
      stage_store4<D, NT>(S, T, t0, total, tid);
    else
      stage_store<D, NT>(S, T, t0, total, tid);
  };
  auto slot = [&](int tile) -> Tile& { return sT[(tile - t_first) & (NSLOT - 1)]; };
  pages.load(pt, t_first, last_page, tid);
  load_stage(t_first * 64);
  pages.load(pt, t_first + 1, last_page, tid);

  // ---- Q^T operand: rows R = wave*32 + rb*16 + r -> (position, head) -------
  // RoPE(q) * scale * log2(e) as an f16 pair hi + lo (~22 bits: a score's
  // rounding error stays ~2^-20 of its largest term, outlier channels
  // included); lane (r, g) holds dims 32ks + 8g .. +7
  v8h qB[RB][KS], qL[RB][KS];
  int qpos[RB];  // absolute position of the row (clamped for dead rows)
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int R = wave * (16 * RB) + rb * 16 + r;
    const int il = q0 + R / G;
    const int hq = kvh * G + R % G;
    const int i = il < p.sq ? il : p.sq - 1;
    const int pos = past + i;
    qpos[rb] = il < p.sq ? pos : -1;
    const size_t qbase = (((size_t)b * p.sq + i) * Hq + hq) * DL;
    float x[KS][8];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // stored dim -> the caller's dim (padding dims of the stored width
        // 192 are 0)
        const int dl = logical_dim<D>(32 * ks + 8 * g + e);
        x[ks][e] = load_elem(p.q, qbase + (dl < 0 ? 0 : dl), p.q_dtype);
        if (dl < 0) x[ks][e] = 0.0f;
      }
    if (p.do_rotary) {
      // partners: interleaved d ^ 1 (same chunk); split-half d +- D/2 (chunk
      // ks +- KS/2, the same lane)
      float y[KS][8];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 32 * ks + 8 * g + e;
          const int dl = logical_dim<D>(d);
          const bool first = p.interleaved ? (e & 1) == 0 : d < HALF;
          const int pi = dl < 0 ? 0 : (p.interleaved ? (dl >> 1) : (first ? d : d - HALF));
          const float partner = p.interleaved ? x[ks][e ^ 1] : x[(ks + KS / 2) % KS][e];
          y[ks][e] = rope_elem(p.cos_cache[(size_t)pos * HL + pi],
                               p.sin_cache[(size_t)pos * HL + pi], x[ks][e], partner, first);
          if (dl < 0) y[ks][e] = 0.0f;
        }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[ks][e] = y[ks][e];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float xs = x[ks][e] * p.scale_log2;
        // one rounded product feeds both halves of the split
        __asm__("" : "+v"(xs));
        const _Float16 hi = (_Float16)xs;
        qB[rb][ks][e] = hi;
        qL[rb][ks][e] = (_Float16)(xs - (float)hi);
      }
  }

  store_stage(slot(t_first), t_first * 64);
  if (PER_BARRIER == 2 && t_first + 1 < t_last) {
    load_stage((t_first + 1) * 64);
    pages.load(pt, t_first + 2, last_page, tid);
    store_stage(slot(t_first + 1), (t_first + 1) * 64);
  }
  __syncthreads();

  // ---- online softmax state ----------------------------------------------------
  // m_run: the row's reference point (set from its first visible keys; 0 only
  // while the row has seen none), l_run: sum of exp2(score - m_run)
  float m_run[RB], l_run[RB];  // lane (row r): row r of block rb
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = 0.0f;
    l_run[rb] = 0.0f;
  }
  v4f acc[RB][JB];  // lane (dim r of block jb, g): rows 4g+e of block rb
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) acc[rb][jb] = v4f{0.f, 0.f, 0.f, 0.f};
  // int8: acc holds sum p * v in units of 2^vexp_run, the largest V-scale
  // exponent of the tiles so far (0 while every tile's V is small; uniform)
  int vexp_run = 0;

  // one tile: QK^T, mask, softmax, PV against the tile in LDS slot T
  auto process = [&](const Tile& T, int tile) __attribute__((always_inline)) {
    const int t0 = tile * 64;
    // int8 large V: a tile whose exponent passes the running one raises it
    // (acc rescaled by an exact power of two); a tile below it has its
    // weights taken 2^(vexp_tile - vexp_run) smaller, and the precise pass's
    // 2^kPrecLift larger: p' = p * 2^dexp (dexp added to every score), so
    // that p' * (s_v / 2^vexp_tile) = p * s_v * 2^(kPrecLift - vexp_run)
    int dexp = 0;
    float svm = 1.0f;  // largest V scale of the tile, / 2^vexp_tile
    if constexpr (!INT4) {
      const int et = PREC ? __builtin_amdgcn_readfirstlane(T.vexp) : 0;  // fast pass: 0
      if (PREC && et > vexp_run) {
        const float f = __builtin_ldexpf(1.0f, vexp_run - et);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int jb = 0; jb < JB; ++jb) acc[rb][jb] *= f;
        vexp_run = et;
      }
      dexp = et - vexp_run + (PREC ? kPrecLift : 0);
      svm = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, T.svmax)));
    }
    const float lc = (float)dexp;

    // S^T for both row blocks: 4 column blocks of 16 tokens; k steps outer so
    // that eight independent accumulation chains interleave on the MFMA pipe.
    // s holds each score relative to its row's reference point:
    // s = <q', k> * s_k - m_run + dexp (masked keys: -inf)
    auto scores = [&](float (&s)[RB][4][4]) __attribute__((always_inline)) {
      v4f c[4][RB];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) c[cb][rb] = v4f{0.f, 0.f, 0.f, 0.f};
      // K fragments of k step ks + 1 are read while the MFMAs of step ks run
      // (the fence keeps the reads ahead of them)
      v8h kf[2][4];
      auto kfrag = [&](int ks, int cb) {
        return *(const v8h*)(T.k + (16 * cb + r) * KROW + 8 * g + 32 * ks);
      };
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) kf[0][cb] = kfrag(0, cb);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) kf[(ks + 1) & 1][cb] = kfrag(ks + 1, cb);
        }
        __builtin_amdgcn_sched_barrier(0);
        // one term at a time over all eight accumulators, so that consecutive
        // MFMAs never wait for each other's result
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            c[cb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[ks & 1][cb], qB[rb][ks], c[cb][rb], 0, 0, 0);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            c[cb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[ks & 1][cb], qL[rb][ks], c[cb][rb], 0, 0, 0);
        if constexpr (INT4) {
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) {
            const v8h al = *(const v8h*)(T.klo + (16 * cb + r) * KROW + 8 * g + 32 * ks);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              c[cb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, qB[rb][ks], c[cb][rb], 0, 0, 0);
          }
        }
      }
      float mref[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) mref[rb] = INT4 ? m_run[rb] : m_run[rb] - lc;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        float skx[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (!INT4) {
          const float4 skv = *(const float4*)(T.sk + 16 * cb + 4 * g);
          skx[0] = skv.x, skx[1] = skv.y, skx[2] = skv.z, skx[3] = skv.w;
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s[rb][cb][e] = INT4 ? c[cb][rb][e] - mref[rb]
                                : __builtin_fmaf(c[cb][rb][e], skx[e], -mref[rb]);
      }
      if (tile >= full_tiles || tile < lo_full) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int t = t0 + 16 * cb + 4 * g + e;
              const bool vis = t <= qpos[rb] && (W <= 0 || t > qpos[rb] - W);
              s[rb][cb][e] = vis ? s[rb][cb][e] : -INFINITY;
            }
      }
    };
    // s -> p = exp2(s) in place; rsum = the row's sum over the tile
    auto weights = [&](float (&s)[RB][4][4], float (&rsum)[RB]) __attribute__((always_inline)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float psum = 0.0f;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[rb][cb][e] = fast_exp2(s[rb][cb][e]);
            psum += s[rb][cb][e];
          }
        rsum[rb] = xgroup_sum(psum);
      }
    };

    // The reference point moves when a row's tile maximum exceeds it by more
    // than kMaxLead (or on the row's first visible keys), so p = exp2(s) stays
    // <= 2^kMaxLead. Any reference point gives the same softmax; it only has
    // to keep p and the sums in range.
    float s[RB][4][4];
    float rsum[RB];
    auto settle = [&]() __attribute__((always_inline)) {
      scores(s);
      float lead[RB];
      bool move = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float mt = -INFINITY;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int e = 0; e < 4; ++e) mt = fmaxf(mt, s[rb][cb][e]);
        mt = xgroup_max(mt) - lc;  // relative to the reference point
        const bool row_moves = mt > kMaxLead || (l_run[rb] == 0.0f && mt != -INFINITY);
        lead[rb] = row_moves ? mt : 0.0f;
        move = move || row_moves;
      }
      if (__builtin_amdgcn_ballot_w64(move) != 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          m_run[rb] += lead[rb];
          // 1 for rows that keep their reference; 0 for rows with no history
          // (their first keys may sit far below 0, where exp2(-lead) is inf
          // and would turn the zero sums into NaN)
          const float alpha = l_run[rb] > 0.0f ? fast_exp2(-lead[rb]) : 0.0f;
          l_run[rb] *= alpha;
#pragma unroll
          for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e) s[rb][cb][e] -= lead[rb];
          // accumulator rows 4g+e: the alpha of row j lives in lane j
          float ae[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) ae[e] = __shfl(alpha, 4 * g + e, 64);
#pragma unroll
          for (int jb = 0; jb < JB; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[rb][jb][e] *= ae[e];
        }
      }
      weights(s, rsum);
    };
    if constexpr (INT4) {
      settle();
    } else {
      // Fast path (int8): the weights against the current reference point are
      // kept when they provably fit: a row sum <= kFastSum / max(s_v) bounds
      // every PV operand p * s_v by kFastSum (binary16), the cap bounds the
      // running sums, and a row that has seen no keys yet needs a sum >= 1
      // (its largest weight is then >= 1/64, so the reference is not far above
      // its scores). Otherwise (a row's first keys, scores that rose far above
      // the reference, inf or NaN) the tile is settled as above, its scores
      // recomputed from the tile still in LDS. (The sums here are 2^dexp of
      // the weights' own.)
      scores(s);
      weights(s, rsum);
      const float cap = __builtin_ldexpf(kFastCap, dexp);
      const float one = __builtin_ldexpf(1.0f, dexp);
      bool bad = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const bool ok = rsum[rb] <= cap && rsum[rb] * svm <= kFastSum &&
                        (l_run[rb] > 0.0f || rsum[rb] >= one);
        bad = bad || !ok;
      }
      if (__builtin_amdgcn_ballot_w64(bad) != 0) settle();
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      l_run[rb] += INT4 ? rsum[rb] : __builtin_ldexpf(rsum[rb], -dexp);

    auto vfrag = [&](int i) {
      const int kst = i / JB, jb = i % JB;
      return *(const v8h*)(T.v + ((size_t)kst * D + 16 * jb + r) * VROW + 8 * g);
    };
    // PV operand: p (x 2^dexp) * s_v (/ 2^vexp_tile) for int8, p * 2^5 for int4
    auto operand = [&](int rb, int cb, int e, const float (&svx)[4]) {
      return s[rb][cb][e] * (INT4 ? kInt4PUp : svx[e]);
    };
    if constexpr (!PREC) {
      v8h pa[RB][2];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          float svx[4] = {1.0f, 1.0f, 1.0f, 1.0f};
          if constexpr (!INT4) {
            const float4 svv = *(const float4*)(T.sv + 16 * cb + 4 * g);
            svx[0] = svv.x, svx[1] = svv.y, svx[2] = svv.z, svx[3] = svv.w;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) pa[rb][cb >> 1][(cb & 1) * 4 + e] = (_Float16)operand(rb, cb, e, svx);
        }
      }
      // PV over the 2 x JB V fragments, kVPrefetch of them in flight ahead of
      // the MFMAs that consume them (the scheduler fence keeps each read ahead
      // of its consumer by that many MFMA pairs, so the LDS latency is covered)
      constexpr int NV = 2 * JB;
      constexpr int PF = INT4 ? kVPrefetchInt4 : kVPrefetch;
      v8h vf[NV];
#pragma unroll
      for (int i = 0; i < PF && i < NV; ++i) vf[i] = vfrag(i);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (i + PF < NV) vf[i + PF] = vfrag(i + PF);
        const int kst = i / JB, jb = i % JB;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rb][kst], vf[i], acc[rb][jb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // int8 with large V (some tile's V scales above kBigVScale): the
      // operand as binary16 hi + lo (~22 significant bits), both against the
      // same V fragment
      v8h ph[RB][2], pl[RB][2];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const float4 svv = *(const float4*)(T.sv + 16 * cb + 4 * g);
        const float svx[4] = {svv.x, svv.y, svv.z, svv.w};
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float w = operand(rb, cb, e, svx);
            // one rounded product feeds both halves of the split
            __asm__("" : "+v"(w));
            const _Float16 hi = (_Float16)w;
            ph[rb][cb >> 1][(cb & 1) * 4 + e] = hi;
            pl[rb][cb >> 1][(cb & 1) * 4 + e] = (_Float16)(w - (float)hi);
          }
      }
#pragma unroll
      for (int i = 0; i < 2 * JB; ++i) {
        const v8h vf = vfrag(i);
        const int kst = i / JB, jb = i % JB;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[rb][kst], vf, acc[rb][jb], 0, 0, 0);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[rb][kst], vf, acc[rb][jb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Tiles in order. PER_BARRIER tiles between barriers; each stages the
  // tile PER_BARRIER ahead into the slot the previous round finished reading
  // (its global loads in flight while the tile is computed, the page ids of
  // the one after). The fast pass (every int4 tile; int8 while every V
  // scale so far is at most kBigVScale) gives up at the first int8 tile with
  // large V: it flags the workgroup and returns before writing anything, and
  // the precise pass (a second launch of this kernel) recomputes the
  // workgroup with the large-V bookkeeping. As a separate kernel the
  // bookkeeping costs the fast pass no registers.
  auto big = [&](const Tile& T) {
    if constexpr (INT4 || PREC) return false;
    else return __builtin_amdgcn_readfirstlane(T.vexp) > 0;
  };
  // the loops end early (their bound drops to the current tile) when the fast
  // pass gives up: one loop exit, as without the check
  int t_stop = t_last;
  if constexpr (NSLOT == 1) {
    // one slot: the next tile's loads are in flight while this one is
    // computed, and it is stored once every wave has finished reading
    for (int tile = t_first; tile < t_stop; ++tile) {
      if (big(sT[0])) {  // every wave sees the same tile
        t_stop = tile;
        break;
      }
      const bool more = tile + 1 < t_last;
      if (more) {
        load_stage((tile + 1) * 64);
        pages.load(pt, tile + 2, last_page, tid);
      }
      process(sT[0], tile);
      __syncthreads();
      if (more) {
        store_stage(sT[0], (tile + 1) * 64);
        __syncthreads();
      }
    }
  } else {
    for (int tile = t_first; tile < t_stop; tile += PER_BARRIER) {
      // the tiles of this round are in LDS (the barrier below orders them)
      bool any_big = big(slot(tile));
      if (PER_BARRIER == 2 && tile + 1 < t_last) any_big = any_big || big(slot(tile + 1));
      if (any_big) {
        t_stop = tile;
        break;
      }
      // not unrolled: one copy of the tile body keeps the register budget
#pragma nounroll
      for (int h = 0; h < PER_BARRIER; ++h) {
        const int tt = tile + h;
        if (tt < t_last) {
          const int nxt = tt + PER_BARRIER;
          const bool more = nxt < t_last;
          if (more) {
            load_stage(nxt * 64);
            pages.load(pt, nxt + 1, last_page, tid);  // consumed by the next stage
          }
          process(slot(tt), tt);
          if (more) store_stage(slot(nxt), nxt * 64);
        }
      }
      __syncthreads();
    }
  }

  if (!PREC && t_stop < t_last) {
    if (tid == 0) *prec_flag = 1;
    return;
  }

  // ---- write O / l ------------------------------------------------------------
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * g + e;  // row within the block
      const float l = __shfl(l_run[rb], row, 64);
      const int R = wave * (16 * RB) + rb * 16 + row;
      const int il = q0 + R / G;
      if (il >= p.sq) continue;
      const int hq = kvh * G + R % G;
      const size_t o = (((size_t)b * p.sq + il) * Hq + hq) * DL;
      if (nks > 1) {
        // the key split's partial in true units: weights p * 2^m_run summing
        // to l * 2^m_run, acc * 2^(vexp_run - kPrecLift) in the precise pass;
        // every stored dim (padding dims hold 0); m = -inf where no key was
        // visible
        const float m = __shfl(m_run[rb], row, 64);
        const float u = __builtin_ldexpf(1.0f, PREC ? vexp_run - kPrecLift : 0);
        float* part = partial_of(il, R % G);
        if (r == 0) {
          part[0] = l > 0.0f ? m : -INFINITY;
          part[1] = l;
        }
#pragma unroll
        for (int jb = 0; jb < JB; ++jb) part[2 + 16 * jb + r] = acc[rb][jb][e] * u;
        continue;
      }
      // acc is in units of 2^(vexp_run - kPrecLift) in the precise pass (exact)
      const float f =
          l > 0.0f ? __builtin_ldexpf(1.0f / l, PREC ? vexp_run - kPrecLift : 0) : 0.0f;
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) {
        const int dl = logical_dim<D>(16 * jb + r);  // -1: padding, not written
        if (dl >= 0) store_out(p.out, o + dl, acc[rb][jb][e] * f, p.out_bf16);
      }
    }
  }
}

// Rows per workgroup (query positions x heads of one kv head) and the grid.
template <int D, int NW>
dim3 prefill_grid(const PrefillParams& p, int group) {
  constexpr int RB = D > 128 ? 1 : 2;  // as in the kernel
  const int qt = 16 * RB * NW / group;
  const int nks = p.nksplit > 1 ? p.nksplit : 1;
  return dim3((p.sq + qt - 1) / qt * nks, p.kv_heads, p.batch);
}

template <int D, int NW, int Q, bool PREC>
hipError_t launch_pass(const PrefillParams& p, int group, hipStream_t st) {
  const dim3 grid = prefill_grid<D, NW>(p, group);
  const dim3 block(64 * NW);
  switch (group) {
    case 1: hipLaunchKernelGGL((gqa_prefill_kernel<D, 1, NW, Q, PREC>), grid, block, 0, st, p); break;
    case 2: hipLaunchKernelGGL((gqa_prefill_kernel<D, 2, NW, Q, PREC>), grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL((gqa_prefill_kernel<D, 4, NW, Q, PREC>), grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL((gqa_prefill_kernel<D, 8, NW, Q, PREC>), grid, block, 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The fast pass, then (int8) the precise pass over the workgroups it flagged.
template <int D, int NW, int Q>
hipError_t launch_dn(const PrefillParams& p, int group, hipStream_t st) {
  hipError_t e = launch_pass<D, NW, Q, false>(p, group, st);
  if (e != hipSuccess || Q != kQuantInt8) return e;
  return launch_pass<D, NW, Q, true>(p, group, st);
}

// 8 waves (256 rows) per workgroup: the staged K/V tile serves twice the rows
// of a 4-wave workgroup at the same LDS footprint (measured 10% faster on the
// 2 x 2048-over-8192 chunk).
template <int D>
hipError_t launch_d(const PrefillParams& p, int group, int quant, hipStream_t st) {
  if (quant == kQuantInt4) return launch_dn<D, 8, kQuantInt4>(p, group, st);
  return launch_dn<D, 8, kQuantInt8>(p, group, st);
}

}  // namespace

size_t prefill_workgroups(const PrefillParams& p, int head_dim, int group) {
  const dim3 g = head_dim > 128 ? prefill_grid<256, 8>(p, group) : prefill_grid<128, 8>(p, group);
  return (size_t)g.x * g.y * g.z;
}

hipError_t launch_gqa_prefill(const PrefillParams& p, int head_dim, int group, int quant,
                              hipStream_t st) {
  if (quant != kQuantInt8 && quant != kQuantInt4) return hipErrorInvalidValue;
  if (head_dim == 64) return launch_d<64>(p, group, quant, st);
  if (head_dim == 128) return launch_d<128>(p, group, quant, st);
  if (head_dim == 256)
    return quant == kQuantInt8 ? launch_dn<256, 8, kQuantInt8>(p, group, st)
                               : launch_dn<256, 8, kQuantInt4>(p, group, st);
  // head_dim 168: the stored width 192, int8 only
  if (head_dim == 168 && quant == kQuantInt8) return launch_dn<192, 8, kQuantInt8>(p, group, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
