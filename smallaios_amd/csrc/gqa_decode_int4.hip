// Kernel 2, int4 cache: split-K flash decode over pages of 4-bit asymmetric
// codes with a binary16 (scale, zero) per (token, kv head, group of 32 dims).
// head_dim 128 (4 groups), 64 (2 groups: lane groups 2 and 3 carry zero query
// dims and zero group parameters, so they add nothing) or 256 (two halves of 128
// dims, each in the 128 layout, their group-scaled dots summed before the
// softmax), GQA group G <= 8 (<= 4 at 256).
//
// Same work split, prologue, double-buffered tile stream and split merge as
// the int8 kernel (gqa_decode.hip); what changes is the math:
//   score(t,h) = sum_G s_tG * <c_t,G , q_h,G> + sum_G z_tG * sum(q_h,G)
//   out(h,d)   = sum_t (p_t * s_tG(d)) * c_td + sum_t p_t * z_tG(d)
//
// Column layout ("block-diagonal"): MFMA column j = 4*hh + G' stands for
// (head hh of a quad of heads, dim group G'). Lane (r, g) of the QK A
// operand holds token r's dims of group g (one 16-byte load); the B operand
// of lane (j, g) is q_hh on those dims if g == G' and zero otherwise, so the
// accumulation over the four 8-dim chunks leaves <c_t,G', q_hh,G'> in column
// j. The lane scales it by its own group's s_tG', adds z_tG' * sum(q_hh,G'),
// and a quad reduction over G' gives the score. All 16 columns are useful for
// G = 4; G = 8 runs two quads.
//
// Codes as f16 subnormals: the mask (w & 0x000F000F) turns two nibbles into
// the exact binary16 values c * 2^-24, and (w & 0x00F000F0) gives c * 2^-20,
// so a dword of 8 nibbles unpacks with one shift and four masks. The factor
// 16 between the two is folded into the other operand (Q x16 on the 2^-24
// dims; p / 16 on the 2^-20 slots, taken in the exponent), and the powers of
// two into the score scale and the merge. v_mfma_f32_16x16x32_f16 multiplies
// subnormal inputs exactly.
//
// QK: Q / max|Q| is split into f16 hi + lo summed along k (22 significant
// bits, so keys with large outlier channels do not amplify the query's
// rounding). PV: A row j = p_t(hh) * s_v,tG' (f16), B = V nibbles; output row
// (hh, G') is read for the dims of group G'. The zero-point term
// sum_t p_t z_v,tG' is accumulated per lane next to the softmax state and
// added at the merge.
#include <type_traits>

#include "append_row.h"
#include "decode_common.h"
#include "sai_internal.h"

namespace sai {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kChunks = 4;  // 8-dim chunks of a lane's 32 dims (one group)
constexpr float kTwo20 = 1048576.0f;          // 2^20
constexpr float kTwo24 = 16777216.0f;         // 2^24

// Halves of 128 dims (two at head_dim 256) and the 32-dim groups of a half.
template <int D>
struct Shape4 {
  static constexpr int NG = D / 32;              // groups of a row
  static constexpr int NH = D > 128 ? D / 128 : 1;
  static constexpr int NGH = NG / NH;            // groups of a half: 2 (D = 64) or 4
  static constexpr int JB = D / 16;              // 16-dim column blocks of PV
};

template <int D>
struct Tile4 {
  static constexpr int NH = Shape4<D>::NH;
  v4u ka[NH][4];     // K: token (page r>>2, slot 4*blk + (r&3)), dims 128 hf + 32g .. +31
  v2u vb[D / 16];    // V: slots 0..15 of dim 16*jb + r in page g
  uint4 kp[NH], vp[NH];  // (scale, zero) of the half's groups, f16, of (page g, slot r)
};

template <int D>
__device__ __forceinline__ void load_tile4(Tile4<D>& T, const uint8_t* __restrict__ pool,
                                           const int* sm_pg, int tile, int num_pages, int kvh,
                                           int r, int g, int n_pages_split) {
  constexpr int NG = D / 32;
  constexpr int NH = Shape4<D>::NH;
  constexpr int NGH = Shape4<D>::NGH;
  constexpr size_t BB = block_bytes_int4(D);
  // at head_dim 64 lane groups 2 and 3 re-read group 1's K bytes: their query
  // dims are zero, and the nibbles are finite, so they add exactly nothing
  const int gk = min(g, NGH - 1);
  const int lp = n_pages_split - 1;
  const int pg_g = sm_pg[min(tile * 4 + g, lp)];
  const int pg_k = sm_pg[min(tile * 4 + (r >> 2), lp)];
  const uint8_t* blk_g = pool + block_offset(pg_g, kvh, num_pages, BB);
  const uint8_t* blk_k = pool + block_offset(pg_k, kvh, num_pages, BB);
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
      T.ka[hf][blk] = __builtin_nontemporal_load(
          (const v4u*)(blk_k + (size_t)(4 * blk + (r & 3)) * (D / 2) + 64 * hf + 16 * gk));
#pragma unroll
  for (int jb = 0; jb < D / 16; ++jb)
    T.vb[jb] = __builtin_nontemporal_load((const v2u*)(blk_g + 8 * D + (16 * jb + r) * 8));
  if constexpr (NGH == 4) {
    // half hf: groups 4 hf .. 4 hf + 3, 16 bytes of the slot's 4 NG
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      T.kp[hf] = *(const uint4*)(blk_g + 16 * D + 4 * NG * r + 16 * hf);
      T.vp[hf] = *(const uint4*)(blk_g + 16 * D + 64 * NG + 4 * NG * r + 16 * hf);
    }
  } else {
    // two groups: 8 bytes per slot, the upper (scale, zero) pairs zero
    const uint2 k2 = *(const uint2*)(blk_g + 16 * D + 8 * r);
    const uint2 v2 = *(const uint2*)(blk_g + 16 * D + 64 * NG + 8 * r);
    T.kp[0] = uint4{k2.x, k2.y, 0u, 0u};
    T.vp[0] = uint4{v2.x, v2.y, 0u, 0u};
  }
}

// 8 nibbles (one dword, element k at bits 4k..4k+3) -> f16 subnormals in the
// order k = 0,4,1,5,2,6,3,7 with scales 2^-24, 2^-24, 2^-20, 2^-20, 2^-24,
// 2^-24, 2^-20, 2^-20.
__device__ __forceinline__ v8h unpack_sub(uint32_t w) {
  const uint32_t t = w >> 8;
  const v4u u = v4u{w & 0x000F000Fu, w & 0x00F000F0u, t & 0x000F000Fu, t & 0x00F000F0u};
  return __builtin_bit_cast(v8h, u);
}
// element of the chunk at k position i of that order, and whether its scale
// is 2^-24 (true) or 2^-20
__device__ __forceinline__ constexpr int sub_elem(int i) { return (i >> 1) + ((i & 1) ? 4 : 0); }
__device__ __forceinline__ constexpr bool sub_small(int i) { return ((i >> 1) & 1) == 0; }

// float add of the lane xor 1 / xor 2 neighbour inside a quad
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
  return v;
}

template <int D, int G>
struct State4 {
  static constexpr int HT = (G + 3) / 4;  // quads of heads
  float m_run[HT], l_run[HT];  // per lane (j, g): head 4*qd + j/4, log2 domain
  float zacc[Shape4<D>::NH][HT];  // sum_t p_t z_v,tG' of (head 4*qd + j/4, G' = j&3) per half
  float acc[HT][D / 16];       // lane (dim 16*jb + r, g): head 4*qd + g, x 2^-24
};

// One 64-token tile: lane (r, g) owns page g of the tile (slots 0..15) for
// column j = r. MASK: the tile crosses the end of the split (t_end) or the
// first key of a sliding window (t_lo).
template <int D, int G, bool MASK>
__device__ __forceinline__ void compute_tile4(const Tile4<D>& T, State4<D, G>& st,
                                              const v8h (&Bh)[Shape4<D>::NH][State4<D, G>::HT][kChunks],
                                              const v8h (&Bl)[Shape4<D>::NH][State4<D, G>::HT][kChunks],
                                              const float (&qsn)[Shape4<D>::NH][State4<D, G>::HT],
                                              const float (&q_scale)[State4<D, G>::HT], int tok0,
                                              int t_lo, int t_end, int r, int g, uint4* sm_p) {
  constexpr int HT = State4<D, G>::HT;
  constexpr int NH = Shape4<D>::NH;
  constexpr int JB = D / 16;
  constexpr int JBH = JB / NH;  // column blocks of a half
  const int lane = threadIdx.x & 63;
  const int gp = r & 3;
  // (scale, zero) of every slot of the tile through this wave's LDS slot:
  // K halves, then V halves, 64 lanes each
#pragma unroll
  for (int hf = 0; hf < NH; ++hf) {
    sm_p[64 * hf + lane] = T.kp[hf];
    sm_p[64 * (NH + hf) + lane] = T.vp[hf];
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t* sm_w = (const uint32_t*)sm_p;

  // QK^T: per half and 16-token block, accumulate the four 8-dim chunks (hi
  // and lo)
  v4f cs[NH][HT][4];
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      v8h ka[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) ka[c] = unpack_sub(T.ka[hf][blk][c]);
#pragma unroll
      for (int qd = 0; qd < HT; ++qd) {
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[c], Bh[hf][qd][c], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[c], Bl[hf][qd][c], acc, 0, 0, 0);
        }
        cs[hf][qd][blk] = acc;
      }
    }
  // MASK: slots [nlow, nvalid) of page g are visible (split end, window start)
  const int nvalid = t_end - tok0;
  const int nlow = t_lo - tok0;
  // u = sum_G' (s_G' * dot_G' + z_G' * qsn) over the groups of every half;
  // score (log2) = q_scale * u
  float u[HT][16];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int slot = 4 * blk + e;
#pragma unroll
      for (int qd = 0; qd < HT; ++qd) {
        float t = 0.0f;
#pragma unroll
        for (int hf = 0; hf < NH; ++hf) {
          const v2h sz = __builtin_bit_cast(v2h, sm_w[(64 * hf + 16 * g + slot) * 4 + gp]);
          const float th = fmaf((float)sz[0], cs[hf][qd][blk][e], (float)sz[1] * qsn[hf][qd]);
          t = hf == 0 ? th : t + th;
        }
        u[qd][slot] = quad_sum(t);
      }
    }
  if (MASK) {
#pragma unroll
    for (int qd = 0; qd < HT; ++qd)
#pragma unroll
      for (int i = 0; i < 16; ++i) u[qd][i] = (i < nvalid && i >= nlow) ? u[qd][i] : -INFINITY;
  }
  // p of even slots; odd slots hold p / 16 (their V codes carry 2^-20)
  float p[HT][16];
  float alpha[HT];
#pragma unroll
  for (int qd = 0; qd < HT; ++qd) {
    float mt = u[qd][0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mt = fmaxf(mt, u[qd][i]);
    mt = xgroup_max(mt) * q_scale[qd];
    const float m_new = fmaxf(st.m_run[qd], mt);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    alpha[qd] = fast_exp2(st.m_run[qd] - m_use);
    float se = 0.0f, so = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[qd][i] = fast_exp2(fmaf(u[qd][i], q_scale[qd], (i & 1) ? -m_use - 4.0f : -m_use));
      if (i & 1)
        so += p[qd][i];
      else
        se += p[qd][i];
    }
    const float psum = xgroup_sum(fmaf(so, 16.0f, se));
    st.l_run[qd] = st.l_run[qd] * alpha[qd] + psum;
    st.m_run[qd] = m_new;
  }

  // A operand of P V, per half of the dims: row j = p(head) * s_v of group
  // G' = j&3 of the half, slots of each half-page in the V unpack order;
  // zero-point sums of the same (head, G')
  v8h pa[NH][HT][2];
  float ze[NH][HT], zo[NH][HT];
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int qd = 0; qd < HT; ++qd) ze[hf][qd] = zo[hf][qd] = 0.0f;
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int slot = 8 * half + sub_elem(i);
        const v2h sz =
            __builtin_bit_cast(v2h, sm_w[(64 * (NH + hf) + 16 * g + slot) * 4 + gp]);
#pragma unroll
        for (int qd = 0; qd < HT; ++qd) {
          float a = p[qd][slot] * (float)sz[0];
          float z = p[qd][slot] * (float)sz[1];
          if (MASK) {
            // masked slots may hold stale parameters: select, do not multiply
            a = (slot < nvalid && slot >= nlow) ? a : 0.0f;
            z = (slot < nvalid && slot >= nlow) ? z : 0.0f;
          }
          pa[hf][qd][half][i] = (_Float16)a;
          if (slot & 1)
            zo[hf][qd] += z;
          else
            ze[hf][qd] += z;
        }
      }
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int qd = 0; qd < HT; ++qd)
      st.zacc[hf][qd] =
          st.zacc[hf][qd] * alpha[qd] + xgroup_sum(fmaf(zo[hf][qd], 16.0f, ze[hf][qd]));

  // rescale factor of the head this lane accumulates in P V (4*qd + g)
  float apv[HT];
#pragma unroll
  for (int qd = 0; qd < HT; ++qd) {
    const int a0 = __builtin_amdgcn_readlane(__float_as_int(alpha[qd]), 0);
    const int a1 = __builtin_amdgcn_readlane(__float_as_int(alpha[qd]), 4);
    const int a2 = __builtin_amdgcn_readlane(__float_as_int(alpha[qd]), 8);
    const int a3 = __builtin_amdgcn_readlane(__float_as_int(alpha[qd]), 12);
    apv[qd] = __int_as_float(g == 0 ? a0 : (g == 1 ? a1 : (g == 2 ? a2 : a3)));
  }
  // P V on the matrix cores; lane (dim, g) reads row (head g, group of dim)
  // from the A operand of the dim's half
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
    const int hf = jb / JBH;
    const v8h b0 = unpack_sub(T.vb[jb].x);
    const v8h b1 = unpack_sub(T.vb[jb].y);
#pragma unroll
    for (int qd = 0; qd < HT; ++qd) {
      v4f co = v4f{0.f, 0.f, 0.f, 0.f};
      co = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[hf][qd][0], b0, co, 0, 0, 0);
      co = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[hf][qd][1], b1, co, 0, 0, 0);
      st.acc[qd][jb] = st.acc[qd][jb] * apv[qd] + co[(jb % JBH) >> 1];
    }
  }
}

// head_dim 256 (two halves of tiles, query terms and dots) and group 8 at 128 (two
// quads of heads: twice the query terms, dots and accumulators) run one wave
// per SIMD with the whole register file; at two waves per SIMD group 8 spilled
// ~400 bytes per lane
template <int D, int G>
constexpr bool kOneWavePerSimd = D > 128 || (G > 4 && D == 128);

template <int D, int G, int NW>
__global__ __launch_bounds__(64 * NW, (kOneWavePerSimd<D, G>) ? 1 : 8 / NW) void gqa_decode_int4_kernel(
    DecodeParams p) {
  constexpr int HT = State4<D, G>::HT;
  constexpr int NG = D / 32;
  constexpr int NH = Shape4<D>::NH;
  constexpr int NGH = Shape4<D>::NGH;
  constexpr int JB = D / 16;
  constexpr size_t BB = block_bytes_int4(D);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int work = blockIdx.x;

  int b, split, nsplit, split_base, tps;
  decode_work_item(p, work, lane, b, split, nsplit, split_base, tps);
  if (b < 0 || b >= p.batch) return;  // uniform over the workgroup

  // length first; then the page ids of the split; then the query and the
  // cos / sin of position L-1, all in flight across the barrier and ahead
  // of the first tile
  // (without a window the page-id loads go out beside the length's)
  // sliding window: keys [k_lo, L) visible, splits from the tile holding k_lo
  __shared__ int sm_pg[kMaxSplitPages];
  int L, k_lo, first_page;
  stage_split_pages<64 * NW>(p, b, split, tps, sm_pg, L, k_lo, first_page);
  const int origin = (k_lo / 64) * 64;

  // lane (j = 4*hh + G', g) holds the 32 dims of group g of head 4*qd + hh
  const int gp = r & 3;
  const int hh = r >> 2;
  const int Hq = p.kv_heads * G;
  // lane (r, g) holds dims 128 hf + 32g .. +31 of head 4*qd + hh
  float x[NH][HT][32];
#pragma unroll
  for (int hf = 0; hf < NH; ++hf)
#pragma unroll
    for (int qd = 0; qd < HT; ++qd) {
      const int h = 4 * qd + hh;
      if (h < G && g < NGH) {
        const size_t qbase = ((size_t)b * Hq + kvh * G + h) * D + 128 * hf + 32 * g;
        float t[16];
        load16(p.q, qbase, p.q_dtype, t);
#pragma unroll
        for (int i = 0; i < 16; ++i) x[hf][qd][i] = t[i];
        load16(p.q, qbase + 16, p.q_dtype, t);
#pragma unroll
        for (int i = 0; i < 16; ++i) x[hf][qd][16 + i] = t[i];
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) x[hf][qd][i] = 0.0f;
      }
    }
  // cos / sin of the lane's dims of each half, as two runs of 16
  float4 cq4[NH][2][4], sq4[NH][2][4];
  if (p.do_rotary) {
    const float* cr = p.cos_cache + (size_t)(L - 1) * (D / 2);
    const float* sr = p.sin_cache + (size_t)(L - 1) * (D / 2);
#pragma unroll
    for (int hf = 0; hf < NH; ++hf)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        rope_load16<D>(cr, sr, 128 * hf + 32 * min(g, NGH - 1) + 16 * h2, p.interleaved,
                       cq4[hf][h2], sq4[hf][h2]);
  }

  const int t_begin = origin + split * tps * 64;
  const int t_end = min(L, t_begin + tps * 64);
  const int n_pages_split = (t_end - 1) / kPageTokens - first_page + 1;
  const int n_tiles = (t_end - t_begin + 63) / 64;
  const int last_owner = (n_tiles - 1) % NW;
  __syncthreads();

  // fused append by the wave that streams the split's last tile (the page of
  // the new token): before its first load if that tile is its only one, else
  // while its first tile is in flight
  const bool appender = p.k_new != nullptr && split == nsplit - 1 && wave == last_owner;
  int tile = wave;
  const int my_tiles = tile < n_tiles ? (n_tiles - 1 - tile) / NW + 1 : 0;
  auto append = [&]() {
    const int pos = L - 1;
    uint8_t* blk = (uint8_t*)p.pool +
                   block_offset(sm_pg[pos / kPageTokens - first_page], kvh, p.num_pages, BB);
    const size_t row = ((size_t)b * p.kv_heads + kvh) * D * (p.kv_dtype == kDtypeBf16 ? 2 : 4);
    append_row_int4<D>((const uint8_t*)p.k_new + row, (const uint8_t*)p.v_new + row,
                         p.kv_dtype, lane, pos, blk, pos % kPageTokens, p.do_rotary,
                         p.interleaved != 0, p.cos_cache, p.sin_cache);
    // the page is read back by this wave's last tile
    __threadfence_block();
  };
  if (appender && my_tiles == 1) append();
  Tile4<D> TA;
  if (tile < n_tiles) load_tile4(TA, p.pool, sm_pg, tile, p.num_pages, kvh, r, g, n_pages_split);
  if (appender && my_tiles > 1) append();

  // ---- Q: RoPE at position L-1, normalised by the head's max|Q| ----
  v8h Bh[NH][HT][kChunks], Bl[NH][HT][kChunks];
  float qsn[NH][HT], q_scale[HT];
#pragma unroll
  for (int qd = 0; qd < HT; ++qd) {
    if (p.do_rotary) {
      float y[NH][32], cq[NH][32], sq[NH][32];
#pragma unroll
      for (int hf = 0; hf < NH; ++hf)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          float c16[16], s16[16];
          rope_pick_all<0>(cq4[hf][h2], sq4[hf][h2], p.interleaved != 0, c16, s16);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            cq[hf][16 * h2 + i] = c16[i];
            sq[hf][16 * h2 + i] = s16[i];
          }
        }
      if (p.interleaved) {
#pragma unroll
        for (int hf = 0; hf < NH; ++hf)
#pragma unroll
          for (int i = 0; i < 32; ++i)
            y[hf][i] = rope_elem(cq[hf][i], sq[hf][i], x[hf][qd][i], x[hf][qd][i ^ 1], (i & 1) == 0);
      } else if constexpr (NH == 2) {
        // partner d +- 128: the other half, same lane and element
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int i = 0; i < 32; ++i)
            y[hf][i] = rope_elem(cq[hf][i], sq[hf][i], x[hf][qd][i], x[hf ^ 1][qd][i], hf == 0);
      } else {
        // partner d +- D/2: group g ^ (NGH/2), the lane 16 * NGH / 2 away
        const bool first = g < NGH / 2;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          float xp;
          if constexpr (NGH == 4) {
            // permlane32_swap(x, x): [0] = lanes 0-31's x on both halves, [1] =
            // lanes 32-63's x on both halves
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[0][qd][i]),
                                                       __float_as_uint(x[0][qd][i]), false, false);
            xp = __uint_as_float(first ? sw[1] : sw[0]);
          } else {
            xp = __shfl_xor(x[0][qd][i], 16, 64);
          }
          y[0][i] = rope_elem(cq[0][i], sq[0][i], x[0][qd][i], xp, first);
        }
      }
#pragma unroll
      for (int hf = 0; hf < NH; ++hf)
#pragma unroll
        for (int i = 0; i < 32; ++i) x[hf][qd][i] = y[hf][i];
    }
    float amax = 0.0f, sum[NH];
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      sum[hf] = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        amax = fmaxf(amax, fabsf(x[hf][qd][i]));
        sum[hf] += x[hf][qd][i];
      }
    }
    amax = xgroup_max(amax);
    const float norm = amax > 0.0f ? amax : 1.0f;
    const float inv = 1.0f / norm;
    // dots come out x 2^-20 (see the unpack), folded into the score scale
    q_scale[qd] = norm * p.scale_log2 * kTwo20;
    const v8h zero = v8h{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      // sum over group G' = j&3 of the half for this head: held by lane (j, G')
      const float gsum = __shfl(sum[hf], r + 16 * gp, 64);
      qsn[hf][qd] = gsum * inv * (1.0f / kTwo20);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v8h qh, ql;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float yv = x[hf][qd][8 * c + sub_elem(i)] * inv * (sub_small(i) ? 16.0f : 1.0f);
          // hi and lo must split one f32 value; without this barrier the
          // backend may fold the product into one of the two f16 conversions
          // only (v_fma_mixlo_f16, a single rounding) and hi + lo drifts
          __asm__("" : "+v"(yv));
          const _Float16 hi = (_Float16)yv;
          qh[i] = hi;
          ql[i] = (_Float16)(yv - (float)hi);
        }
        Bh[hf][qd][c] = g == gp ? qh : zero;
        Bl[hf][qd][c] = g == gp ? ql : zero;
      }
    }
  }
  __shared__ uint4 sm_par[NW][128 * NH];

  // ---- stream the split's tiles, ping-pong; the last one may be partial ----
  State4<D, G> st;
#pragma unroll
  for (int qd = 0; qd < HT; ++qd) {
    st.m_run[qd] = -INFINITY;
    st.l_run[qd] = 0.0f;
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) st.zacc[hf][qd] = 0.0f;
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) st.acc[qd][jb] = 0.0f;
  }

  Tile4<D> TB;
  auto tok0 = [&](int k) { return t_begin + (wave + k * NW) * 64 + 16 * g; };
  // With one wave per SIMD the next tile's loads are kept ahead of the
  // current tile's work (the scheduler would otherwise sink them a third of
  // the way into it): 43.5 -> 39.6 us per step at the Gemma-3-4B int4 shape.
  // With two waves per SIMD the other wave covers the latency, and the
  // pinned order measured 3 % slower at 4 x 32k.
  auto ld = [&](Tile4<D>& T, int k) {
    load_tile4(T, p.pool, sm_pg, wave + k * NW, p.num_pages, kvh, r, g, n_pages_split);
    if constexpr (kOneWavePerSimd<D, G>) __builtin_amdgcn_sched_barrier(0);
  };
  // tiles before the split's last one are full
  const bool last_partial = (t_end - t_begin) % 64 != 0;
  auto run = [&](const Tile4<D>& T, int k) {
    const bool partial = last_partial && wave + k * NW == n_tiles - 1;
    if (__builtin_amdgcn_readfirstlane(partial))
      compute_tile4<D, G, true>(T, st, Bh, Bl, qsn, q_scale, tok0(k), k_lo, t_end, r, g, sm_par[wave]);
    else
      compute_tile4<D, G, false>(T, st, Bh, Bl, qsn, q_scale, tok0(k), k_lo, t_end, r, g, sm_par[wave]);
  };
  int k = 0;
  // the window's first key inside the split's first tile (wave 0's tile 0):
  // that tile runs the masked path, and its successor moves into TA so the
  // ping-pong below starts at k = 1
  if (wave == 0 && k_lo > t_begin) {  // uniform over the wave
    if (my_tiles > 1) {
      ld(TB, 1);
      compute_tile4<D, G, true>(TA, st, Bh, Bl, qsn, q_scale, tok0(0), k_lo, t_end, r, g, sm_par[wave]);
      TA = TB;
      k = 1;
    } else {
      compute_tile4<D, G, true>(TA, st, Bh, Bl, qsn, q_scale, tok0(0), k_lo, t_end, r, g, sm_par[wave]);
      k = 1;
    }
  }
  for (; k + 2 < my_tiles; k += 2) {
    ld(TB, k + 1);
    compute_tile4<D, G, false>(TA, st, Bh, Bl, qsn, q_scale, tok0(k), k_lo, t_end, r, g, sm_par[wave]);
    ld(TA, k + 2);
    compute_tile4<D, G, false>(TB, st, Bh, Bl, qsn, q_scale, tok0(k + 1), k_lo, t_end, r, g, sm_par[wave]);
  }
  if (k + 1 < my_tiles) {
    ld(TB, k + 1);
    compute_tile4<D, G, false>(TA, st, Bh, Bl, qsn, q_scale, tok0(k), k_lo, t_end, r, g, sm_par[wave]);
    run(TB, k + 1);
  } else if (k < my_tiles) {
    run(TA, k);
  }

  // ---- merge the NW waves; zero-point sums join per (head, dim group) ----
  __shared__ float sm_m[NW][G];
  __shared__ float sm_l[NW][G];
  __shared__ float sm_z[NW][G][NG];
  __shared__ float sm_o[NW][G][D];
#pragma unroll
  for (int qd = 0; qd < HT; ++qd) {
    const int h = 4 * qd + hh;
    if (g == 0 && h < G) {
#pragma unroll
      for (int hf = 0; hf < NH; ++hf)
        if (gp < NGH) sm_z[wave][h][NGH * hf + gp] = st.zacc[hf][qd];
      if (gp == 0) {
        sm_m[wave][h] = st.m_run[qd];
        sm_l[wave][h] = st.l_run[qd];
      }
    }
    const int hd = 4 * qd + g;
    if (hd < G) {
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) sm_o[wave][hd][16 * jb + r] = st.acc[qd][jb] * kTwo24;
    }
  }
  __syncthreads();

  float* part = p.partials + ((size_t)(split_base + split) * p.kv_heads + kvh) * (G * (D + 2));
  for (int t = threadIdx.x; t < G * D; t += 64 * NW) {
    const int hd = t / D, d = t % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w][hd]);
    float Ls = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (sm_m[w][hd] == -INFINITY) continue;
      const float f = fast_exp2(sm_m[w][hd] - M);
      Ls += sm_l[w][hd] * f;
      O += (sm_o[w][hd][d] + sm_z[w][hd][d >> 5]) * f;
    }
    if (nsplit == 1) {
      store_out(p.out, ((size_t)b * Hq + kvh * G + hd) * D + d, Ls > 0.0f ? O / Ls : 0.0f, p.out_bf16);
    } else if (p.merge_in_kernel) {
      store_partial(part + hd * (D + 2) + 2 + d, O);
      if (d == 0) {
        store_partial(part + hd * (D + 2), M);
        store_partial(part + hd * (D + 2) + 1, Ls);
      }
    } else {
      part[hd * (D + 2) + 2 + d] = O;
      if (d == 0) {
        part[hd * (D + 2)] = M;
        part[hd * (D + 2) + 1] = Ls;
      }
    }
  }
  if (!p.merge_in_kernel) {
    // every sequence records its split range, single-split ones included, so
    // the combine kernel never reads a previous launch's entry
    if (split == 0 && threadIdx.x == 0 && kvh == 0) {
      p.seq_info[2 * b] = split_base;
      p.seq_info[2 * b + 1] = nsplit;
    }
    return;
  }
  if (nsplit == 1) return;

  // ---- in-kernel merge, as in the int8 kernel: the partial stores are
  // agent-scope and complete (each wave waits for its own, then the barrier)
  // before thread 0 takes a ticket of (b, kvh); the workgroup with the last
  // ticket loads every split's partial in split order and writes the output
  __shared__ int sm_last;
  partials_complete();
  __syncthreads();
  int* counter = &p.counters[b * p.kv_heads + kvh];
  if (threadIdx.x == 0) sm_last = last_ticket(counter, nsplit);
  __syncthreads();
  if (!sm_last) return;
  const size_t stride = (size_t)p.kv_heads * (G * (D + 2));
  const float* p0 = p.partials + ((size_t)split_base * p.kv_heads + kvh) * (G * (D + 2));
  for (int t = threadIdx.x; t < G * D; t += 64 * NW) {
    const int hd = t / D, d = t % D;
    float M = -INFINITY, Ls = 0.0f, O = 0.0f;
    const float* ph = p0 + hd * (D + 2);
    merge_all_splits(ph, stride, d, nsplit, M, Ls, O);
    store_out(p.out, ((size_t)b * Hq + kvh * G + hd) * D + d, Ls > 0.0f ? O / Ls : 0.0f, p.out_bf16);
  }
  if (threadIdx.x == 0) reset_ticket(counter);
}

template <int D, int G>
hipError_t launch_g(const DecodeParams& p, int work_items, bool combine, hipStream_t st) {
  // head_dim 256 and group 8: four waves (one per SIMD)
  bool eight = false;
  if constexpr (!kOneWavePerSimd<D, G>) {
    eight = p.waves == 8;
    if (eight)
      hipLaunchKernelGGL((gqa_decode_int4_kernel<D, G, 8>), dim3(work_items, p.kv_heads),
                         dim3(512), 0, st, p);
  }
  if (!eight)
    hipLaunchKernelGGL((gqa_decode_int4_kernel<D, G, 4>), dim3(work_items, p.kv_heads), dim3(256),
                       0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !combine || p.merge_in_kernel) return e;
  return launch_decode_combine(p, D, G, st);
}

template <int D>
hipError_t launch_d(const DecodeParams& p, int group, int work_items, bool combine,
                    hipStream_t st) {
  switch (group) {
    case 1: return launch_g<D, 1>(p, work_items, combine, st);
    case 2: return launch_g<D, 2>(p, work_items, combine, st);
    case 4: return launch_g<D, 4>(p, work_items, combine, st);
    case 8:
      if constexpr (D <= 128) return launch_g<D, 8>(p, work_items, combine, st);
      return hipErrorInvalidValue;  // head_dim 256: groups up to 4
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gqa_decode_int4(const DecodeParams& p, int head_dim, int group, int work_items,
                                  bool combine, hipStream_t st) {
  if (p.split_tokens <= 0 || p.split_tokens % 64 != 0 ||
      p.split_tokens > kMaxSplitPages * kPageTokens)
    return hipErrorInvalidValue;
  if (head_dim == 128) return launch_d<128>(p, group, work_items, combine, st);
  if (head_dim == 64) return launch_d<64>(p, group, work_items, combine, st);
  if (head_dim == 256 && group <= 4) return launch_d<256>(p, group, work_items, combine, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
