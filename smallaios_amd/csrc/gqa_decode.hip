// Kernel 2: split-K flash decode over the paged int8 cache (one query token
// per sequence, GQA group of G query heads per kv head).
//
// Why int8 MFMA. At the Llama-3-8B layer shape (G = 4, D = 128) a decode step
// reads 264 B per (token, kv head) and does 4 * 128 * 2 multiply-adds on them.
// Dequantising every code to f32 and doing those multiply-adds on the VALU
// costs more vector cycles than the HBM stream leaves (~90 SIMD cycles per
// token-head at 80 % of 8 TB/s). Instead the int8 codes go straight from HBM
// into v_mfma_i32_16x16x64_i8 operands and the per-token scales are applied to
// the 32-bit dot products:
//   score(t, h) = s_k[t] * (sq_hi[h] * <k_t, qhi_h> + sq_lo[h] * <k_t, qlo_h>)
//   out(h, :)   = sum_t p'(t, h) * v_t,   p' = p * s_v[t] = sp[h]*(phi + plo/254)
// Q (after RoPE) and P' are split into two int8 terms (hi + residual/254), so
// their representation error is ~1/64516 of the row maximum; both terms ride
// in spare MFMA rows/columns, so the split costs no extra MFMA issue.
//
// Wave layout (lane = r + 16 g, r = lane & 15, g = lane >> 4). A tile is 64
// tokens = 4 pages; lane group g of a tile works on page g.
//   QK  : S^T = K * Q^T.  A = K codes, row i of MFMA #blk is token
//         (page i>>2, slot 4*blk + (i&3)); B = Q terms, column j = head-term
//         (head j>>1, term j&1: 0 = hi, 1 = lo). The result lands with lane
//         (j, g) holding head-term j for all 16 slots of page g -- exactly the
//         A-operand layout the PV product needs, so no LDS transpose.
//         k index: lane group g, k step ks <-> dims kdim0(g, ks) + [0,16):
//         (D/4)*g + 16*ks up to head_dim 128, so one row's 4 lane groups read
//         one contiguous 128-byte line; 16*g + 64*ks at 256, so they read 64
//         contiguous bytes of the row's two lines per load instruction.
//   PV  : O = P' * V.  A = P' codes (row = head-term, k = slots of page g),
//         B = V codes read dim-major from the page (column = dim).
//   Online softmax in the log2 domain; cross-page reductions are two
//   permlane swaps (VALU), the hi/lo pairing one DPP quad swap.
//
// Memory pipeline: the split's page ids are staged in LDS once, and every
// wave double-buffers its tiles in registers (the loads of tile i+NW are in
// flight while tile i is computed).
//
// Work split: grid.x enumerates (sequence, split) pairs over ragged lengths
// (each wave finds its pair by a prefix scan over seq_lens), grid.y is the kv
// head. NW waves of a workgroup take interleaved tiles of the split and merge
// through LDS. A sequence with one split writes its output directly; with
// several, every workgroup writes a partial (m, l, o) and the combine kernel
// (a second launch, so no cross-workgroup fences) merges them.
#include <type_traits>

#include "append_row.h"
#include "decode_common.h"
#include "sai_internal.h"

namespace sai {

namespace {

template <int D>
struct TileRegs {
  static constexpr int KS = D / 64;
  static constexpr int JB = D / 16;
  v4i ka[4][KS];  // K codes, QK A operand per 16-row block
  v4i vb[JB];     // V codes (dim-major), PV B operand per 16-dim block
  float sk, sv;   // K / V scale of (page g, slot r); shared through LDS
};

// Parts of a tile load: K codes and both scales (part 1), V codes (part 2).
// First head dim of lane group g's 16-dim chunk at k step ks (K codes and Q
// terms alike). At head_dim 256, (D/4)*g + 16*ks would spread a load
// instruction's four 16-byte pieces of a row over both of its lines (32
// lines per instruction, 32 bytes used of each); 16*g + 64*ks reads 64
// contiguous bytes (16 lines) and took the gemma-shaped decode from 68.2 to
// 52.3 us. At 128 the same change measured slower (50.2 -> 52.7 us: the
// partner chunk held for RoPE spills registers).
template <int D>
__device__ __forceinline__ constexpr int kdim0(int g, int ks) {
  return D > 128 ? 16 * g + 64 * ks : (D / 4) * g + 16 * ks;
}

template <int D, int PART = 3>
__device__ __forceinline__ void load_tile(TileRegs<D>& T, const uint8_t* __restrict__ pool,
                                          const int* sm_pg, int tile, int num_pages, int kvh,
                                          int r, int g, int n_pages_split) {
  constexpr size_t BB = block_bytes_int8(D);
  const int lp = n_pages_split - 1;
  const int pg_g = sm_pg[min(tile * 4 + g, lp)];
  const int pg_k = sm_pg[min(tile * 4 + (r >> 2), lp)];
  const uint8_t* blk_g = pool + block_offset(pg_g, kvh, num_pages, BB);
  const uint8_t* blk_k = pool + block_offset(pg_k, kvh, num_pages, BB);
  if constexpr ((PART & 1) != 0) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int ks = 0; ks < TileRegs<D>::KS; ++ks)
        T.ka[blk][ks] = __builtin_nontemporal_load(
            (const v4i*)(blk_k + (size_t)(4 * blk + (r & 3)) * D + kdim0<D>(g, ks)));
  }
  if constexpr ((PART & 2) != 0) {
#pragma unroll
    for (int jb = 0; jb < TileRegs<D>::JB; ++jb)
      T.vb[jb] = __builtin_nontemporal_load((const v4i*)(blk_g + 16 * D + (16 * jb + r) * 16));
  }
  if constexpr ((PART & 1) != 0) {
    T.sk = ((const float*)(blk_g + 32 * D))[r];
    T.sv = ((const float*)(blk_g + 32 * D + 64))[r];
  }
}

template <int D, int G>
struct WaveState {
  float m_run, l_run;   // per head (lanes of head-term j), log2 domain
  float acc[D / 16][2]; // lane (dim 16*jb + r, group g): heads 2g, 2g+1
};

struct NoHook {
  __device__ void operator()() const {}
};

// after_qk runs once the tile's K codes and scales are consumed (the QK
// MFMAs issued, the scales in LDS), after_pv once its V codes are: a caller
// with one tile buffer loads the next tile's K and V there.
template <int D, int G, class H1 = NoHook, class H2 = NoHook>
__device__ __forceinline__ void compute_tile(const TileRegs<D>& T, WaveState<D, G>& st,
                                             const v4i (&qB)[D / 64], float q_own, float q_oth,
                                             int tok0, int t_lo, int t_end, bool is_hi, bool live,
                                             int g, float* sm_sc, H1 after_qk = H1{},
                                             H2 after_pv = H2{}) {
  constexpr int KS = D / 64;
  constexpr int JB = D / 16;
  // QK^T on the matrix cores
  v4i cs[4];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    cs[blk] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      cs[blk] = __builtin_amdgcn_mfma_i32_16x16x64_i8(T.ka[blk][ks], qB[ks], cs[blk], 0, 0, 0);
  }
  // scales of page g, slots 0..15 (this wave's LDS slot; lane 16g + r wrote slot r)
  const int lane = threadIdx.x & 63;
  sm_sc[lane] = T.sk;
  sm_sc[64 + lane] = T.sv;
  after_qk();
  __builtin_amdgcn_wave_barrier();  // LDS ops of a wave run in order; keep the compiler from hoisting
  float skv[16], svv[16];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 a = *(const float4*)(sm_sc + 16 * g + 4 * w);
    const float4 c = *(const float4*)(sm_sc + 64 + 16 * g + 4 * w);
    skv[4 * w] = a.x, skv[4 * w + 1] = a.y, skv[4 * w + 2] = a.z, skv[4 * w + 3] = a.w;
    svv[4 * w] = c.x, svv[4 * w + 1] = c.y, svv[4 * w + 2] = c.z, svv[4 * w + 3] = c.w;
  }
  // slots [nlow, nvalid) of page g are visible: inside the split and at or
  // after the first key of the window
  const int nvalid = t_end - tok0;
  const int nlow = t_lo - tok0;
  const bool full =
      __builtin_amdgcn_readfirstlane(t_end - (tok0 - 16 * g) >= 64 && tok0 - 16 * g >= t_lo);
  float s[16];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int slot = 4 * blk + e;
      const int own = cs[blk][e];
      const int oth = swap_pair(own);
      s[slot] = (q_own * (float)own + q_oth * (float)oth) * skv[slot];
    }
  if (!full) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bool vis = i < nvalid && i >= nlow;
      s[i] = vis ? s[i] : -INFINITY;
      svv[i] = vis ? svv[i] : 0.0f;
    }
  }
  float mt = s[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mt = fmaxf(mt, s[i]);
  mt = xgroup_max(mt);
  const float m_new = fmaxf(st.m_run, mt);
  const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
  const float alpha = fast_exp2(st.m_run - m_use);
  float psum = 0.0f, pmax = 0.0f;
  float pv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float pe = fast_exp2(s[i] - m_use);
    psum += pe;
    pv[i] = pe * svv[i];
    pmax = fmaxf(pmax, pv[i]);
  }
  psum = xgroup_sum(psum);
  pmax = xgroup_max(pmax);
  st.l_run = st.l_run * alpha + psum;
  st.m_run = m_new;

  // P' -> int8 (hi, lo) terms; this lane's term is its row of the PV A operand
  const float sp = pmax * (1.0f / 127.0f);
  const float inv_sp = pmax > 0.0f ? 127.0f / pmax : 0.0f;
  int pc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float hi = rintf(pv[i] * inv_sp);
    const float lo = fminf(fmaxf(rintf((pv[i] - hi * sp) * (254.0f * inv_sp)), -127.0f), 127.0f);
    pc[i] = live ? (int)(is_hi ? hi : lo) : 0;
  }
  v4i pa;
#pragma unroll
  for (int w = 0; w < 4; ++w) pa[w] = pack4(pc[4 * w], pc[4 * w + 1], pc[4 * w + 2], pc[4 * w + 3]);

  // rescale factors of the heads this lane accumulates (2g, 2g+1); head h's
  // softmax state sits in lanes with head-term 2h (read from lane 2h)
  float a0 = 0.0f, a1 = 0.0f, s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int h2 = 0; h2 < (G + 1) / 2; ++h2) {
    const int ah0 = __builtin_amdgcn_readlane(__float_as_int(alpha), 4 * h2);
    const int sh0 = __builtin_amdgcn_readlane(__float_as_int(sp), 4 * h2);
    const int ah1 = G > 2 * h2 + 1 ? __builtin_amdgcn_readlane(__float_as_int(alpha), 4 * h2 + 2) : 0;
    const int sh1 = G > 2 * h2 + 1 ? __builtin_amdgcn_readlane(__float_as_int(sp), 4 * h2 + 2) : 0;
    if (g == h2) {
      a0 = __int_as_float(ah0);
      s0 = __int_as_float(sh0);
      a1 = __int_as_float(ah1);
      s1 = __int_as_float(sh1);
    }
  }
  const float s0l = s0 * (1.0f / 254.0f);
  const float s1l = s1 * (1.0f / 254.0f);

  // P' V on the matrix cores
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
    const v4i co = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, T.vb[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
    st.acc[jb][0] = st.acc[jb][0] * a0 + ((float)co[0] * s0 + (float)co[1] * s0l);
    st.acc[jb][1] = st.acc[jb][1] * a1 + ((float)co[2] * s1 + (float)co[3] * s1l);
  }
  after_pv();
}

template <int D, int G, int NW>
__global__ __launch_bounds__(64 * NW, 2) void gqa_decode_int8_kernel(DecodeParams p) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static_assert(G >= 1 && G <= 8, "group");
  constexpr int KS = D / 64;
  constexpr int JB = D / 16;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int work = blockIdx.x;

  // ---- (sequence, split) of this workgroup ------------------------------------
  int b, split, nsplit, split_base;
  decode_work_item(p, work, lane, b, split, nsplit, split_base);
  if (b < 0 || b >= p.batch) return;  // uniform over the workgroup

  // page ids of the split, loaded before the length is known (the page-table
  // row has max_pages entries; the split's range is clamped to it)
  const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
  // length first; then the page ids of the split and the query, in flight
  // across the barrier
  const int L = p.seq_lens[b] + p.pending;
  // sliding window: keys [k_lo, L) visible, splits from the tile holding k_lo
  const int k_lo = window_first_key(L, p.window);
  const int origin = (k_lo / 64) * 64;
  const int first_page = origin / kPageTokens + split * (p.split_tokens / kPageTokens);
  __shared__ int sm_pg[kMaxSplitPages];
  const int split_pages = p.split_tokens / kPageTokens;
  for (int i = threadIdx.x; i < split_pages; i += 64 * NW)
    sm_pg[i] = pt[min(first_page + i, p.max_pages - 1)];

  constexpr int HALF = D / 2;
  const int hterm = r;  // column j of the QK product
  const int h = hterm >> 1;
  const bool is_hi = (hterm & 1) == 0;
  const bool live = h < G;
  const int Hq = p.kv_heads * G;
  const size_t qbase = ((size_t)b * Hq + kvh * G + (live ? h : 0)) * D;
  float xq[KS][16];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) load16(p.q, qbase + kdim0<D>(g, ks), p.q_dtype, xq[ks]);
  const int t_begin = origin + split * p.split_tokens;
  const int t_end = min(L, t_begin + p.split_tokens);
  const int n_pages_split = (t_end - 1) / kPageTokens - first_page + 1;
  const int n_tiles = (t_end - t_begin + 63) / 64;
  // the wave that streams the split's last tile (it holds the newest token)
  const int last_owner = (n_tiles - 1) % NW;
  __syncthreads();

  // cos / sin of position L-1: issued ahead of the first tile, so the query's
  // RoPE only waits for them and not for the tile (head_dim 256 loads them per
  // chunk in the RoPE loop and its first tile after the query: the registers
  // of both would not fit)
  constexpr bool BIG = D > 128;
  float cq[BIG ? 1 : KS][16], sq[BIG ? 1 : KS][16];
  if (!BIG && p.do_rotary) {
    const float* cr = p.cos_cache + (size_t)(L - 1) * HALF;
    const float* sr = p.sin_cache + (size_t)(L - 1) * HALF;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c0 = kdim0<D>(g, ks);
      const int base = p.interleaved ? (c0 >> 1) : (c0 < HALF ? c0 : c0 - HALF);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int idx = base + (p.interleaved ? (i >> 1) : i);
        cq[ks][i] = cr[idx];
        sq[ks][i] = sr[idx];
      }
    }
  }

  // ---- fused append by the last tile's owner: before its first load if that
  // tile is its only one, else while its first tile is in flight -----------------
  const bool appender = p.k_new != nullptr && split == nsplit - 1 && wave == last_owner;
  int tile = wave;
  const int my_tiles = tile < n_tiles ? (n_tiles - 1 - tile) / NW + 1 : 0;
  auto append = [&]() {
    const int pos = L - 1;
    uint8_t* blk = (uint8_t*)p.pool +
                   block_offset(sm_pg[pos / kPageTokens - first_page], kvh, p.num_pages,
                                block_bytes_int8(D));
    const size_t row = ((size_t)b * p.kv_heads + kvh) * D * (p.kv_dtype == kDtypeBf16 ? 2 : 4);
    append_row_int8<D>((const uint8_t*)p.k_new + row, (const uint8_t*)p.v_new + row, p.kv_dtype,
                       lane, pos, blk, pos % kPageTokens, p.do_rotary, p.interleaved != 0,
                       p.cos_cache, p.sin_cache);
    // this wave reads the page back in its last tile: order the stores first
    __threadfence_block();
  };
  if (appender && my_tiles == 1) append();
  const int tile_off = 0;  // splits start on a tile (64-token) boundary
  TileRegs<D> TA;
  if (!BIG && tile < n_tiles)
    load_tile<D>(TA, p.pool, sm_pg + tile_off, tile, p.num_pages, kvh, r, g, n_pages_split);
  // The wave's second tile is touched (one dword per 128-byte line) so that
  // it streams into L2 while the query is prepared, instead of the memory
  // pipe idling until the loop issues its load. Its own lines only: the new
  // token's page may be rewritten by the append below. The values are
  // consumed only where the first tile is needed anyway.
  // Branch-free (lanes past the last line repeat it): a divergent branch here
  // would make the compiler wait for every outstanding load at its join.
  constexpr int kLines = (int)(block_bytes_int8(D) / 128);  // 33 for D = 128
  constexpr int kTouch = (4 * kLines + 63) / 64;              // loads per lane
  uint32_t touch[kTouch];
#pragma unroll
  for (int j = 0; j < kTouch; ++j) touch[j] = 0;
  if (!BIG && my_tiles > 1 && !(appender && my_tiles == 2)) {  // uniform over the wave
    const int t1 = tile + NW;
#pragma unroll
    for (int j = 0; j < kTouch; ++j) {
      const int line = min(lane + 64 * j, 4 * kLines - 1);
      const int pg = sm_pg[min(t1 * 4 + line / kLines, n_pages_split - 1)];
      const uint8_t* a = p.pool + block_offset(pg, kvh, p.num_pages, block_bytes_int8(D)) +
                         (size_t)(line % kLines) * 128;
      touch[j] = *(const uint32_t*)a;
    }
  }
  if (appender && my_tiles > 1) append();

  // ---- Q: RoPE at position L-1, split into int8 (hi, lo) terms -------------
  v4i qB[KS];
  float sq_hi;
  {
    float qv[KS][16];
    float amax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c0 = kdim0<D>(g, ks);  // first dim of this lane's chunk
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = xq[ks][i];
      if (p.do_rotary) {
        float y[16];
        float cc[16], ss[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if constexpr (BIG) {
            const int base = p.interleaved ? (c0 >> 1) : (c0 < HALF ? c0 : c0 - HALF);
            const int idx = base + (p.interleaved ? (i >> 1) : i);
            cc[i] = p.cos_cache[(size_t)(L - 1) * HALF + idx];
            ss[i] = p.sin_cache[(size_t)(L - 1) * HALF + idx];
          } else {
            cc[i] = cq[ks][i];
            ss[i] = sq[ks][i];
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // split-half partner d +- D/2: up to head_dim 128 the same element
          // of lane g ^ 2 (32 lanes away; permlane32_swap(x, x) gives [0] =
          // lanes 0-31's x, [1] = lanes 32-63's x on both halves); at 256 the
          // same lane's chunk ks ^ 2
          float half_partner;
          if constexpr (BIG) {
            half_partner = xq[ks ^ 2][i];
          } else {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[i]),
                                                       __float_as_uint(x[i]), false, false);
            half_partner = __uint_as_float(c0 < HALF ? sw[1] : sw[0]);
          }
          const float partner = p.interleaved ? x[i ^ 1] : half_partner;
          const bool first = p.interleaved ? (i & 1) == 0 : c0 < HALF;
          y[i] = rope_elem(cc[i], ss[i], x[i], partner, first);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = y[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        qv[ks][i] = live ? x[i] : 0.0f;
        amax = fmaxf(amax, fabsf(qv[ks][i]));
      }
    }
    amax = xgroup_max(amax);
    sq_hi = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
    const float inv_sq = 1.0f / sq_hi;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      int c[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float y = qv[ks][i];
        const float hi = fminf(fmaxf(rintf(y * inv_sq), -127.0f), 127.0f);
        const float lo = fminf(fmaxf(rintf((y - hi * sq_hi) * (254.0f * inv_sq)), -127.0f), 127.0f);
        c[i] = live ? (int)(is_hi ? hi : lo) : 0;
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) qB[ks][w] = pack4(c[4 * w], c[4 * w + 1], c[4 * w + 2], c[4 * w + 3]);
    }
  }
  // the softmax scale (log2 domain) rides on the Q term scales
  const float sq_hi_s = sq_hi * p.scale_log2;
  const float sq_lo_s = sq_hi_s * (1.0f / 254.0f);
  const float q_own = is_hi ? sq_hi_s : sq_lo_s;
  const float q_oth = is_hi ? sq_lo_s : sq_hi_s;
  __shared__ float sm_sc[NW][128];

  // ---- stream the split's tiles, double-buffered --------------------------------
  WaveState<D, G> st;
  st.m_run = -INFINITY;
  st.l_run = 0.0f;
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) st.acc[jb][0] = st.acc[jb][1] = 0.0f;

  // Ping-pong over this wave's tiles wave, wave+NW, ... Every prefetch inside
  // the loop is unconditional (straight-line code), so the compiler's wait
  // counts only cover the tile being computed, never the one in flight.
  TileRegs<D> TB;
  auto tok0 = [&](int k) { return t_begin + (wave + k * NW) * 64 + 16 * g; };
  auto ld = [&](TileRegs<D>& T, int k) {
    load_tile<D>(T, p.pool, sm_pg + tile_off, wave + k * NW, p.num_pages, kvh, r, g,
                 n_pages_split);
  };
  // the touch loads, consumed (an empty asm use keeps them): issued right
  // after the first tile, which the loop waits for first anyway
#pragma unroll
  for (int j = 0; j < kTouch; ++j) __asm__ volatile("" ::"v"(touch[j]));
  int k = 0;
  if constexpr (D <= 128) {
    for (; k + 2 < my_tiles; k += 2) {
      ld(TB, k + 1);
      compute_tile<D, G>(TA, st, qB, q_own, q_oth, tok0(k), k_lo, t_end, is_hi, live, g, sm_sc[wave]);
      ld(TA, k + 2);
      compute_tile<D, G>(TB, st, qB, q_own, q_oth, tok0(k + 1), k_lo, t_end, is_hi, live, g, sm_sc[wave]);
    }
    if (k + 1 < my_tiles) {  // two left
      ld(TB, k + 1);
      compute_tile<D, G>(TA, st, qB, q_own, q_oth, tok0(k), k_lo, t_end, is_hi, live, g, sm_sc[wave]);
      compute_tile<D, G>(TB, st, qB, q_own, q_oth, tok0(k + 1), k_lo, t_end, is_hi, live, g, sm_sc[wave]);
    } else if (k < my_tiles) {  // one left
      compute_tile<D, G>(TA, st, qB, q_own, q_oth, tok0(k), k_lo, t_end, is_hi, live, g, sm_sc[wave]);
    }
  } else {
    // head_dim 256: a tile is ~128 registers, so one buffer, refilled by
    // phase: the next tile's K (and scales) load as soon as this tile's QK is
    // issued, its V as soon as this tile's PV is (the last tile reloads
    // itself, so the code stays straight-line)
    if (my_tiles > 0) ld(TA, 0);
    for (; k < my_tiles; ++k) {
      const int kn = wave + min(k + 1, my_tiles - 1) * NW;
      compute_tile<D, G>(
          TA, st, qB, q_own, q_oth, tok0(k), k_lo, t_end, is_hi, live, g, sm_sc[wave],
          [&]() {
            load_tile<D, 1>(TA, p.pool, sm_pg + tile_off, kn, p.num_pages, kvh, r, g, n_pages_split);
          },
          [&]() {
            load_tile<D, 2>(TA, p.pool, sm_pg + tile_off, kn, p.num_pages, kvh, r, g, n_pages_split);
          });
    }
  }

  // ---- merge the NW waves of the workgroup --------------------------------------
  __shared__ float sm_m[NW][G];
  __shared__ float sm_l[NW][G];
  __shared__ float sm_o[NW][G][D];
  if (g == 0 && is_hi && live) {
    sm_m[wave][h] = st.m_run;
    sm_l[wave][h] = st.l_run;
  }
#pragma unroll
  for (int jb = 0; jb < JB; ++jb)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int hd = 2 * g + hh;
      if (hd < G) sm_o[wave][hd][16 * jb + r] = st.acc[jb][hh];
    }
  __syncthreads();

  float* part = p.partials + ((size_t)(split_base + split) * p.kv_heads + kvh) * (G * (D + 2));
  // (m, l, o) of this split for the (head, dim) entries t = threadIdx.x + k*64*NW
  constexpr int PER = (G * D + 64 * NW - 1) / (64 * NW);
  float mM[PER], mL[PER], mO[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int t = threadIdx.x + k * 64 * NW;
    if (G * D % (64 * NW) != 0 && t >= G * D) break;
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
      O += sm_o[w][hd][d] * f;
    }
    mM[k] = M;
    mL[k] = Ls;
    mO[k] = O;
    if (nsplit == 1) {
      p.out[((size_t)b * Hq + kvh * G + hd) * D + d] = Ls > 0.0f ? O / Ls : 0.0f;
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

  // ---- in-kernel merge: the last workgroup of (b, kvh) to finish merges -------
  // Every thread releases its own partial stores at agent scope (the splits
  // run on different XCDs, whose L2s are not coherent with each other), the
  // barrier orders those releases before thread 0's counter increment, and
  // the last workgroup acquires before reading. The counter resets itself.
  __shared__ int sm_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&p.counters[b * p.kv_heads + kvh], 1);
    sm_last = (prev == nsplit - 1);
    if (sm_last) __threadfence();
  }
  __syncthreads();
  if (!sm_last) return;
  const size_t stride = (size_t)p.kv_heads * (G * (D + 2));
  const float* p0 = p.partials + ((size_t)split_base * p.kv_heads + kvh) * (G * (D + 2));
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int t = threadIdx.x + k * 64 * NW;
    if (G * D % (64 * NW) != 0 && t >= G * D) break;
    const int hd = t / D, d = t % D;
    float M = mM[k], Ls = mL[k], O = mO[k];
    // the other splits' (m, l, o), up to 16 loads in flight per round
    for (int s0 = 0; s0 < nsplit; s0 += 16) {
      float pm[16], pl[16], po[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float* ps = p0 + (size_t)min(s0 + j, nsplit - 1) * stride + hd * (D + 2);
        pm[j] = ps[0];
        pl[j] = ps[1];
        po[j] = ps[2 + d];
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int sidx = s0 + j;
        if (sidx >= nsplit || sidx == split || pm[j] == -INFINITY) continue;
        const float Mn = fmaxf(M, pm[j]);
        const float fa = fast_exp2(M - Mn);
        const float fb = fast_exp2(pm[j] - Mn);
        Ls = Ls * fa + pl[j] * fb;
        O = O * fa + po[j] * fb;
        M = Mn;
      }
    }
    p.out[((size_t)b * Hq + kvh * G + hd) * D + d] = Ls > 0.0f ? O / Ls : 0.0f;
  }
  if (threadIdx.x == 0) atomicExch(&p.counters[b * p.kv_heads + kvh], 0);
}

// Merge of the split partials of one (sequence, kv head): grid (batch, Hkv),
// one thread per (head, dim) entry. The partials were just written by other
// workgroups (often on other XCDs), so every global read is a full memory
// latency: each thread loads the (m, l, o) of C splits in one batch and merges
// them online (C = the split count rounded up to 2, 4, 8 or 16, so a 2-split
// merge is one round trip of 6 loads); with a uniform split count the range
// comes from the launch, not from seq_info.
template <int D, int G, int C>
__global__ __launch_bounds__(G * D) void gqa_decode_combine_kernel(DecodeParams p) {
  const int b = blockIdx.x;
  const int kvh = blockIdx.y;
  int split_base, nsplit;
  if (p.uniform_nsplit > 0) {
    nsplit = p.uniform_nsplit;
    split_base = b * nsplit;
  } else {
    split_base = p.seq_info[2 * b];
    nsplit = p.seq_info[2 * b + 1];
  }
  if (nsplit <= 1) return;
  const int Hq = p.kv_heads * G;
  const size_t stride = (size_t)p.kv_heads * (G * (D + 2));
  const float* p0 = p.partials + ((size_t)split_base * p.kv_heads + kvh) * (G * (D + 2));
  const int t = threadIdx.x;
  const int hd = t / D, d = t % D;
  const float* ph = p0 + hd * (D + 2);
  float M = -INFINITY, Ls = 0.0f, O = 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += C) {
    float m[C], l[C], o[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const bool in = s0 + i < nsplit;
      const float* ps = ph + (size_t)(in ? s0 + i : s0) * stride;
      m[i] = in ? ps[0] : -INFINITY;
      l[i] = ps[1];
      o[i] = ps[2 + d];
    }
    float mb = M;
#pragma unroll
    for (int i = 0; i < C; ++i) mb = fmaxf(mb, m[i]);
    if (mb == -INFINITY) continue;
    const float f0 = M == -INFINITY ? 0.0f : fast_exp2(M - mb);
    Ls *= f0;
    O *= f0;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float f = m[i] == -INFINITY ? 0.0f : fast_exp2(m[i] - mb);
      Ls += l[i] * f;
      O += o[i] * f;
    }
    M = mb;
  }
  p.out[((size_t)b * Hq + kvh * G + hd) * D + d] = Ls > 0.0f ? O / Ls : 0.0f;
}

template <int D, int G>
hipError_t launch_combine_dg(const DecodeParams& p, hipStream_t st) {
  // the largest split count decides the batch width (uniform: the launch's;
  // ragged: bounded by the longest sequence)
  const int n = p.uniform_nsplit > 0 ? p.uniform_nsplit : p.max_nsplit;
  const dim3 grid(p.batch, p.kv_heads), block(G * D);
  if (n <= 2)
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, G, 2>), grid, block, 0, st, p);
  else if (n <= 4)
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, G, 4>), grid, block, 0, st, p);
  else if (n <= 8)
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, G, 8>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, G, 16>), grid, block, 0, st, p);
  return hipGetLastError();
}

template <int D, int G>
hipError_t launch_dg(const DecodeParams& p, int work_items, bool combine, hipStream_t st) {
  const dim3 grid(work_items, p.kv_heads);
  if (p.waves == 8)
    hipLaunchKernelGGL((gqa_decode_int8_kernel<D, G, 8>), grid, dim3(512), 0, st, p);
  else
    hipLaunchKernelGGL((gqa_decode_int8_kernel<D, G, 4>), grid, dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !combine || p.merge_in_kernel) return e;
  return launch_combine_dg<D, G>(p, st);
}

template <int D>
hipError_t launch_d(const DecodeParams& p, int group, int work_items, bool combine,
                    hipStream_t st) {
  switch (group) {
    case 1: return launch_dg<D, 1>(p, work_items, combine, st);
    case 2: return launch_dg<D, 2>(p, work_items, combine, st);
    case 4: return launch_dg<D, 4>(p, work_items, combine, st);
    case 8:
      // the combine block is one thread per (head, dim): 8 x 256 is past 1024
      if constexpr (D <= 128) return launch_dg<D, 8>(p, work_items, combine, st);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_decode_combine(const DecodeParams& p, int head_dim, int group, hipStream_t st) {
  auto by_group = [&](auto d) -> hipError_t {
    constexpr int D = decltype(d)::value;
    switch (group) {
      case 1: return launch_combine_dg<D, 1>(p, st);
      case 2: return launch_combine_dg<D, 2>(p, st);
      case 4: return launch_combine_dg<D, 4>(p, st);
      case 8: return launch_combine_dg<D, 8>(p, st);
      default: return hipErrorInvalidValue;
    }
  };
  if (head_dim == 64) return by_group(std::integral_constant<int, 64>{});
  if (head_dim == 128) return by_group(std::integral_constant<int, 128>{});
  if (head_dim == 256 && group <= 4) return by_group(std::integral_constant<int, 256>{});
  return hipErrorInvalidValue;
}

hipError_t launch_gqa_decode(const DecodeParams& p, int head_dim, int group, int quant,
                             int work_items, bool combine, hipStream_t st) {
  if (quant == kQuantInt4) return launch_gqa_decode_int4(p, head_dim, group, work_items, combine, st);
  if (quant != kQuantInt8) return hipErrorInvalidValue;
  if (p.split_tokens <= 0 || p.split_tokens % 64 != 0 ||
      p.split_tokens > kMaxSplitPages * kPageTokens)
    return hipErrorInvalidValue;
  if (head_dim == 64) return launch_d<64>(p, group, work_items, combine, st);
  if (head_dim == 128) return launch_d<128>(p, group, work_items, combine, st);
  if (head_dim == 256 && group <= 4) return launch_d<256>(p, group, work_items, combine, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
