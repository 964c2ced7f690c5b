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
//   score(t, h) = s_k[t] * sq[h] * (<k_t, qhi_h> + <k_t, qmid_h>/254 + <k_t, qlo_h>/254^2)
//   out(h, :)   = sum_t p'(t, h) * v_t,   p' = p * s_v[t] = sp[h]*(phi + plo/254)
// Q (after RoPE) is split into three int8 terms (~24 significant bits, so
// keys with large outlier channels do not amplify its rounding) and each
// tile's P' into two (hi + residual/254, error ~1/64516 of the tile's
// maximum); the terms ride in spare MFMA rows/columns (a DPP quad holds one
// head's terms), so the split costs no extra MFMA issue.
//
// Wave layout (lane = r + 16 g, r = lane & 15, g = lane >> 4). A tile is 64
// tokens = 4 pages; lane group g of a tile works on page g.
//   QK  : S^T = K * Q^T.  A = K codes, row i of MFMA #blk is token
//         (page i>>2, slot 4*blk + (i&3)); B = Q terms, column j = head-term
//         (head j>>2, term j&3: 0 = hi, 1 = mid, 2 = lo, 3 = zero). The
//         result lands with lane (j, g) holding head-term j for all 16 slots
//         of page g -- exactly the A-operand layout the PV product needs (its
//         rows j = hi and lo terms of P'), so no LDS transpose.
//         k index: lane group g, k step ks <-> dims kdim0(g, ks) + [0,16):
//         (D/4)*g + 16*ks up to head_dim 128, so one row's 4 lane groups read
//         one contiguous 128-byte line; 16*g + 64*ks at the stored widths 192
//         and 256, so they read 64 contiguous bytes of a longer row per load
//         instruction. (head_dim 168 runs at the stored width 192: each
//         84-dim half padded to 96 with zeros; the query, RoPE tables and the
//         output go through that mapping.)
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
// head. The NW waves of a workgroup take the split's tiles from an LDS
// counter and merge through LDS. A sequence with one split writes its output
// directly; with several, every workgroup writes a partial (m, l, o), and
// either the workgroup that takes the last ticket of its (sequence, kv head)
// merges them (agent-scope stores and loads, below) or the combine kernel, a
// second launch, does.
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
// partner chunk held for RoPE spills registers). The stored width 192 (rows
// of 1.5 lines) takes 16*g + 64*ks too: 57.5 % of HBM with (D/4)*g + 16*ks.
template <int D>
__device__ __forceinline__ constexpr int kdim0(int g, int ks) {
  return D > 128 ? 16 * g + 64 * ks : (D / 4) * g + 16 * ks;
}

// The 16 query elements of stored dims [c0, c0 + 16) of a row of the caller's
// kLogicalDim<D> elements (qrow: element offset of the row). At the stored
// width 192 a chunk may hold padding dims, loaded as 0, and its real dims
// start at an element offset that is only a multiple of 4: four loads of 4
// elements each.
template <int D>
__device__ __forceinline__ void load_q16(const void* q, size_t qrow, int c0, int dtype,
                                         float (&x)[16]) {
  if constexpr (kLogicalDim<D> == D) {
    load16(q, qrow + c0, dtype, x);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int el = logical_dim<D>(c0 + 4 * k);  // 4 dims, all real or all padding
      const size_t at = qrow + (el < 0 ? 0 : el);
      float v[4];
      if (dtype == kDtypeBf16) {
        const uint2 w = *(const uint2*)((const uint16_t*)q + at);
        v[0] = __uint_as_float(w.x << 16), v[1] = __uint_as_float(w.x & 0xFFFF0000u);
        v[2] = __uint_as_float(w.y << 16), v[3] = __uint_as_float(w.y & 0xFFFF0000u);
      } else {
        const float4 f = *(const float4*)((const float*)q + at);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * k + i] = el < 0 ? 0.0f : v[i];
    }
  }
}

// Per-dim cos / sin of stored dims [c0, c0 + 16) at the stored width 192
// (tables of 84 entries per position): one load each, padding dims read
// entry 0 (their values are 0 and stay 0).
template <int D>
__device__ __forceinline__ void rope_table16_padded(const float* cr, const float* sr, int c0,
                                                    bool interleaved, float (&c)[16],
                                                    float (&s)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = c0 + i;
    const int el = logical_dim<D>(e);
    const int t = el < 0 ? 0 : (interleaved ? (el >> 1) : (e < D / 2 ? e : e - D / 2));
    c[i] = cr[t];
    s[i] = sr[t];
  }
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

// Heads of a group are taken four at a time (a "pass"): column j = 4*hq + t
// of the QK product is term t of head 4*pass + hq, so the four lanes of a
// DPP quad hold the terms of one head.
template <int G>
struct Passes {
  static constexpr int N = G > 4 ? 2 : 1;
};

template <int D, int G>
struct WaveState {
  static constexpr int NP = Passes<G>::N;
  float m_run[NP], l_run[NP];  // this lane's head of each pass, log2 domain
  float acc[NP][D / 16];       // lane (dim 16*jb + r, group g): head 4*pass + g
};

struct NoHook {
  __device__ void operator()() const {}
};

// sum over the four lanes of a DPP quad; every lane gets the same bits
// (x0 + x1) + (x2 + x3), since f32 addition commutes
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
  return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
}

// One 64-token tile. qB[pass] holds this lane's query term (t = r & 3 of head
// 4*pass + (r >> 2); t = 3 is zero) and qw[pass] its weight, so that
//   score(t, h) = s_k[t] * sum over the quad of qw * <k_t, term>.
// after_qk runs once the tile's K codes and scales are consumed (the QK
// MFMAs issued, the scales in LDS), after_pv once its V codes are: a caller
// with one tile buffer loads the next tile's K and V there.
template <int D, int G, class H1 = NoHook, class H2 = NoHook>
__device__ __forceinline__ void compute_tile(const TileRegs<D>& T, WaveState<D, G>& st,
                                             const v4i (&qB)[Passes<G>::N][D / 64],
                                             const float (&qw)[Passes<G>::N],
                                             int tok0, int t_lo, int t_end, int r, int g,
                                             float* sm_sc, H1 after_qk = H1{},
                                             H2 after_pv = H2{}) {
  constexpr int KS = D / 64;
  constexpr int JB = D / 16;
  constexpr int NP = Passes<G>::N;
  // QK^T of a pass on the matrix cores (the first pass's before the scales
  // are exchanged, the second's when its turn comes: one set of results live)
  v4i cs[4];
  auto qk = [&](int ps) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      cs[blk] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        cs[blk] = __builtin_amdgcn_mfma_i32_16x16x64_i8(T.ka[blk][ks], qB[ps][ks], cs[blk], 0, 0, 0);
    }
  };
  qk(0);
  // scales of page g, slots 0..15 (this wave's LDS slot; lane 16g + r wrote slot r)
  const int lane = threadIdx.x & 63;
  sm_sc[lane] = T.sk;
  sm_sc[64 + lane] = T.sv;
  // with two passes (group 8) the second pass's QK below still reads this
  // tile's K codes, so the hook waits for it
  if constexpr (NP == 1) after_qk();
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
  if (!full) {
#pragma unroll
    for (int i = 0; i < 16; ++i) svv[i] = i < nvalid && i >= nlow ? svv[i] : 0.0f;
  }
  const int t = r & 3;
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const bool live = 4 * ps + (r >> 2) < G;
    if (ps > 0) {
      qk(ps);
      if (ps == NP - 1) after_qk();
    }
    float s[16];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int slot = 4 * blk + e;
        s[slot] = quad_sum(qw[ps] * (float)cs[blk][e]) * skv[slot];
      }
    if (!full) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = i < nvalid && i >= nlow ? s[i] : -INFINITY;
    }
    float mt = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mt = fmaxf(mt, s[i]);
    mt = xgroup_max(mt);
    const float m_new = fmaxf(st.m_run[ps], mt);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = fast_exp2(st.m_run[ps] - m_use);
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
    st.l_run[ps] = st.l_run[ps] * alpha + psum;
    st.m_run[ps] = m_new;

    // P' -> int8 (hi, lo) terms: term t = 0 / 1 of the quad is its row of
    // the PV A operand (rows 4*hq + 2, 4*hq + 3 are zero)
    const float sp = pmax * (1.0f / 127.0f);
    // hardware reciprocal (1 ulp): hi stays within +-127 (rint of at most
    // 127 (1 + 2^-22)), and lo takes up the difference
    const float inv_sp = pmax > 0.0f ? 127.0f * __builtin_amdgcn_rcpf(pmax) : 0.0f;
    int pc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float hi = rintf(pv[i] * inv_sp);
      const float lo =
          fminf(fmaxf(rintf((pv[i] - hi * sp) * (254.0f * inv_sp)), -127.0f), 127.0f);
      pc[i] = live && t < 2 ? (int)(t == 0 ? hi : lo) : 0;
    }
    v4i pa;
#pragma unroll
    for (int w = 0; w < 4; ++w) pa[w] = pack4(pc[4 * w], pc[4 * w + 1], pc[4 * w + 2], pc[4 * w + 3]);

    // rescale factor and P' scale of the head this lane accumulates
    // (4*ps + g); head 4*ps + hq's softmax state sits in lanes r = 4*hq + t
    float a_g = 0.0f, sp_g = 0.0f;
#pragma unroll
    for (int hq = 0; hq < 4; ++hq) {
      if (4 * ps + hq >= G) break;
      const float ah = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), 4 * hq));
      const float sh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sp), 4 * hq));
      a_g = g == hq ? ah : a_g;
      sp_g = g == hq ? sh : sp_g;
    }
    const float sp_gl = sp_g * (1.0f / 254.0f);

    // P' V on the matrix cores: output rows 4g .. 4g + 3 are head 4*ps + g's terms
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) {
      const v4i co = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, T.vb[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
      st.acc[ps][jb] = st.acc[ps][jb] * a_g + ((float)co[0] * sp_g + (float)co[1] * sp_gl);
    }
  }
  after_pv();
}

// Two waves per SIMD, except group 8 at head_dim 128 and 256: its two passes
// of query terms and accumulators do not fit beside the tile buffers in 256
// registers, so it runs one wave per SIMD with the whole register file.
template <int D, int G>
constexpr bool kInt8OneWavePerSimd = G > 4 && D >= 128;

template <int D, int G, int NW>
__global__ __launch_bounds__(64 * NW, (kInt8OneWavePerSimd<D, G>) ? 1 : 2) void gqa_decode_int8_kernel(
    DecodeParams p) {
  static_assert(D == 64 || D == 128 || D == 192 || D == 256, "stored head_dim");
  static_assert(G >= 1 && G <= 8, "group");
  constexpr int KS = D / 64;
  constexpr int JB = D / 16;
  constexpr int DL = kLogicalDim<D>;  // the caller's rows (q, k_new, v_new, out)

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int work = blockIdx.x;

  // ---- (sequence, split) of this workgroup ------------------------------------
  int b, split, nsplit, split_base, tps;
  decode_work_item(p, work, lane, b, split, nsplit, split_base, tps);
  if (b < 0 || b >= p.batch) return;  // uniform over the workgroup

  // length and the split's page ids (the page-table row has max_pages
  // entries; the split's range is clamped to it), then the query, all in
  // flight across the barrier. Sliding window: keys [k_lo, L) visible, splits
  // from the tile holding k_lo.
  __shared__ int sm_pg[kMaxSplitPages];
  int L, k_lo, first_page;
  stage_split_pages<64 * NW>(p, b, split, tps, sm_pg, L, k_lo, first_page);
  const int origin = (k_lo / 64) * 64;

  constexpr int HALF = D / 2;
  constexpr int HL = DL / 2;  // table entries per position
  constexpr int NP = Passes<G>::N;
  // column r = 4*hq + t of the QK product: term t of head 4*pass + hq
  const int tq = r & 3;
  const int Hq = p.kv_heads * G;
  float xq[NP][KS][16];
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const int h = 4 * ps + (r >> 2);
    const size_t qbase = ((size_t)b * Hq + kvh * G + (h < G ? h : 0)) * DL;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) load_q16<D>(p.q, qbase, kdim0<D>(g, ks), p.q_dtype, xq[ps][ks]);
  }
  const int t_begin = origin + split * tps * 64;
  const int t_end = min(L, t_begin + tps * 64);
  const int n_pages_split = (t_end - 1) / kPageTokens - first_page + 1;
  const int n_tiles = (t_end - t_begin + 63) / 64;
  // next tile of the split to hand out (see below)
  __shared__ int sm_next;
  if (threadIdx.x == 0) sm_next = 0;
  __syncthreads();

  // cos / sin of position L-1: issued ahead of the first tile, so the query's
  // RoPE only waits for them and not for the tile (the stored widths 192 and
  // 256 load them per chunk in the RoPE loop and their first tile after the
  // query: the registers of both would not fit)
  constexpr bool BIG = D > 128;
  constexpr bool WIDE = D == 256;  // split-half partners in the lane's own chunks
  float4 cq[BIG ? 1 : KS][4], sq[BIG ? 1 : KS][4];
  if (!BIG && p.do_rotary) {
    const float* cr = p.cos_cache + (size_t)(L - 1) * HL;
    const float* sr = p.sin_cache + (size_t)(L - 1) * HL;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) rope_load16<D>(cr, sr, kdim0<D>(g, ks), p.interleaved, cq[ks], sq[ks]);
  }

  // ---- tiles are handed out one at a time from an LDS counter (a wave takes
  // the index of its next tile one tile ahead, and loads that tile just
  // before computing the current one), so the waves of a workgroup finish
  // together however their loads are served. Each wave's first tile is fixed
  // (its index). The split that holds the step's new token keeps its last
  // tile out of the count: the appender wave (the last one) writes the token
  // and then streams that tile first; no other wave touches that page.
  // (Sharing one counter in memory between the workgroups of a sequence was
  // measured 18 % slower at 16 x 8k: its atomics serialise.)
  const bool appender_split = p.k_new != nullptr && split == nsplit - 1;
  const bool appender = appender_split && wave == NW - 1;
  const int pool_end = appender_split ? n_tiles - 1 : n_tiles;
  const int slots = NW;  // fixed first tiles
  const int pool_start = slots - (appender_split ? 1 : 0);
  // Static order (p.static_tiles): wave w takes tiles w, w + NW, w + 2 NW, ...
  // (the appender wave NW - 1, 2 NW - 1, ... after the new token's tile), so
  // every launch accumulates the same tiles in the same order in each wave
  // and the output is bit-reproducible.
  const int static_base = appender ? NW - 1 : wave + NW;
  int grabs = 0;
  auto grab_issue = [&]() {  // dynamic: lane 0 holds the counter's old value
    int t = 0;
    if (p.static_tiles)
      t = grabs++;
    else if (lane == 0)
      t = atomicAdd(&sm_next, 1);
    return t;
  };
  auto grab_value = [&](int t) {
    return p.static_tiles ? static_base + NW * t : pool_start + __builtin_amdgcn_readfirstlane(t);
  };
  if (appender) {
    const int pos = L - 1;
    uint8_t* blk = (uint8_t*)p.pool +
                   block_offset(sm_pg[pos / kPageTokens - first_page], kvh, p.num_pages,
                                block_bytes_int8(D));
    const size_t row = ((size_t)b * p.kv_heads + kvh) * DL * (p.kv_dtype == kDtypeBf16 ? 2 : 4);
    append_row_int8<D>((const uint8_t*)p.k_new + row, (const uint8_t*)p.v_new + row, p.kv_dtype,
                       lane, pos, blk, pos % kPageTokens, p.do_rotary, p.interleaved != 0,
                       p.cos_cache, p.sin_cache);
    // this wave reads the page back right below: order the stores first
    __threadfence_block();
  }
  const int first = appender ? n_tiles - 1 : wave;
  const bool have_first = appender || first < pool_end;
  // the next tile's index, asked for before the first tile's loads so that
  // waiting for it never waits for them
  int gq = 0;
  if (have_first) gq = grab_issue();
  // The first tile's loads and the touch below are issued by every wave (a
  // wave without a tile re-reads tile 0 of its split, which always exists):
  // behind a branch, the compiler's wait counts for the query's loads would
  // have to assume the branch was not taken and wait for these loads too.
  TileRegs<D> TA;
  const int first_ld = have_first ? first : 0;
  if constexpr (!BIG)
    load_tile<D>(TA, p.pool, sm_pg, first_ld, p.num_pages, kvh, r, g, n_pages_split);
  // Tile first + slots (the one this wave most likely takes next, never the
  // appender's; else the first tile again) is touched (one dword per 128-byte
  // line) so that it streams into L2 while the query is prepared, instead of
  // the memory pipe idling until the loop issues its load. The values are
  // consumed only where the first tile is needed anyway. Branch-free (lanes
  // past the last line repeat it).
  constexpr int kLines = (int)(block_bytes_int8(D) / 128);  // 33 for D = 128
  constexpr int kTouch = (4 * kLines + 63) / 64;              // loads per lane
  uint32_t touch[kTouch];
#pragma unroll
  for (int j = 0; j < kTouch; ++j) touch[j] = 0;
  if constexpr (!BIG) {
    const int t1 = have_first && first + slots < pool_end ? first + slots : first_ld;
#pragma unroll
    for (int j = 0; j < kTouch; ++j) {
      const int line = min(lane + 64 * j, 4 * kLines - 1);
      const int pg = sm_pg[min(t1 * 4 + line / kLines, n_pages_split - 1)];
      const uint8_t* a = p.pool + block_offset(pg, kvh, p.num_pages, block_bytes_int8(D)) +
                         (size_t)(line % kLines) * 128;
      touch[j] = *(const uint32_t*)a;
    }
  }

  // ---- Q: RoPE at position L-1, split into three int8 terms ------------------
  // y = sq * (hi + mid / 254 + lo / 254^2), sq = max|y| / 127 over the head:
  // ~24 significant bits, about f32's own. (Two terms, ~16 bits, put keys
  // with x20 outlier channels at 0.96 of the output tolerance: their score
  // terms reach the hundreds.) Each lane packs its own term t; t = 3 is zero.
  v4i qB[NP][KS];
  float qw[NP];
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const bool live = 4 * ps + (r >> 2) < G;
    float qv[KS][16];
    float amax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c0 = kdim0<D>(g, ks);  // first dim of this lane's chunk
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = xq[ps][ks][i];
      if (p.do_rotary) {
        float y[16];
        float cc[16], ss[16];
        if constexpr (DL != D) {
          rope_table16_padded<D>(p.cos_cache + (size_t)(L - 1) * HL,
                                 p.sin_cache + (size_t)(L - 1) * HL, c0, p.interleaved != 0, cc, ss);
        } else if constexpr (BIG) {
          float4 lc[4], ls[4];
          rope_load16<D>(p.cos_cache + (size_t)(L - 1) * HALF, p.sin_cache + (size_t)(L - 1) * HALF,
                         c0, p.interleaved, lc, ls);
          rope_pick_all<0>(lc, ls, p.interleaved != 0, cc, ss);
        } else {
          rope_pick_all<0>(cq[ks], sq[ks], p.interleaved != 0, cc, ss);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // split-half partner d +- D/2: up to head_dim 128 the same element
          // of lane g ^ 2 (32 lanes away; permlane32_swap(a, b) gives [1] =
          // a of lanes 32-63 on lanes 0-31, [0] = b of lanes 0-31 on lanes
          // 32-63); at 256 the same lane's chunk ks ^ 2; at the stored width
          // 192 chunk (ks + 1) % 3 of lane group g + 2 for g < 2 and chunk
          // (ks + 2) % 3 of lane group g - 2 for g >= 2
          float half_partner;
          if constexpr (WIDE) {
            half_partner = xq[ps][ks ^ 2][i];
          } else if constexpr (D == 192) {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(xq[ps][(ks + 1) % 3][i]),
                                                       __float_as_uint(xq[ps][(ks + 2) % 3][i]),
                                                       false, false);
            half_partner = __uint_as_float(g < 2 ? sw[1] : sw[0]);
          } else {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[i]),
                                                       __float_as_uint(x[i]), false, false);
            half_partner = __uint_as_float(c0 < HALF ? sw[1] : sw[0]);
          }
          const float partner = p.interleaved ? x[i ^ 1] : half_partner;
          const bool first = p.interleaved ? (i & 1) == 0 : c0 < HALF;
          y[i] = rope_elem(cc[i], ss[i], x[i], partner, first);
          // padding dims stay 0 whatever the table holds
          if constexpr (DL != D) y[i] = logical_dim<D>(c0 + i) < 0 ? 0.0f : y[i];
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
    const float s0 = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
    const float inv = 1.0f / s0;
    const float s1 = s0 * (1.0f / 254.0f);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      int c[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float y = qv[ks][i];
        const float hi = fminf(fmaxf(rintf(y * inv), -127.0f), 127.0f);
        const float r1 = y - hi * s0;
        const float mid = fminf(fmaxf(rintf(r1 * (254.0f * inv)), -127.0f), 127.0f);
        const float r2 = r1 - mid * s1;
        const float lo = fminf(fmaxf(rintf(r2 * (64516.0f * inv)), -127.0f), 127.0f);
        c[i] = live && tq < 3 ? (int)(tq == 0 ? hi : (tq == 1 ? mid : lo)) : 0;
      }
#pragma unroll
      for (int w = 0; w < 4; ++w)
        qB[ps][ks][w] = pack4(c[4 * w], c[4 * w + 1], c[4 * w + 2], c[4 * w + 3]);
    }
    // the softmax scale (log2 domain) rides on the term weights
    const float w0 = s0 * p.scale_log2;
    qw[ps] = tq == 0 ? w0 : (tq == 1 ? w0 * (1.0f / 254.0f) : (tq == 2 ? w0 * (1.0f / 64516.0f) : 0.0f));
  }
  __shared__ float sm_sc[NW][128];

  // ---- stream the split's tiles, double-buffered --------------------------------
  WaveState<D, G> st;
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    st.m_run[ps] = -INFINITY;
    st.l_run[ps] = 0.0f;
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) st.acc[ps][jb] = 0.0f;
  }

  // Ping-pong between two tile buffers: the next tile is taken and its load
  // issued before the current one is computed, so one tile is always in
  // flight; the loads inside the loop are unconditional once a tile is taken.
  TileRegs<D> TB;
  auto tok0 = [&](int tile) { return t_begin + tile * 64 + 16 * g; };
  auto ld = [&](TileRegs<D>& T, int tile) {
    load_tile<D>(T, p.pool, sm_pg, tile, p.num_pages, kvh, r, g, n_pages_split);
  };
  // the touch loads, consumed (an empty asm use keeps them): issued right
  // after the first tile, which the loop waits for first anyway
#pragma unroll
  for (int j = 0; j < kTouch; ++j) __asm__ volatile("" ::"v"(touch[j]));
  // (the index for the tile after next is asked for before the next tile's
  // loads are issued, for the same reason as above)
  if constexpr (D <= 128) {
    if (have_first) {
      int cur = first;
      for (;;) {
        const int n1 = grab_value(gq);
        if (n1 >= pool_end) {
          compute_tile<D, G>(TA, st, qB, qw, tok0(cur), k_lo, t_end, r, g, sm_sc[wave]);
          break;
        }
        gq = grab_issue();
        ld(TB, n1);
        compute_tile<D, G>(TA, st, qB, qw, tok0(cur), k_lo, t_end, r, g, sm_sc[wave]);
        const int n2 = grab_value(gq);
        if (n2 >= pool_end) {
          compute_tile<D, G>(TB, st, qB, qw, tok0(n1), k_lo, t_end, r, g, sm_sc[wave]);
          break;
        }
        gq = grab_issue();
        ld(TA, n2);
        compute_tile<D, G>(TB, st, qB, qw, tok0(n1), k_lo, t_end, r, g, sm_sc[wave]);
        cur = n2;
      }
    }
  } else {
    // head_dim 256: a tile is ~128 registers, so one buffer, refilled by
    // phase: the next tile's K (and scales) load as soon as this tile's QK is
    // issued, its V as soon as this tile's PV is (the last tile reloads
    // itself, so the code stays straight-line)
    if (have_first) {
      int cur = first;
      ld(TA, cur);
      for (;;) {
        const int n1 = grab_value(gq);
        const bool more = n1 < pool_end;
        const int kn = more ? n1 : cur;
        // asked for unconditionally (straight-line code); the last one is
        // never used
        gq = grab_issue();
        compute_tile<D, G>(
            TA, st, qB, qw, tok0(cur), k_lo, t_end, r, g, sm_sc[wave],
            [&]() { load_tile<D, 1>(TA, p.pool, sm_pg, kn, p.num_pages, kvh, r, g, n_pages_split); },
            [&]() { load_tile<D, 2>(TA, p.pool, sm_pg, kn, p.num_pages, kvh, r, g, n_pages_split); });
        if (!more) break;
        cur = n1;
      }
    }
  }

  // ---- merge the NW waves of the workgroup --------------------------------------
  __shared__ float sm_m[NW][G];
  __shared__ float sm_l[NW][G];
  __shared__ float sm_o[NW][G][D];
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const int h = 4 * ps + (r >> 2);
    if (g == 0 && tq == 0 && h < G) {
      sm_m[wave][h] = st.m_run[ps];
      sm_l[wave][h] = st.l_run[ps];
    }
    const int hd = 4 * ps + g;
#pragma unroll
    for (int jb = 0; jb < JB; ++jb)
      if (hd < G) sm_o[wave][hd][16 * jb + r] = st.acc[ps][jb];
  }
  __syncthreads();

  float* part = p.partials + ((size_t)(split_base + split) * p.kv_heads + kvh) * (G * (D + 2));
  // (m, l, o) of this split for the (head, dim) entries t = threadIdx.x + k*64*NW
  constexpr int PER = (G * D + 64 * NW - 1) / (64 * NW);
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
    const int dl = logical_dim<D>(d);  // -1: a padding dim, not written
    if (nsplit == 1) {
      if (dl >= 0)
        store_out(p.out, ((size_t)b * Hq + kvh * G + hd) * DL + dl, Ls > 0.0f ? O / Ls : 0.0f,
                  p.out_bf16);
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

  // ---- in-kernel merge: the workgroup with the last ticket of (b, kvh) -------
  // Its partial stores are agent-scope, so once they have completed (every
  // wave waits for its own, then the barrier) they are visible to the other
  // XCDs; thread 0 then takes a ticket. The last workgroup loads the other
  // splits' partials with agent-scope loads and writes the output.
  __shared__ int sm_last;
  partials_complete();
  __syncthreads();
  int* counter = &p.counters[b * p.kv_heads + kvh];
  if (threadIdx.x == 0) sm_last = last_ticket(counter, nsplit);
  __syncthreads();
  if (!sm_last) return;
  const size_t stride = (size_t)p.kv_heads * (G * (D + 2));
  const float* p0 = p.partials + ((size_t)split_base * p.kv_heads + kvh) * (G * (D + 2));
  // every split's partial, this workgroup's own included, in split order: the
  // result does not depend on which workgroup finished last
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int t = threadIdx.x + k * 64 * NW;
    if (G * D % (64 * NW) != 0 && t >= G * D) break;
    const int hd = t / D, d = t % D;
    float M = -INFINITY, Ls = 0.0f, O = 0.0f;
    const float* ph = p0 + hd * (D + 2);
    merge_all_splits(ph, stride, d, nsplit, M, Ls, O);
    const int dl = logical_dim<D>(d);
    if (dl >= 0)
      store_out(p.out, ((size_t)b * Hq + kvh * G + hd) * DL + dl, Ls > 0.0f ? O / Ls : 0.0f,
                p.out_bf16);
  }
  if (threadIdx.x == 0) reset_ticket(counter);
}

// Merge of the split partials of one (sequence, kv head): grid (batch, Hkv),
// one thread per (head, dim) entry. The partials were just written by other
// workgroups (often on other XCDs), so every global read is a full memory
// latency: each thread loads the (m, l, o) of C splits in one batch and merges
// them online (C = the split count rounded up to 2, 4, 8 or 16, so a 2-split
// merge is one round trip of 6 loads); with a uniform split count the range
// comes from the launch, not from seq_info.
template <int D, int G>
constexpr int kCombineThreads = G * D < 1024 ? G * D : 1024;

template <int D, int G, int C>
__global__ __launch_bounds__((kCombineThreads<D, G>)) void gqa_decode_combine_kernel(DecodeParams p) {
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
  // (head, dim) entries t, t + 1024, ... (8 x 256 entries take two rounds)
  for (int t = threadIdx.x; t < G * D; t += kCombineThreads<D, G>) {
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
  const int dl = logical_dim<D>(d);
  if (dl >= 0)
    store_out(p.out, ((size_t)b * Hq + kvh * G + hd) * kLogicalDim<D> + dl,
              Ls > 0.0f ? O / Ls : 0.0f, p.out_bf16);
  }
}

template <int D, int G>
hipError_t launch_combine_dg(const DecodeParams& p, hipStream_t st) {
  // the largest split count decides the batch width (uniform: the launch's;
  // ragged: bounded by the longest sequence)
  const int n = p.uniform_nsplit > 0 ? p.uniform_nsplit : p.max_nsplit;
  const dim3 grid(p.batch, p.kv_heads), block(kCombineThreads<D, G>);
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
  // group 8 at head_dim 128 and 256 needs one wave per SIMD (see the kernel),
  // which an 8-wave workgroup cannot give: always 4 waves there
  constexpr bool kEightWaves = !kInt8OneWavePerSimd<D, G>;
  if (kEightWaves && p.waves == 8)
    hipLaunchKernelGGL((gqa_decode_int8_kernel<D, G, kEightWaves ? 8 : 4>), grid,
                       dim3(kEightWaves ? 512 : 256), 0, st, p);
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
    case 8: return launch_dg<D, 8>(p, work_items, combine, st);
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
  if (head_dim == 256) return by_group(std::integral_constant<int, 256>{});
  if (head_dim == 168) return by_group(std::integral_constant<int, 192>{});
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
  if (head_dim == 256) return launch_d<256>(p, group, work_items, combine, st);
  if (head_dim == 168) return launch_d<192>(p, group, work_items, combine, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
