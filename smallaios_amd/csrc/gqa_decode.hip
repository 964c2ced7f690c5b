// Kernel 2: split-K flash decode over the paged int8 cache (one query token
// per sequence, GQA group of G query heads per kv head).
//
// Why int8 MFMA. At the Llama-3-8B layer shape (G = 4, D = 128) a decode step
// reads 264 B per (token, kv head) and does 4 * 128 * 2 multiply-adds on them.
// Dequantising every code to f32 and doing those multiply-adds on the VALU
// costs more vector cycles than the HBM stream leaves (~90 SIMD cycles per
// token-head at 80 % of 8 TB/s); the VALU would be the bound. Instead the int8
// codes go straight from HBM into v_mfma_i32_16x16x64_i8 operands and the
// per-token scales are applied to the 32-bit dot products:
//   score(t, h) = s_k[t] * (sq_hi[h] * <k_t, qhi_h> + sq_lo[h] * <k_t, qlo_h>)
//   out(h, :)   = sum_t p'(t, h) * v_t,   p' = p * s_v[t] = sp[h]*(phi + plo/254)
// Q (after RoPE) and P' are split into two int8 terms (hi + residual/254) so
// their representation error is ~1/64516 of the row maximum; both terms ride in
// spare MFMA rows/columns, so the split costs no extra MFMA issue.
//
// Wave layout (lane = r + 16 g, r = lane & 15, g = lane >> 4). A tile is 64
// tokens = 4 pages; "group" g of a tile is page g.
//   QK  : S^T = K * Q^T.  A = K codes, row i of MFMA #blk is token
//         (page i>>2, slot 4*blk + (i&3)); B = Q terms, column j = head-term
//         (head j>>1, term j&1: 0 = hi, 1 = lo). The result lands with lane
//         (j, g) holding head-term j for all 16 slots of page g -- exactly the
//         A-operand layout the PV product needs, so no LDS transpose.
//   PV  : O = P' * V.  A = P' codes (row = head-term, k = slots of page g),
//         B = V codes read dim-major from the page (column = dim).
//   Online softmax in the log2 domain; cross-page reductions are two
//   shuffles (lanes j, j+16, j+32, j+48), the hi/lo pairing one DPP swap.
//
// Work split: grid.x enumerates (sequence, split) pairs for ragged lengths
// (each wave finds its pair by a prefix scan over seq_lens), grid.y is the kv
// head. NW waves of a workgroup take interleaved tiles of the split and merge
// through LDS; when a sequence has several splits, every workgroup writes a
// partial (m, l, o) and the last one to finish (atomic counter, no waiting)
// merges them and resets the counter.
#include "sai_internal.h"

namespace sai {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// RoPE of one element, unfused like rotate_rope_block
// (onnx-rt/src/ops/microsoft.rs:137-160).
__device__ __forceinline__ float rope_elem(float c, float s, float own, float partner,
                                           bool first) {
#pragma clang fp contract(off)
  return first ? (c * own - s * partner) : (s * partner + c * own);
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

__device__ __forceinline__ int swap_pair(int v) {
  // quad_perm(1,0,3,2): exchange with the neighbouring lane
  return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}

__device__ __forceinline__ float xgroup_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

__device__ __forceinline__ float xgroup_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D, int G, int NW>
__global__ __launch_bounds__(64 * NW) void gqa_decode_int8_kernel(DecodeParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  static_assert(G >= 1 && G <= 8, "group");
  constexpr int KS = D / 64;  // 64-dim k steps of the QK product
  constexpr int JB = D / 16;  // 16-dim column blocks of the PV product
  constexpr size_t BB = block_bytes_int8(D);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int work = blockIdx.x;

  // ---- (sequence, split) of this workgroup: prefix scan over split counts ----
  int b = -1, split = 0, nsplit = 0, split_base = 0;
  {
    int base = 0;
    for (int c0 = 0; c0 < p.batch; c0 += 64) {
      const int bi = c0 + lane;
      const int L = bi < p.batch ? p.seq_lens[bi] + p.pending : 0;
      const int n = (L + p.split_tokens - 1) / p.split_tokens;
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
        break;
      }
      base += total;
    }
  }
  if (b < 0) return;  // uniform over the workgroup

  const int L = p.seq_lens[b] + p.pending;
  const int t_begin = split * p.split_tokens;
  const int t_end = min(L, t_begin + p.split_tokens);
  const int last_page = (L - 1) / kPageTokens;
  const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
  const uint8_t* pool = p.pool;
  const int Hq = p.kv_heads * G;

  // ---- Q: RoPE at position L-1, split into int8 (hi, lo) terms -------------
  const int hterm = r;  // column j of the QK product
  const int h = hterm >> 1;
  const bool is_hi = (hterm & 1) == 0;
  const bool live = h < G;
  float qv[KS][16];
  float amax = 0.0f;
  {
    const int pos = L - 1;
    const int hq = kvh * G + (live ? h : 0);
    const size_t qbase = ((size_t)b * Hq + hq) * D;
    constexpr int HALF = D / 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 16 * g + 64 * ks + i;
        float x = load_elem(p.q, qbase + d, p.q_dtype);
        if (p.do_rotary) {
          int dp, pi;
          bool first;
          if (p.interleaved) {
            dp = d ^ 1;
            pi = d >> 1;
            first = (d & 1) == 0;
          } else {
            first = d < HALF;
            dp = first ? d + HALF : d - HALF;
            pi = first ? d : d - HALF;
          }
          const float xp = load_elem(p.q, qbase + dp, p.q_dtype);
          x = rope_elem(p.cos_cache[(size_t)pos * HALF + pi], p.sin_cache[(size_t)pos * HALF + pi],
                        x, xp, first);
        }
        qv[ks][i] = live ? x : 0.0f;
        amax = fmaxf(amax, fabsf(qv[ks][i]));
      }
    }
  }
  amax = xgroup_max(amax);
  const float sq_hi = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
  const float inv_sq = 1.0f / sq_hi;
  const float sq_lo = sq_hi * (1.0f / 254.0f);
  v4i qB[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    int c[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float y = qv[ks][i];
      float hi = rintf(y * inv_sq);
      hi = fminf(fmaxf(hi, -127.0f), 127.0f);
      const float res = y - hi * sq_hi;
      float lo = rintf(res * (254.0f * inv_sq));
      lo = fminf(fmaxf(lo, -127.0f), 127.0f);
      c[i] = live ? (int)(is_hi ? hi : lo) : 0;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) qB[ks][w] = pack4(c[4 * w], c[4 * w + 1], c[4 * w + 2], c[4 * w + 3]);
  }
  const float q_own = is_hi ? sq_hi : sq_lo;
  const float q_oth = is_hi ? sq_lo : sq_hi;

  // ---- stream the split's tiles ---------------------------------------------
  float m_run = -INFINITY;  // per head (lanes of head-term j), log2 domain
  float l_run = 0.0f;
  float acc[JB][2];  // lane (dim 16*jb + r, group g): heads 2g, 2g+1
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) acc[jb][0] = acc[jb][1] = 0.0f;

  const int n_tiles = (t_end - t_begin + 63) / 64;
  for (int tile = wave; tile < n_tiles; tile += NW) {
    const int t0 = t_begin + tile * 64;
    const int pg_g = min(t0 / kPageTokens + g, last_page);
    const int pg_k = min(t0 / kPageTokens + (r >> 2), last_page);
    const uint8_t* blk_g = pool + ((size_t)pt[pg_g] * p.kv_heads + kvh) * BB;
    const uint8_t* blk_k = pool + ((size_t)pt[pg_k] * p.kv_heads + kvh) * BB;

    v4i ka[4][KS];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        ka[blk][ks] =
            *(const v4i*)(blk_k + (size_t)(4 * blk + (r & 3)) * D + 16 * g + 64 * ks);
    v4i vb[JB];
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) vb[jb] = *(const v4i*)(blk_g + 16 * D + (16 * jb + r) * 16);
    float sk[16], sv[16];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 a = *(const float4*)(blk_g + 32 * D + 16 * w);
      const float4 c = *(const float4*)(blk_g + 32 * D + 64 + 16 * w);
      sk[4 * w] = a.x, sk[4 * w + 1] = a.y, sk[4 * w + 2] = a.z, sk[4 * w + 3] = a.w;
      sv[4 * w] = c.x, sv[4 * w + 1] = c.y, sv[4 * w + 2] = c.z, sv[4 * w + 3] = c.w;
    }

    // QK^T on the matrix cores
    v4i cs[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      cs[blk] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        cs[blk] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[blk][ks], qB[ks], cs[blk], 0, 0, 0);
    }

    // scores of page g, slots 0..15 (slot = 4*blk + e)
    float s[16];
    const int tok0 = t0 + 16 * g;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int slot = 4 * blk + e;
        const int own = cs[blk][e];
        const int oth = swap_pair(own);
        const float raw = q_own * (float)own + q_oth * (float)oth;
        const float sc = raw * sk[slot] * p.scale_log2;
        s[slot] = (tok0 + slot < t_end) ? sc : -INFINITY;
      }
    }
    float mt = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mt = fmaxf(mt, s[i]);
    mt = xgroup_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float psum = 0.0f, pmax = 0.0f;
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float pe = fast_exp2(s[i] - m_use);
      psum += pe;
      pv[i] = (tok0 + i < t_end) ? pe * sv[i] : 0.0f;
      pmax = fmaxf(pmax, pv[i]);
    }
    psum = xgroup_sum(psum);
    pmax = xgroup_max(pmax);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // P' -> int8 (hi, lo) terms; this lane's term is its row of the PV A operand
    const float sp = pmax * (1.0f / 127.0f);
    const float inv_sp = pmax > 0.0f ? 127.0f / pmax : 0.0f;
    int pc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float hi = rintf(pv[i] * inv_sp);
      const float res = pv[i] - hi * sp;
      float lo = rintf(res * (254.0f * inv_sp));
      lo = fminf(fmaxf(lo, -127.0f), 127.0f);
      pc[i] = live ? (int)(is_hi ? hi : lo) : 0;
    }
    v4i pa;
#pragma unroll
    for (int w = 0; w < 4; ++w) pa[w] = pack4(pc[4 * w], pc[4 * w + 1], pc[4 * w + 2], pc[4 * w + 3]);

    // rescale factors of the two heads this lane accumulates (2g, 2g+1):
    // held by lanes with head-term 4g + 2hh, i.e. lane 20g + 2hh
    const float a0 = __shfl(alpha, 20 * g, 64);
    const float a1 = __shfl(alpha, 20 * g + 2, 64);
    const float s0 = __shfl(sp, 20 * g, 64);
    const float s1 = __shfl(sp, 20 * g + 2, 64);
    const float s0l = s0 * (1.0f / 254.0f);
    const float s1l = s1 * (1.0f / 254.0f);

    // P' V on the matrix cores
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) {
      const v4i co = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
      acc[jb][0] = acc[jb][0] * a0 + (float)co[0] * s0 + (float)co[1] * s0l;
      acc[jb][1] = acc[jb][1] * a1 + (float)co[2] * s1 + (float)co[3] * s1l;
    }
  }

  // ---- merge the NW waves of the workgroup --------------------------------------
  __shared__ float sm_m[NW][G];
  __shared__ float sm_l[NW][G];
  __shared__ float sm_o[NW][G][D];
  if (g == 0 && is_hi && live) {
    sm_m[wave][h] = m_run;
    sm_l[wave][h] = l_run;
  }
#pragma unroll
  for (int jb = 0; jb < JB; ++jb)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int hd = 2 * g + hh;
      if (hd < G) sm_o[wave][hd][16 * jb + r] = acc[jb][hh];
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
      O += sm_o[w][hd][d] * f;
    }
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
  if (nsplit == 1) return;

  // ---- last workgroup of this (sequence, kv head) merges the splits -----------
  __shared__ int sm_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&p.counters[b * p.kv_heads + kvh], 1);
    sm_last = (prev == nsplit - 1);
  }
  __syncthreads();
  if (!sm_last) return;
  __threadfence();
  const size_t stride = (size_t)p.kv_heads * (G * (D + 2));
  const float* p0 = p.partials + ((size_t)split_base * p.kv_heads + kvh) * (G * (D + 2));
  for (int t = threadIdx.x; t < G * D; t += 64 * NW) {
    const int hd = t / D, d = t % D;
    float M = -INFINITY;
    for (int sidx = 0; sidx < nsplit; ++sidx) M = fmaxf(M, p0[sidx * stride + hd * (D + 2)]);
    float Ls = 0.0f, O = 0.0f;
    for (int sidx = 0; sidx < nsplit; ++sidx) {
      const float* ps = p0 + sidx * stride + hd * (D + 2);
      if (ps[0] == -INFINITY) continue;
      const float f = fast_exp2(ps[0] - M);
      Ls += ps[1] * f;
      O += ps[2 + d] * f;
    }
    p.out[((size_t)b * Hq + kvh * G + hd) * D + d] = Ls > 0.0f ? O / Ls : 0.0f;
  }
  if (threadIdx.x == 0) atomicExch(&p.counters[b * p.kv_heads + kvh], 0);
}

template <int D, int G>
hipError_t launch_dg(const DecodeParams& p, int work_items, hipStream_t st) {
  constexpr int NW = 4;
  hipLaunchKernelGGL((gqa_decode_int8_kernel<D, G, NW>), dim3(work_items, p.kv_heads),
                     dim3(64 * NW), 0, st, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(const DecodeParams& p, int group, int work_items, hipStream_t st) {
  switch (group) {
    case 1: return launch_dg<D, 1>(p, work_items, st);
    case 2: return launch_dg<D, 2>(p, work_items, st);
    case 4: return launch_dg<D, 4>(p, work_items, st);
    case 8: return launch_dg<D, 8>(p, work_items, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gqa_decode(const DecodeParams& p, int head_dim, int group, int quant,
                             int work_items, hipStream_t st) {
  if (quant != kQuantInt8) return hipErrorInvalidValue;
  if (head_dim == 64) return launch_d<64>(p, group, work_items, st);
  if (head_dim == 128) return launch_d<128>(p, group, work_items, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
