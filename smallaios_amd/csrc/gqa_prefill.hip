// Kernel 3: prefill chunk -- causal GQA attention of sq new query tokens per
// sequence over the paged int8 cache (past + the chunk, already appended by
// kernel 1), on f16 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Workgroup = 4 waves = 128 attention rows = (128/G query positions) x (G
// heads of one kv head), so every K/V tile is loaded once per workgroup and
// shared by the whole GQA group. Per 64-token KV tile (4 pages):
//   staging  all threads: int8 codes -> f16 (exact: |code| <= 128) into LDS,
//            K token-major, V in the permuted k-order the PV operand needs;
//            rows padded so the 16-byte LDS reads are bank-conflict free.
//   S^T      A = K tile (LDS), B = Q^T (registers, f16 of q / rowmax|q|);
//            lane (row r, g) receives tokens 4g+e of each 16-token block,
//            so the row softmax is in-lane plus two cross-group shuffles and
//            P feeds the PV A operand straight from registers.
//   PV       A = P * s_v / max(s_v) (f16), B = V codes (LDS f16); the tile's
//            max(s_v) is carried in the accumulator's running scale.
// Scores are rescaled per element: s = <q', k_code> * rowmax|q| * s_k[t] *
// scale * log2(e); online softmax in the log2 domain.
#include "sai_internal.h"

namespace sai {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float rope_elem(float c, float s, float own, float partner,
                                           bool first) {
#pragma clang fp contract(off)
  return first ? (c * own - s * partner) : (s * partner + c * own);
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

__device__ __forceinline__ float xgroup_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float xgroup_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D, int G>
__global__ __launch_bounds__(256) void gqa_prefill_int8_kernel(PrefillParams p) {
  constexpr int KS = D / 32;       // 32-dim k steps of QK
  constexpr int JB = D / 16;       // 16-dim column blocks of PV
  constexpr int QT = 128 / G;      // query positions per workgroup
  constexpr int KROW = D + 8;      // padded f16 row of the K tile
  constexpr int VROW = 4 * 8 + 8;  // padded f16 (kstep, dim) row of the V tile: 4 groups x 8
  constexpr size_t BB = block_bytes_int8(D);

  __shared__ _Float16 sK[64 * KROW];
  __shared__ _Float16 sV[2 * D * VROW];
  __shared__ float sSk[64];
  __shared__ float sSv[64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int n_qt = (p.sq + QT - 1) / QT;
  const int qtile = n_qt - 1 - (int)blockIdx.x;  // longest rows first
  const int q0 = qtile * QT;
  const int past = p.seq_lens[b];
  const int total = past + p.sq;
  const int Hq = p.kv_heads * G;
  const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
  const int last_page = (total - 1) / kPageTokens;

  // ---- Q^T operand: rows R = wave*32 + rb*16 + r -> (position, head) -------
  v8h qB[2][KS];
  float qfac[2];   // rowmax|q| * scale * log2(e)
  int qpos[2];     // absolute position of the row (clamped for dead rows)
  bool qlive[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int R = wave * 32 + rb * 16 + r;
    const int il = q0 + R / G;
    const int hq = kvh * G + R % G;
    qlive[rb] = il < p.sq;
    const int i = qlive[rb] ? il : p.sq - 1;
    const int pos = past + i;
    qpos[rb] = pos;
    const size_t qbase = (((size_t)b * p.sq + i) * Hq + hq) * D;
    constexpr int HALF = D / 2;
    float x[KS][8];
    float amax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * g + 32 * ks + e;
        float v = load_elem(p.q, qbase + d, p.q_dtype);
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
          const float vp = load_elem(p.q, qbase + dp, p.q_dtype);
          v = rope_elem(p.cos_cache[(size_t)pos * HALF + pi], p.sin_cache[(size_t)pos * HALF + pi],
                        v, vp, first);
        }
        x[ks][e] = v;
        amax = fmaxf(amax, fabsf(v));
      }
    amax = xgroup_max(amax);
    const float inv = amax > 0.0f ? 1.0f / amax : 0.0f;
    qfac[rb] = amax * p.scale_log2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) qB[rb][ks][e] = (_Float16)(x[ks][e] * inv);
  }

  // ---- online softmax state ----------------------------------------------------
  float m_run[2] = {-INFINITY, -INFINITY};  // lane (row r): row r of block rb
  float l_run[2] = {0.0f, 0.0f};
  v4f acc[2][JB];  // lane (dim r of block jb, g): rows 4g+e of block rb
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) acc[rb][jb] = v4f{0.f, 0.f, 0.f, 0.f};
  float vscale = 1.0f;  // accumulator units: true O = acc * vscale

  const int max_pos = past + min(q0 + QT, p.sq) - 1;
  const int n_tiles = max_pos / 64 + 1;
  for (int tile = 0; tile < n_tiles; ++tile) {
    const int t0 = tile * 64;
    __syncthreads();  // previous tile's LDS reads are done
    // -- stage K: 64 tokens x D codes, 16-code chunks
    for (int c = tid; c < 64 * (D / 16); c += 256) {
      const int tok = c / (D / 16);
      const int dp = c % (D / 16);
      const int pg = min((t0 + tok) / kPageTokens, last_page);
      const uint8_t* blk = p.pool + block_offset(pt[pg], kvh, p.num_pages, BB);
      const uint4 w = *(const uint4*)(blk + (size_t)((t0 + tok) % kPageTokens) * D + 16 * dp);
      uint32_t h[8];
      codes4_to_f16(w.x, h[0], h[1]);
      codes4_to_f16(w.y, h[2], h[3]);
      codes4_to_f16(w.z, h[4], h[5]);
      codes4_to_f16(w.w, h[6], h[7]);
      uint4* dst = (uint4*)(sK + tok * KROW + 16 * dp);
      dst[0] = uint4{h[0], h[1], h[2], h[3]};
      dst[1] = uint4{h[4], h[5], h[6], h[7]};
    }
    // -- stage V: (page cb, dim d) rows of 16 slots -> sV[kst][d][g][elem]
    for (int c = tid; c < 4 * D; c += 256) {
      const int cb = c / D;
      const int d = c % D;
      const int pg = min(t0 / kPageTokens + cb, last_page);
      const uint8_t* blk = p.pool + block_offset(pt[pg], kvh, p.num_pages, BB);
      const uint4 w = *(const uint4*)(blk + 16 * D + (size_t)d * 16);
      const int kst = cb >> 1;
      const int half = (cb & 1) * 4;
      _Float16* row = sV + ((size_t)kst * D + d) * VROW;
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {  // slots 4gg..4gg+3
        uint32_t h01, h23;
        codes4_to_f16(ws[gg], h01, h23);
        *(uint2*)(row + gg * 8 + half) = uint2{h01, h23};
      }
    }
    if (tid < 128) {
      const int which = tid >> 6;
      const int tok = tid & 63;
      const int pg = min((t0 + tok) / kPageTokens, last_page);
      const uint8_t* blk = p.pool + block_offset(pt[pg], kvh, p.num_pages, BB);
      const float v = ((const float*)(blk + 32 * D + 64 * which))[(t0 + tok) % kPageTokens];
      const bool ok = t0 + tok < total;
      if (which == 0)
        sSk[tok] = ok ? v : 0.0f;
      else
        sSv[tok] = ok ? v : 0.0f;
    }
    __syncthreads();

    const float svmax = wave_max(sSv[lane]);
    const float inv_svmax = svmax > 0.0f ? 1.0f / svmax : 0.0f;

#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      // S^T for this row block: 4 column blocks of 16 tokens
      float s[4][4];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        v4f c = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const v8h a = *(const v8h*)(sK + (16 * cb + r) * KROW + 8 * g + 32 * ks);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qB[rb][ks], c, 0, 0, 0);
        }
        const float4 skv = *(const float4*)(sSk + 16 * cb + 4 * g);
        const float skx[4] = {skv.x, skv.y, skv.z, skv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = t0 + 16 * cb + 4 * g + e;
          const float sc = c[e] * qfac[rb] * skx[e];
          s[cb][e] = (t <= qpos[rb]) ? sc : -INFINITY;
        }
      }
      float mt = -INFINITY;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mt = fmaxf(mt, s[cb][e]);
      mt = xgroup_max(mt);
      const float m_new = fmaxf(m_run[rb], mt);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run[rb] - m_use);
      float psum = 0.0f;
      v8h pa[2];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const float4 svv = *(const float4*)(sSv + 16 * cb + 4 * g);
        const float svx[4] = {svv.x, svv.y, svv.z, svv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = fast_exp2(s[cb][e] - m_use);
          psum += pe;
          pa[cb >> 1][(cb & 1) * 4 + e] = (_Float16)(pe * svx[e] * inv_svmax);
        }
      }
      psum = xgroup_sum(psum);
      l_run[rb] = l_run[rb] * alpha + psum;
      m_run[rb] = m_new;

      // rescale the accumulator rows 4g+e (alpha of row j lives in lane j)
      const float ratio = vscale * inv_svmax;  // old units -> new units
      float ae[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ae[e] = __shfl(alpha, 4 * g + e, 64) * (svmax > 0.0f ? ratio : 1.0f);
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) {
        v4f o = acc[rb][jb];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] *= ae[e];
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
          const v8h bv = *(const v8h*)(sV + ((size_t)kst * D + 16 * jb + r) * VROW + 8 * g);
          o = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kst], bv, o, 0, 0, 0);
        }
        acc[rb][jb] = o;
      }
    }
    if (svmax > 0.0f) vscale = svmax;
  }

  // ---- write O / l ------------------------------------------------------------
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * g + e;  // row within the block
      const float l = __shfl(l_run[rb], row, 64);
      const int R = wave * 32 + rb * 16 + row;
      const int il = q0 + R / G;
      if (il >= p.sq) continue;
      const int hq = kvh * G + R % G;
      float* o = p.out + (((size_t)b * p.sq + il) * Hq + hq) * D;
      const float f = l > 0.0f ? vscale / l : 0.0f;
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) o[16 * jb + r] = acc[rb][jb][e] * f;
    }
  }
}

template <int D>
hipError_t launch_d(const PrefillParams& p, int group, hipStream_t st) {
  auto grid = [&](int qt) { return dim3((p.sq + qt - 1) / qt, p.kv_heads, p.batch); };
  switch (group) {
    case 1: hipLaunchKernelGGL((gqa_prefill_int8_kernel<D, 1>), grid(128), dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((gqa_prefill_int8_kernel<D, 2>), grid(64), dim3(256), 0, st, p); break;
    case 4: hipLaunchKernelGGL((gqa_prefill_int8_kernel<D, 4>), grid(32), dim3(256), 0, st, p); break;
    case 8: hipLaunchKernelGGL((gqa_prefill_int8_kernel<D, 8>), grid(16), dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gqa_prefill(const PrefillParams& p, int head_dim, int group, int quant,
                              hipStream_t st) {
  if (quant != kQuantInt8) return hipErrorInvalidValue;
  if (head_dim == 64) return launch_d<64>(p, group, st);
  if (head_dim == 128) return launch_d<128>(p, group, st);
  return hipErrorInvalidValue;
}

}  // namespace sai
