// TurboQuant compressed KV cache (CompressedKVCache of
// onnx-rt/src/kv_compression.rs:738-963, without the optional low-rank K)
// on gfx950: write, read, and the decode-attention fast path of the design
// (docs/kv-compression-design.md section 9) over the stored codes.
//
// A row (one token of one kv head, K or V) is PolarQuant-encoded
// (kv_compression.rs:216-268): signs s (the head's xorshift +-1 vector),
// normalised Walsh-Hadamard butterfly y = H(s*x)/sqrt(D), one min/max
// quantiser over y (codes of 3, 4 or 8 bits, packed LSB first), and, with
// QJL on (:365-395), the sign bits of r = x - decode(codes) and C = mean|r|.
// The write kernel does these f32 steps in the reference's order (no
// contraction, IEEE division), so codes, scale, zero, sign bits and C are the
// reference's bit for bit.
//
// Attention never decodes a key. Decoding is linear and orthonormal, so
//   <decode(q), decode(k_t)> = <q^, k^_t>   with  k^_t = s_t * code_t + z_t
// in the rotated domain, where q^ is the encoded query's rotated
// reconstruction; the logit adds the QJL popcount correction
// C_q C_t (D - 2 popcount(sq ^ s_t)) / D. The values are likewise summed in
// the rotated domain (sum_t p_t v^_t) and rotated back once per output
// (inverse butterfly, signs), in the merge kernel.
//
// Storage per (layer, K|V): codes [H][B][R][CBP] bytes, params [H][B][R]
// float4 (scale, zero, C, 0), sign words [H][B][R][D/32]; rows [0, R) of a
// (head, sequence).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode_common.h"
#include "sai_internal.h"

namespace sai {
namespace {

// round_f32 of kv_compression.rs:27-37 (half away from zero through a
// truncation); x >= 0 here.
__device__ __forceinline__ float round_half_away(float x) {
#pragma clang fp contract(off)
  const float t = (float)sat_i32(x);
  const float f = x - t;
  if (f >= 0.5f) return t + 1.0f;
  if (f <= -0.5f) return t - 1.0f;
  return t;
}

// The reference's butterfly (wht_butterfly_normalize, :81-110) on a register
// array: stage h pairs (j, j + h) inside blocks of 2h; then * norm.
template <int D>
__device__ __forceinline__ void butterfly(float (&y)[D], float norm) {
#pragma clang fp contract(off)
#pragma unroll
  for (int h = 1; h < D; h *= 2)
#pragma unroll
    for (int i = 0; i < D; i += 2 * h)
#pragma unroll
      for (int j = i; j < i + h; ++j) {
        const float a = y[j], b = y[j + h];
        y[j] = a + b;
        y[j + h] = a - b;
      }
#pragma unroll
  for (int i = 0; i < D; ++i) y[i] *= norm;
}

template <int D, int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[D * BITS / 32], int i) {
  const int bit = BITS * i, word = bit >> 5, off = bit & 31;
  uint32_t v = w[word] >> off;
  if (off + BITS > 32) v |= w[word + 1] << (32 - off);
  return v & ((1u << BITS) - 1u);
}

__device__ __forceinline__ float load_row_elem(const void* p, size_t i, bool bf16) {
  return bf16 ? __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16) : ((const float*)p)[i];
}

// ---- write: one thread per (b, s, head, K|V) row ---------------------------
template <int D, int BITS>
__global__ __launch_bounds__(64) void tq_write_kernel(const TqArgs a, const void* k, const void* v,
                                                      int bf16, int batch, int s_new) {
#pragma clang fp contract(off)
  constexpr int W = D * BITS / 32;
  constexpr uint32_t LEVELS = (1u << BITS) - 1u;
  const int idx = blockIdx.x * 64 + threadIdx.x;
  const int total = batch * s_new * a.heads * 2;
  if (idx >= total) return;
  const int kind = idx & 1;  // 0: K, 1: V
  int r = idx >> 1;
  const int h = r % a.heads;
  r /= a.heads;
  const int s = r % s_new;
  const int b = r / s_new;
  const void* src = kind ? v : k;
  const size_t in_off = (((size_t)b * s_new + s) * a.heads + h) * D;
  const int8_t* sg = a.signs + (size_t)h * D;
  float y[D];
#pragma unroll
  for (int i = 0; i < D; ++i) y[i] = load_row_elem(src, in_off + i, bf16 != 0) * (float)sg[i];
  butterfly<D>(y, a.norm);
  float mn = y[0], mx = y[0];
#pragma unroll
  for (int i = 1; i < D; ++i) {
    mn = y[i] < mn ? y[i] : mn;
    mx = y[i] > mx ? y[i] : mx;
  }
  const float range = mx - mn;
  const float scale = range > 0.0f ? range / (float)LEVELS : 1.0f;
  const float zero = mn;
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = 0u;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    uint32_t q = scale > 0.0f ? sat_u32(round_half_away((y[i] - zero) / scale)) : 0u;
    q = q < LEVELS ? q : LEVELS;
    const int bit = BITS * i, word = bit >> 5, off = bit & 31;
    w[word] |= q << off;
    if (off + BITS > 32) w[word + 1] |= q >> (32 - off);
    y[i] = (float)q;  // keep the code for the QJL decode
  }
  const int pos = a.seq_lens[b] + s;
  const size_t row = ((size_t)h * a.batch_cap + b) * a.rows_cap + pos;
  uint8_t* codes = (kind ? a.codes_v : a.codes_k) + row * a.code_stride;
#pragma unroll
  for (int j = 0; j < W; ++j) ((uint32_t*)codes)[j] = w[j];
  float c = 0.0f;
  if (a.qjl) {
    // decode (:270-291) then the residual's signs and mean |r| (:365-395),
    // summed in index order
#pragma unroll
    for (int i = 0; i < D; ++i) y[i] = y[i] * scale + zero;
    butterfly<D>(y, a.norm);
    uint32_t sb[D / 32];
#pragma unroll
    for (int j = 0; j < D / 32; ++j) sb[j] = 0u;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const float approx = y[i] * (float)sg[i];
      const float rr = load_row_elem(src, in_off + i, bf16 != 0) - approx;
      sum += fabsf(rr);
      if (rr >= 0.0f) sb[i >> 5] |= 1u << (i & 31);
    }
    c = sum / (float)D;
    uint32_t* sw = (kind ? a.signs_v : a.signs_k) + row * (D / 32);
#pragma unroll
    for (int j = 0; j < D / 32; ++j) sw[j] = sb[j];
  }
  float4* par = (kind ? a.par_v : a.par_k) + row;
  *par = make_float4(scale, zero, c, 0.0f);
}

// ---- read: one thread per (row, K|V), decode to f32 -------------------------
template <int D, int BITS>
__global__ __launch_bounds__(64) void tq_read_kernel(const TqArgs a, int b, int h, int start,
                                                     int len, float* k_out, float* v_out) {
#pragma clang fp contract(off)
  constexpr int W = D * BITS / 32;
  const int idx = blockIdx.x * 64 + threadIdx.x;
  if (idx >= 2 * len) return;
  const int kind = idx & 1;
  const int t = idx >> 1;
  const size_t row = ((size_t)h * a.batch_cap + b) * a.rows_cap + start + t;
  const uint32_t* cw = (const uint32_t*)((kind ? a.codes_v : a.codes_k) + row * a.code_stride);
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = cw[j];
  const float4 par = (kind ? a.par_v : a.par_k)[row];
  float y[D];
#pragma unroll
  for (int i = 0; i < D; ++i) y[i] = (float)code_at<D, BITS>(w, i) * par.x + par.y;
  butterfly<D>(y, a.norm);
  const int8_t* sg = a.signs + (size_t)h * D;
  float* out = (kind ? v_out : k_out) + (size_t)t * D;
#pragma unroll
  for (int i = 0; i < D; ++i) out[i] = y[i] * (float)sg[i];
}

// ---- query encoding: one thread per (sequence, query head) ------------------
// The query row through the head's PolarQuantizer (as a cache row): its
// rotated reconstruction q^ = code * scale + zero, sum(q^), and with QJL the
// residual's C and sign words, as [D + 2 + D/32] floats per query head.
template <int D, int BITS>
__global__ __launch_bounds__(64) void tq_query_kernel(const TqArgs a, TqAttendArgs t, int batch) {
#pragma clang fp contract(off)
  constexpr uint32_t LEVELS = (1u << BITS) - 1u;
  constexpr int QREC = D + 2 + D / 32;
  const int idx = blockIdx.x * 64 + threadIdx.x;
  if (idx >= batch * t.num_heads) return;
  const int qh = idx % t.num_heads;
  const int kvh = qh / (t.num_heads / a.heads);
  const size_t qo = (size_t)idx * D;
  const int8_t* sg = a.signs + (size_t)kvh * D;
  float* rec = t.qenc + (size_t)idx * QREC;
  float y[D];
#pragma unroll
  for (int i = 0; i < D; ++i) y[i] = load_row_elem(t.q, qo + i, t.q_bf16 != 0) * (float)sg[i];
  butterfly<D>(y, a.norm);
  float mn = y[0], mx = y[0];
#pragma unroll
  for (int i = 1; i < D; ++i) {
    mn = y[i] < mn ? y[i] : mn;
    mx = y[i] > mx ? y[i] : mx;
  }
  const float range = mx - mn;
  const float scale = range > 0.0f ? range / (float)LEVELS : 1.0f;
  float qs = 0.0f;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    uint32_t q = scale > 0.0f ? sat_u32(round_half_away((y[i] - mn) / scale)) : 0u;
    q = q < LEVELS ? q : LEVELS;
    y[i] = (float)q * scale + mn;
    rec[i] = y[i];
    qs += y[i];
  }
  rec[D] = qs;
  float c = 0.0f;
  uint32_t sb[D / 32];
#pragma unroll
  for (int j = 0; j < D / 32; ++j) sb[j] = 0u;
  if (a.qjl) {
    butterfly<D>(y, a.norm);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const float rr = load_row_elem(t.q, qo + i, t.q_bf16 != 0) - y[i] * (float)sg[i];
      sum += fabsf(rr);
      if (rr >= 0.0f) sb[i >> 5] |= 1u << (i & 31);
    }
    c = sum / (float)D;
  }
  rec[D + 1] = c;
#pragma unroll
  for (int j = 0; j < D / 32; ++j) rec[D + 2 + j] = __uint_as_float(sb[j]);
}

// ---- attention ---------------------------------------------------------------
// Workgroup = (sequence b, kv head, split of split_rows rows), NW waves; a
// wave takes 64-row tiles (lane = row for the logits, lane = dims for the
// value sum); the group's encoded queries sit in LDS.
template <int D, int BITS, int G, int NW>
__global__ __launch_bounds__(64 * NW) void tq_attend_kernel(const TqArgs a, TqAttendArgs t) {
  constexpr int W = D * BITS / 32;
  constexpr uint32_t LEVELS = (1u << BITS) - 1u;
  constexpr int DPL = D / 64;  // value dims per lane
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int split = blockIdx.x;
  const int L = a.seq_lens[b] + a.pending;
  const int r0 = split * t.split_rows;
  if (r0 >= L) return;  // uniform: this split is past the sequence
  const int r1 = min(L, r0 + t.split_rows);

  __shared__ float sq[G][D];       // q^
  __shared__ float sqsum[G];       // sum_i q^_i
  __shared__ float sqc[G];         // C_q
  __shared__ uint32_t sqs[G][D / 32];
  __shared__ uint32_t svk[NW][64][W + 1];  // a wave's tile of K codes (row-major, padded)
  __shared__ uint32_t svc[NW][64][W + 1];  // a wave's tile of V codes
  __shared__ float spv[NW][64][G];         // p * s_v of the tile's rows
  {
    // the group's encoded queries (tq_query_kernel): [G][QREC]
    constexpr int QREC = D + 2 + D / 32;
    const float* qe = t.qenc + ((size_t)b * t.num_heads + kvh * G) * QREC;
    for (int e = threadIdx.x; e < G * QREC; e += 64 * NW) {
      const int g = e / QREC, j = e % QREC;
      const float v = qe[e];
      if (j < D) sq[g][j] = v;
      else if (j == D) sqsum[g] = v;
      else if (j == D + 1) sqc[g] = v;
      else sqs[g][j - D - 2] = __float_as_uint(v);
    }
  }
  __syncthreads();

  float m_run[G], l_run[G], acc[G][DPL], zacc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
    zacc[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[g][e] = 0.0f;
  }
  const size_t base = ((size_t)kvh * a.batch_cap + b) * a.rows_cap;
  const float inv_d = 1.0f / (float)D;
  for (int tile0 = r0 + wave * 64; tile0 < r1; tile0 += 64 * NW) {
    // q^ is re-read from LDS in every tile: kept out of registers, where the
    // G * D values would not fit
    __asm__ volatile("" ::: "memory");
    const int row = tile0 + lane;
    const bool live = row < r1;
    const size_t rr = base + (live ? row : tile0);
    // K and V codes of this lane's row into the wave's LDS tiles
    const uint32_t* kc = (const uint32_t*)(a.codes_k + rr * a.code_stride);
    const uint32_t* vc = (const uint32_t*)(a.codes_v + rr * a.code_stride);
#pragma unroll
    for (int j = 0; j < W; ++j) {
      svk[wave][lane][j] = kc[j];
      svc[wave][lane][j] = vc[j];
    }
    const float4 kp = a.par_k[rr];
    const float4 vp = a.par_v[rr];
    uint32_t ks[D / 32];
    if (a.qjl) {
#pragma unroll
      for (int j = 0; j < D / 32; ++j) ks[j] = a.signs_k[rr * (D / 32) + j];
    }
    __builtin_amdgcn_wave_barrier();
    // logits: 32 codes (BITS words) at a time, rolled, so that only one
    // group's q^ values are live
    float lg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) lg[g] = 0.0f;
#pragma unroll 1
    for (int grp = 0; grp < D / 32; ++grp) {
      uint32_t u[BITS + 1];
#pragma unroll
      for (int k = 0; k < BITS; ++k) u[k] = svk[wave][lane][grp * BITS + k];
      u[BITS] = 0u;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const int bit = BITS * c, word = bit >> 5, off = bit & 31;
        uint32_t v = u[word] >> off;
        if (off + BITS > 32) v |= u[word + 1] << (32 - off);
        const float cf = (float)(v & LEVELS);
#pragma unroll
        for (int g = 0; g < G; ++g) lg[g] += sq[g][grp * 32 + c] * cf;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float dot = kp.x * lg[g] + kp.y * sqsum[g];
      if (a.qjl) {
        int pop = 0;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) pop += __popc(sqs[g][j] ^ ks[j]);
        dot += sqc[g] * kp.z * ((float)(D - 2 * pop) * inv_d);
      }
      lg[g] = live ? dot * t.scale_log2 : -INFINITY;
    }
    // online softmax over the wave's 64 rows
    float alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mt = wave_max(lg[g]);
      const float m_new = fmaxf(m_run[g], mt);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      alpha[g] = fast_exp2(m_run[g] - m_use);
      const float p = fast_exp2(lg[g] - m_use);
      l_run[g] = l_run[g] * alpha[g] + wave_sum(p);
      m_run[g] = m_new;
      spv[wave][lane][g] = p * vp.x;
      zacc[g] = zacc[g] * alpha[g] + wave_sum(p * vp.y);
    }
    __builtin_amdgcn_wave_barrier();  // this wave's LDS tile, written above, read below
    // values: lane owns dims DPL*lane .. +DPL-1
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[g][e] *= alpha[g];
    const int nrows = min(64, r1 - tile0);
    for (int j = 0; j < nrows; ++j) {
      float pv[G];
#pragma unroll
      for (int g = 0; g < G; ++g) pv[g] = spv[wave][j][g];
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const int bit = BITS * (DPL * lane + e), word = bit >> 5, off = bit & 31;
        uint32_t u = svc[wave][j][word] >> off;
        if (BITS == 3 && off > 29) u |= svc[wave][j][word + 1] << (32 - off);
        const float c = (float)(u & LEVELS);
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g][e] += pv[g] * c;
      }
    }
    __builtin_amdgcn_wave_barrier();  // this wave's LDS tile, written above, read below
  }
  // merge the waves through LDS, then one partial per workgroup
  __shared__ float sm_m[NW][G], sm_l[NW][G], sm_z[NW][G];
  __shared__ float sm_o[NW][G][D];
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sm_m[wave][g] = m_run[g];
      sm_l[wave][g] = l_run[g];
      sm_z[wave][g] = zacc[g];
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) sm_o[wave][g][DPL * lane + e] = acc[g][e];
  __syncthreads();
  float* part = t.partials + (((size_t)b * a.heads + kvh) * t.max_splits + split) * (G * (D + 2));
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
    part[g * (D + 2) + 2 + i] = O;
    if (i == 0) {
      part[g * (D + 2)] = M;
      part[g * (D + 2) + 1] = Ls;
    }
  }
}

// Merge the splits of one (sequence, kv head), rotate back (inverse
// butterfly through LDS, then the signs) and normalise. One thread per
// (head, dim).
template <int D, int G>
__global__ __launch_bounds__(G * D) void tq_merge_kernel(const TqArgs a, TqAttendArgs t) {
#pragma clang fp contract(off)
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int g = threadIdx.x / D, i = threadIdx.x % D;
  const int L = a.seq_lens[b] + a.pending;
  const int nsplit = (L + t.split_rows - 1) / t.split_rows;
  const float* part = t.partials + ((size_t)b * a.heads + kvh) * t.max_splits * (G * (D + 2));
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part[(size_t)s * (G * (D + 2)) + g * (D + 2)]);
  float Ls = 0.0f, O = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float* ps = part + (size_t)s * (G * (D + 2)) + g * (D + 2);
    if (ps[0] == -INFINITY) continue;
    const float f = fast_exp2(ps[0] - M);
    Ls += ps[1] * f;
    O += ps[2 + i] * f;
  }
  __shared__ float sy[G][D];
  sy[g][i] = Ls > 0.0f ? O / Ls : 0.0f;
  __syncthreads();
  // inverse rotation: the same butterfly stages, one element per thread
  for (int h = 1; h < D; h *= 2) {
    const float a0 = sy[g][i], a1 = sy[g][i ^ h];
    __syncthreads();
    sy[g][i] = (i & h) ? a1 - a0 : a0 + a1;
    __syncthreads();
  }
  const float y = sy[g][i] * a.norm * (float)a.signs[(size_t)kvh * D + i];
  t.out[((size_t)b * t.num_heads + kvh * G + g) * D + i] = y;
}

template <int D, int BITS>
hipError_t attend_db(const TqArgs& a, const TqAttendArgs& t, int group, int nsplit, int batch,
                     hipStream_t st) {
  const int nq = batch * t.num_heads;
  hipLaunchKernelGGL((tq_query_kernel<D, BITS>), dim3((nq + 63) / 64), dim3(64), 0, st, a, t,
                     batch);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const dim3 grid(nsplit, a.heads, batch);
  switch (group) {
    case 1: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 1, 4>), grid, dim3(256), 0, st, a, t); break;
    case 2: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 2, 4>), grid, dim3(256), 0, st, a, t); break;
    case 4: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 4, 4>), grid, dim3(256), 0, st, a, t); break;
    case 8: hipLaunchKernelGGL((tq_attend_kernel<D, BITS, 8, 4>), grid, dim3(256), 0, st, a, t); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 mg(a.heads, batch);
  switch (group) {
    case 1: hipLaunchKernelGGL((tq_merge_kernel<D, 1>), mg, dim3(D), 0, st, a, t); break;
    case 2: hipLaunchKernelGGL((tq_merge_kernel<D, 2>), mg, dim3(2 * D), 0, st, a, t); break;
    case 4: hipLaunchKernelGGL((tq_merge_kernel<D, 4>), mg, dim3(4 * D), 0, st, a, t); break;
    case 8: hipLaunchKernelGGL((tq_merge_kernel<D, 8>), mg, dim3(8 * D), 0, st, a, t); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename F>
hipError_t dispatch_dbits(int d, int bits, F&& f) {
  auto by_bits = [&](auto dd) -> hipError_t {
    constexpr int DD = decltype(dd)::value;
    switch (bits) {
      case 3: return f(dd, std::integral_constant<int, 3>{});
      case 4: return f(dd, std::integral_constant<int, 4>{});
      case 8: return f(dd, std::integral_constant<int, 8>{});
      default: (void)DD; return hipErrorInvalidValue;
    }
  };
  if (d == 64) return by_bits(std::integral_constant<int, 64>{});
  if (d == 128) return by_bits(std::integral_constant<int, 128>{});
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_tq_write(const TqArgs& a, const void* k, const void* v, int bf16, int batch,
                           int s_new, hipStream_t st) {
  const int total = batch * s_new * a.heads * 2;
  if (total <= 0) return hipSuccess;
  return dispatch_dbits(a.head_dim, a.bits, [&](auto dd, auto bb) -> hipError_t {
    constexpr int D = decltype(dd)::value, B = decltype(bb)::value;
    hipLaunchKernelGGL((tq_write_kernel<D, B>), dim3((total + 63) / 64), dim3(64), 0, st, a, k,
                       v, bf16, batch, s_new);
    return hipGetLastError();
  });
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

hipError_t launch_tq_attend(const TqArgs& a, const TqAttendArgs& t, int group, int nsplit,
                            int batch, hipStream_t st) {
  return dispatch_dbits(a.head_dim, a.bits, [&](auto dd, auto bb) -> hipError_t {
    constexpr int D = decltype(dd)::value, B = decltype(bb)::value;
    return attend_db<D, B>(a, t, group, nsplit, batch, st);
  });
}

}  // namespace sai
